"""`interpret=True`: a NumPy interpreter of kernel jaxprs, vectorised over
program instances.

This is the backend's counterpart of JAX's Pallas interpreter, which the
reference exposes as `.interpret` (`src/palladium/__init__.py:110`,
`src/palladium/ffi.py:127`): an explicitly requested CPU evaluation of the
same kernel, used to cross-check the emitter on arbitrary kernels. It is
never a fallback of `hip_call` (which fails loudly without a GPU).

Every value carries a leading instance axis: a jaxpr value of shape `s`
is held as an array of shape `(P, *s)` for `P` program instances. Loops run
in lockstep; `while` masks finished instances (their stores are
suppressed), `cond` evaluates each branch under its instance mask.
Arithmetic is NumPy's, in the kernel's dtypes (fp32 ops are IEEE; libm-style
functions may differ from the device by an ulp); `min`/`max` on floats are
NaN-suppressing `fmin`/`fmax` with -0 ordered below +0, matching what the
emitted code computes on gfx950. bfloat16 values
are carried as float32 arrays: each operation is evaluated in float32 and
rounded to bfloat16 (ties to even), and bfloat16 sums and contractions
accumulate in float32 and round once. Float sums add one element at a time
in the emitted order (row-major over the reduced indices).
"""

from __future__ import annotations

import dataclasses
import math
from typing import Any

import numpy as np

from palladium_amd import exact
from palladium_amd.dtypes import bits_from_f32, f32_from_bits, from_float, is_bf16, round_f32, to_float
from palladium_amd.emit.core import check_contiguous
from palladium_amd.errors import EmitError, UnsupportedPrimitiveError
from palladium_amd.ir import Jaxpr, JaxprEqn, KeyAval, Literal, Slice, Var
from palladium_amd.trace import BlockInfo, KernelSpec, trace

__all__ = ["block_offsets", "check_block_bounds", "eval_index_map", "interpret_call", "interpret_spec"]

_U32 = np.uint32


def _threefry(k0, k1, c0, c1):
    """Threefry-2x32-20 over uint32 arrays (wrapping arithmetic)."""
    k0 = np.asarray(k0, _U32)
    k1 = np.asarray(k1, _U32)
    ks = (k0, k1, k0 ^ k1 ^ _U32(0x1BD11BDA))
    rots = ((13, 15, 26, 6), (17, 29, 16, 24))
    x0 = np.asarray(c0, _U32) + ks[0]
    x1 = np.asarray(c1, _U32) + ks[1]
    for g in range(5):
        for r in rots[g & 1]:
            x0 = x0 + x1
            x1 = (x1 << _U32(r)) | (x1 >> _U32(32 - r))
            x1 = x1 ^ x0
        x0 = x0 + ks[(g + 1) % 3]
        x1 = x1 + ks[(g + 2) % 3] + _U32(g + 1)
    return x0, x1


class _Ref:
    """A kernel operand as seen by P instances: the full flat array, each
    instance's element offset, and the element strides of the ref dims."""

    def __init__(self, flat: np.ndarray, base: np.ndarray, shape: tuple[int, ...], strides: tuple[int, ...], readonly: bool):
        self.flat = flat
        self.base = base
        self.shape = shape
        self.strides = strides
        self.readonly = readonly

    def index(self, indexer: Any, env: "_Env", n: int) -> tuple[np.ndarray, tuple[int, ...]]:
        """Flat element indices, shape (P, *kept) for this access."""
        off = self.base.astype(np.int64).reshape(n, *([1] * 0))
        kept_sizes: list[int] = []
        kept_strides: list[int] = []
        if indexer is None:
            kept_sizes = list(self.shape)
            kept_strides = list(self.strides)
        else:
            for d, idx in enumerate(indexer.indices):
                st = self.strides[d]
                if isinstance(idx, Slice):
                    if idx.stride != 1:
                        raise EmitError(f"ref access dim {d}: stride {idx.stride} != 1 is unimplemented")
                    start = idx.start
                    sv = np.int64(start) if isinstance(start, (int, np.integer)) else _per_instance(env.read(start), n)
                    off = off + sv * st
                    kept_sizes.append(int(idx.size))
                    kept_strides.append(st)
                else:
                    iv = _per_instance(env.read(idx), n)
                    off = off + iv * st
        grid = np.zeros((1,) + tuple(kept_sizes), np.int64)
        for k, (sz, st) in enumerate(zip(kept_sizes, kept_strides)):
            shape = [1] * (len(kept_sizes) + 1)
            shape[k + 1] = sz
            grid = grid + (np.arange(sz, dtype=np.int64) * st).reshape(shape)
        idx = off.reshape((n,) + (1,) * len(kept_sizes)) + grid
        return idx, tuple(kept_sizes)


def _per_instance(v: Any, n: int) -> np.ndarray:
    v = np.asarray(v).astype(np.int64).reshape(-1)
    return np.broadcast_to(v, (n,)) if v.size == 1 else v.reshape(n)


class _Env:
    def __init__(self, n: int, pids: list[np.ndarray], grid: tuple[int, ...], reproducible: bool = False):
        self.n = n
        self.pids = pids
        self.grid = grid
        self.reproducible = reproducible
        self.vals: dict[Var, Any] = {}

    def read(self, atom: Any) -> Any:
        if isinstance(atom, Literal):
            if is_bf16(atom.aval.dtype):
                return round_f32(np.float32(atom.val))
            return np.asarray(atom.val, dtype=atom.aval.dtype)
        return self.vals[atom]

    def write(self, var: Var, val: Any) -> None:
        self.vals[var] = val


def _align(x: Any, rank: int, n: int) -> Any:
    """Give an instance-batched operand `rank` value dims, right-aligned."""
    x = np.asarray(x)
    if x.ndim == 0:
        return x
    extra = rank - (x.ndim - 1)
    if extra > 0:
        x = x.reshape((x.shape[0],) + (1,) * extra + x.shape[1:])
    return x


def _fmin(a: Any, b: Any) -> np.ndarray:
    """NaN-suppressing minimum with -0 ordered below +0 (IEEE 754-2019
    minimumNumber): what gfx950's v_min_f32 returns for `fminf`. NumPy's
    fmin returns its second operand when the two compare equal, so it
    differs on zeros of opposite sign."""
    r = np.fmin(a, b)
    zeros = (np.asarray(a) == 0) & (np.asarray(b) == 0)
    if np.any(zeros):
        neg = np.signbit(a) | np.signbit(b)
        r = np.where(zeros, np.where(neg, -np.zeros_like(r), np.zeros_like(r)), r)
    return r


def _fmax(a: Any, b: Any) -> np.ndarray:
    """NaN-suppressing maximum with +0 ordered above -0 (maximumNumber),
    as gfx950's v_max_f32 returns for `fmaxf`."""
    r = np.fmax(a, b)
    zeros = (np.asarray(a) == 0) & (np.asarray(b) == 0)
    if np.any(zeros):
        neg = np.signbit(a) & np.signbit(b)
        r = np.where(zeros, np.where(neg, -np.zeros_like(r), np.zeros_like(r)), r)
    return r


def _fold(op: Any, src: np.ndarray, axes: tuple[int, ...]) -> np.ndarray:
    """Reduce `src` over `axes` with a binary `op` (order-free here: the
    signed-zero ordering makes min/max a total order on non-NaN values).
    An empty reduction gives the identity, -inf for max and +inf for min."""
    src = np.asarray(src)
    kept = [d for d in range(src.ndim) if d not in axes]
    moved = np.transpose(src, kept + list(axes))
    flat = moved.reshape(moved.shape[: len(kept)] + (-1,))
    if flat.shape[-1] == 0:
        return np.full(flat.shape[:-1], -np.inf if op is _fmax else np.inf, src.dtype)
    acc = flat[..., 0]
    for r in range(1, flat.shape[-1]):
        acc = op(acc, flat[..., r])
    return acc


def _int_div(a: Any, b: Any, dt: np.dtype) -> np.ndarray:
    """Integer division truncating toward zero, defined everywhere as XLA
    defines it: x / 0 = -1 (all ones unsigned), INT_MIN / -1 = INT_MIN."""
    a64 = np.asarray(a).astype(np.int64)
    b64 = np.asarray(b).astype(np.int64)
    safe = np.where(b64 == 0, 1, b64)
    q = np.abs(a64) // np.abs(safe) * np.sign(a64) * np.sign(safe)
    q = np.where(b64 == 0, -1, q)
    return (q & 0xFFFFFFFF).astype(np.uint32).view(np.int32).astype(dt) if dt.kind == "i" else \
        (q & 0xFFFFFFFF).astype(np.uint32).astype(dt)


def _int_rem(a: Any, b: Any, dt: np.dtype) -> np.ndarray:
    """Remainder with the sign of the dividend; x % 0 = x and
    INT_MIN % -1 = 0."""
    a64 = np.asarray(a).astype(np.int64)
    b64 = np.asarray(b).astype(np.int64)
    safe = np.where(b64 == 0, 1, b64)
    r = np.abs(a64) % np.abs(safe) * np.sign(a64)
    r = np.where(b64 == 0, a64, r)
    return r.astype(dt)


def _float_to_int(a: Any, dt: np.dtype) -> np.ndarray:
    """Truncating float -> int32/uint32 conversion that saturates and maps
    NaN to 0 (C leaves out-of-range values undefined)."""
    x = np.asarray(a).astype(np.float64)
    info = np.iinfo(dt)
    x = np.where(np.isnan(x), 0.0, np.clip(np.trunc(x), info.min, info.max))
    return x.astype(dt)


def _round_half_away(x):
    """C roundf: nearest integer, halves away from zero, zeros keep their
    sign. Exact: x - trunc(x) is representable, so nothing rounds on the way
    (the shortcut floor(|x| + 0.5) does: 0.49999997 + 0.5 rounds up to 1,
    as does 2^23 + 1 + 0.5 to 2^23 + 2)."""
    x = np.asarray(x)
    t = np.trunc(x)
    step = (np.abs(x - t) >= np.asarray(0.5, x.dtype)).astype(x.dtype)
    return t + np.copysign(step, x)


def _sign(x):
    """sign with zeros (and NaN) returned unchanged, as the emitted
    `(a > 0) ? 1 : ((a < 0) ? -1 : a)` does (NumPy turns -0 into +0)."""
    x = np.asarray(x)
    return np.where((x == 0) | np.isnan(x), x, np.sign(x))


# REPRODUCIBLE's exp, log, sin, cos and tanh (float32 on the device, also where
# the operands are bfloat16 or float16)
_DETERMINISTIC = {"exp": exact.dexpf, "log": exact.dlogf, "sin": exact.dsinf, "cos": exact.dcosf,
                  "tanh": exact.dtanhf}


def _elementwise(name: str, ops: list[Any], eqn: JaxprEqn, n: int, reproducible: bool = False) -> Any:
    out_aval = eqn.outvars[0].aval
    bf_out = is_bf16(out_aval.dtype)
    dt = np.dtype(np.float32) if bf_out else np.dtype(out_aval.dtype)
    rank = len(out_aval.shape)
    ops = [_align(o, rank, n) for o in ops]
    a = ops[0] if ops else None
    b = ops[1] if len(ops) > 1 else None
    isf = np.asarray(a).dtype.kind == "f" if a is not None else False
    # the REPRODUCIBLE forms are float32's (bfloat16 and float16 stay IEEE)
    f32_out = not bf_out and dt == np.float32
    with np.errstate(all="ignore"):
        if name == "add":
            r = a + b
        elif name == "sub":
            r = a - b
        elif name == "mul":
            r = a * b
        elif name == "fma":
            c = ops[2]
            r = exact.fma_f32(-a if eqn.params.get("neg_ab") else a, b, -c if eqn.params.get("neg_c") else c)
        elif name == "div" and reproducible and isf and f32_out:
            r = exact.rdiv(a, b)
        elif name == "pow" and reproducible and f32_out:
            r = exact.rpow(a, b)
        elif name == "log2" and reproducible and f32_out:
            r = exact.dlog2f(a)
        elif name == "exp2" and reproducible and f32_out:
            r = exact.dexp2f(a)
        elif name in _DETERMINISTIC and reproducible and isf:
            # computed in float32 on the device for every float type
            r = _DETERMINISTIC[name](np.asarray(a, np.float32))
        elif name == "logistic" and reproducible and isf:
            one = np.float32(1.0)
            r = one / (one + exact.dexpf(-np.asarray(a, np.float32)))
        elif name == "div":
            r = a / b if isf else _int_div(a, b, dt)
        elif name == "rem":
            r = np.fmod(a, b) if isf else _int_rem(a, b, dt)
        elif name == "min":
            r = _fmin(a, b) if isf else np.minimum(a, b)
        elif name == "max":
            r = _fmax(a, b) if isf else np.maximum(a, b)
        elif name == "pow":
            r = np.power(a, b)
        elif name == "neg":
            r = -a
        elif name == "abs":
            r = np.abs(a)
        elif name == "sign":
            r = _sign(a) if isf else np.sign(a)
        elif name in ("exp", "exp2", "log", "log2", "log1p", "expm1", "sin", "cos", "tan", "tanh", "sqrt", "floor", "ceil"):
            r = getattr(np, name)(a)
        elif name == "rsqrt":
            r = np.asarray(1.0, a.dtype) / np.sqrt(a)
        elif name == "round":
            r = np.rint(a) if int(eqn.params.get("rounding_method", 0)) == 1 else _round_half_away(a)
        elif name == "logistic":
            r = np.asarray(1.0, a.dtype) / (np.asarray(1.0, a.dtype) + np.exp(-a))
        elif name == "atan2":
            r = np.arctan2(a, b)
        elif name in ("lt", "le", "gt", "ge", "eq", "ne"):
            r = {"lt": np.less, "le": np.less_equal, "gt": np.greater, "ge": np.greater_equal,
                 "eq": np.equal, "ne": np.not_equal}[name](a, b)
        elif name == "and":
            r = np.bitwise_and(a, b)
        elif name == "or":
            r = np.bitwise_or(a, b)
        elif name == "xor":
            r = np.bitwise_xor(a, b)
        elif name == "not":
            r = np.logical_not(a) if np.asarray(a).dtype == np.bool_ else np.invert(a)
        elif name == "shift_right_logical":
            ua = np.asarray(a).astype(np.uint32)
            sb = np.asarray(b).astype(np.uint32)
            r = np.where(sb < 32, ua >> np.minimum(sb, 31), 0).astype(dt)
        elif name == "shift_right_arithmetic":
            # the amount is taken as unsigned: negative or >= 32 fills with the sign
            sb = np.asarray(b).astype(np.uint32).astype(np.int64)
            r = (np.asarray(a) >> np.minimum(sb, 31)).astype(dt)
        elif name == "shift_left":
            sb = np.asarray(b).astype(np.uint32)
            r = np.where(sb < 32, np.asarray(a) << np.minimum(sb, 31), 0).astype(dt)
        elif name == "clamp":
            lo, x, hi = ops
            r = (_fmin(_fmax(x, lo), hi) if np.asarray(x).dtype.kind == "f" else np.minimum(np.maximum(x, lo), hi))
        elif name == "select_n":
            pred, cases = ops[0], ops[1:]
            if np.asarray(pred).dtype == np.bool_:
                r = np.where(pred, cases[1], cases[0])
            else:
                idx = np.clip(pred, 0, len(cases) - 1)
                r = cases[-1]
                for k in reversed(range(len(cases) - 1)):
                    r = np.where(idx <= k, cases[k], r)
        elif name == "integer_pow":
            y = int(eqn.params["y"])
            if y == 0:
                r = np.ones_like(a)
            else:
                r = a
                for _ in range(abs(y) - 1):
                    r = r * a
                if y < 0:
                    r = np.asarray(1.0, r.dtype) / r
        elif name == "convert_element_type":
            if dt == np.bool_:
                r = np.asarray(a) != 0
            elif dt.kind in "iu" and np.asarray(a).dtype.kind == "f":
                r = _float_to_int(a, dt)
            else:
                r = np.asarray(a).astype(dt)
        elif name == "bitcast_convert_type":
            if bf_out:  # float16 bits -> bfloat16
                r = f32_from_bits(np.ascontiguousarray(np.asarray(a)).view(np.uint16))
            elif is_bf16(eqn.invars[0].aval.dtype):  # bfloat16 bits -> float16
                r = bits_from_f32(a).view(dt)
            else:
                r = np.ascontiguousarray(np.asarray(a)).view(dt)
        else:
            raise UnsupportedPrimitiveError(f"interpreter has no rule for primitive '{name}'")
    r = np.asarray(r)
    if r.dtype != dt:
        with np.errstate(over="ignore", invalid="ignore"):  # narrowing saturates to inf, as on the device
            r = r.astype(dt)
    if bf_out:
        r = round_f32(r)
    full = (n,) + tuple(out_aval.shape)
    if r.shape != full:
        r = np.broadcast_to(r, full).copy()
    return r


_ELEMENTWISE = set(
    "add sub mul div rem min max pow neg abs sign exp exp2 log log2 log1p expm1 sin cos tan tanh sqrt rsqrt floor "
    "ceil round logistic atan2 lt le gt ge eq ne and or xor not shift_right_logical shift_right_arithmetic "
    "shift_left clamp select_n integer_pow convert_element_type bitcast_convert_type fma".split()
)


def _eval(jaxpr: Jaxpr, env: _Env, invals: list[Any], mask: np.ndarray) -> list[Any]:
    n = env.n
    for v, val in zip(jaxpr.invars, invals):
        env.write(v, val)
    for eqn in jaxpr.eqns:
        name = eqn.primitive.name
        if name in _ELEMENTWISE:
            env.write(eqn.outvars[0], _elementwise(name, [env.read(a) for a in eqn.invars], eqn, n, env.reproducible))
        elif name == "get":
            ref: _Ref = env.read(eqn.invars[0])
            tree = eqn.params["tree"].unflatten(eqn.invars[1:])
            idx, _ = ref.index(tree[0] if tree else None, env, n)
            shape = (n,) + tuple(eqn.outvars[0].aval.shape)
            safe = np.where(mask.reshape((n,) + (1,) * (idx.ndim - 1)), idx, 0)
            if np.any(safe < 0) or np.any(safe >= ref.flat.size):
                raise IndexError("kernel read outside its operand")
            env.write(eqn.outvars[0], ref.flat[safe].reshape(shape))
        elif name == "swap":
            ref = env.read(eqn.invars[0])
            val = np.asarray(env.read(eqn.invars[1]))
            tree = eqn.params["tree"].unflatten(eqn.invars[2:])
            idx, kept = ref.index(tree[0] if tree else None, env, n)
            shape = (n,) + tuple(eqn.outvars[0].aval.shape)
            vals = np.broadcast_to(_align(val, len(shape) - 1, n), shape)
            m = np.broadcast_to(mask.reshape((n,) + (1,) * (idx.ndim - 1)), idx.shape)
            sel = idx[m]
            if sel.size and (sel.min() < 0 or sel.max() >= ref.flat.size):
                raise IndexError("kernel wrote outside its operand")
            old = ref.flat[np.where(m, idx, 0)].reshape(shape)
            ref.flat[sel] = vals.reshape(idx.shape)[m]
            env.write(eqn.outvars[0], old)
        elif name == "iota":
            shape = tuple(eqn.params["shape"])
            dim = int(eqn.params["dimension"])
            bf = is_bf16(eqn.outvars[0].aval.dtype)
            r = np.arange(shape[dim], dtype=np.float32 if bf else eqn.outvars[0].aval.dtype)
            r = (round_f32(r) if bf else r).reshape([-1 if k == dim else 1 for k in range(len(shape))])
            env.write(eqn.outvars[0], np.broadcast_to(r, (n,) + shape).copy())
        elif name == "program_id":
            env.write(eqn.outvars[0], env.pids[int(eqn.params["axis"])])
        elif name == "num_programs":
            env.write(eqn.outvars[0], np.full((n,), env.grid[int(eqn.params["axis"])], np.int32))
        elif name == "broadcast_in_dim":
            src = np.asarray(env.read(eqn.invars[0]))
            shape = tuple(eqn.params["shape"])
            bd = tuple(eqn.params["broadcast_dimensions"])
            if src.ndim == 0:
                src = np.broadcast_to(src, (n,))
            sshape = src.shape[1:]
            tgt = [1] * len(shape)
            for k, d in enumerate(bd):
                tgt[d] = sshape[k]
            env.write(eqn.outvars[0], np.broadcast_to(src.reshape((src.shape[0],) + tuple(tgt)), (n,) + shape).copy())
        elif name in ("reshape", "squeeze", "expand_dims"):
            src = np.asarray(env.read(eqn.invars[0]))
            if src.ndim == 0:
                src = np.broadcast_to(src, (n,))
            env.write(eqn.outvars[0], src.reshape((n,) + tuple(eqn.outvars[0].aval.shape)))
        elif name == "transpose":
            src = env.read(eqn.invars[0])
            perm = tuple(eqn.params["permutation"])
            env.write(eqn.outvars[0], np.transpose(src, (0,) + tuple(p + 1 for p in perm)).copy())
        elif name == "dot_general":
            env.write(eqn.outvars[0], _dot_general(eqn, env.read(eqn.invars[0]), env.read(eqn.invars[1]), n))
        elif name in ("reduce_sum", "reduce_max", "reduce_min", "reduce_or", "reduce_and"):
            src = np.asarray(env.read(eqn.invars[0]))
            axes = tuple(int(a) + 1 for a in eqn.params["axes"])
            f = {"reduce_sum": np.sum, "reduce_or": np.any, "reduce_and": np.all}.get(name)
            bf = is_bf16(eqn.outvars[0].aval.dtype)
            if name == "reduce_max":
                r = _fold(_fmax, src, axes) if src.dtype.kind == "f" else np.max(src, axis=axes)
            elif name == "reduce_min":
                r = _fold(_fmin, src, axes) if src.dtype.kind == "f" else np.min(src, axis=axes)
            elif name == "reduce_sum" and (bf or src.dtype.kind == "f"):
                r = _ordered_sum(src, axes, np.float32 if bf else src.dtype)
            else:
                r = f(src, axis=axes)
            r = round_f32(r) if bf else np.asarray(r).astype(eqn.outvars[0].aval.dtype)
            env.write(eqn.outvars[0], r)
        elif name in ("random_wrap", "random_unwrap"):
            env.write(eqn.outvars[0], np.asarray(env.read(eqn.invars[0])).reshape(n, 2))
        elif name == "random_fold_in":
            k = np.asarray(env.read(eqn.invars[0])).reshape(n, 2)
            d = np.broadcast_to(np.asarray(env.read(eqn.invars[1])).astype(_U32).reshape(-1), (n,))
            with np.errstate(over="ignore"):
                a, b = _threefry(k[:, 0], k[:, 1], np.zeros(n, _U32), d)
            env.write(eqn.outvars[0], np.stack([a, b], axis=1))
        elif name == "random_bits":
            k = np.asarray(env.read(eqn.invars[0])).reshape(n, 2)
            shape = tuple(eqn.outvars[0].aval.shape)
            size = math.prod(shape)
            ctr = np.broadcast_to(np.arange(size, dtype=_U32), (n, size))
            with np.errstate(over="ignore"):
                a, b = _threefry(k[:, :1], k[:, 1:], np.zeros_like(ctr), ctr)
            env.write(eqn.outvars[0], (a ^ b).reshape((n,) + shape))
        elif name == "threefry2x32":
            ops = [np.broadcast_to(_align(env.read(a), len(eqn.outvars[0].aval.shape), n),
                                   (n,) + tuple(eqn.outvars[0].aval.shape)).astype(_U32) for a in eqn.invars]
            with np.errstate(over="ignore"):
                a, b = _threefry(*ops)
            env.write(eqn.outvars[0], a)
            env.write(eqn.outvars[1], b)
        elif name in ("pjit", "jit", "closed_call", "core_call", "custom_jvp_call", "custom_vjp_call"):
            inner = eqn.params.get("jaxpr") or eqn.params.get("call_jaxpr")
            body = getattr(inner, "jaxpr", inner)
            outs = _eval(body, env, [env.read(a) for a in eqn.invars], mask)
            for ov, o in zip(eqn.outvars, outs):
                env.write(ov, o)
        elif name == "scan":
            _scan(eqn, env, mask)
        elif name == "while":
            _while(eqn, env, mask)
        elif name == "cond":
            _cond(eqn, env, mask)
        else:
            raise UnsupportedPrimitiveError(f"interpreter has no rule for primitive '{name}'")
    return [env.read(v) for v in jaxpr.outvars]


def _ordered_sum(src: np.ndarray, axes: tuple[int, ...], acc_dtype: Any) -> np.ndarray:
    """Sum over `axes` in row-major order of the reduced indices, one add
    at a time in `acc_dtype` (the emitter's accumulation order; NumPy's own
    sum is pairwise)."""
    src = np.asarray(src, acc_dtype)
    kept = [d for d in range(src.ndim) if d not in axes]
    moved = np.transpose(src, kept + list(axes))
    flat = moved.reshape(moved.shape[: len(kept)] + (-1,))
    acc = np.zeros(flat.shape[:-1], acc_dtype)
    for r in range(flat.shape[-1]):
        acc = acc + flat[..., r]
    return acc


def _dot_general(eqn: JaxprEqn, lhs: Any, rhs: Any, n: int) -> np.ndarray:
    """Contraction accumulated in k order from zero in the output dtype,
    `acc = acc + a*b`, the operation sequence the emitter produces
    (bfloat16: accumulated in float32, rounded once)."""
    (lc, rc), (lb, rb) = eqn.params["dimension_numbers"]
    if tuple(lb) or tuple(rb):
        raise EmitError("dot_general: batch dims are unimplemented")
    bf = is_bf16(eqn.outvars[0].aval.dtype)
    out_dt = np.dtype(np.float32) if bf else np.dtype(eqn.outvars[0].aval.dtype)
    la, ra = eqn.invars[0].aval, eqn.invars[1].aval
    lhs = np.broadcast_to(np.asarray(lhs), (n,) + tuple(la.shape)).astype(out_dt)
    rhs = np.broadcast_to(np.asarray(rhs), (n,) + tuple(ra.shape)).astype(out_dt)
    # Move the contracting dim last on both sides: (n, m?, k) and (n, n_?, k).
    lhs = np.moveaxis(lhs, int(lc[0]) + 1, -1)
    rhs = np.moveaxis(rhs, int(rc[0]) + 1, -1)
    m_shape, r_shape = lhs.shape[1:-1], rhs.shape[1:-1]
    a = lhs.reshape(n, -1, 1, lhs.shape[-1])
    b = rhs.reshape(n, 1, -1, rhs.shape[-1])
    acc = np.zeros((n, a.shape[1], b.shape[2]), out_dt)
    with np.errstate(all="ignore"):
        for kk in range(a.shape[-1]):
            acc = acc + a[..., kk] * b[..., kk]
    if bf:
        acc = round_f32(acc)
    return acc.reshape((n,) + tuple(m_shape) + tuple(r_shape))


def _full(val: Any, aval: Any, n: int) -> np.ndarray:
    shape = (n, 2) if isinstance(aval, KeyAval) else (n,) + tuple(aval.shape)
    v = np.asarray(val)
    if v.shape != shape:
        v = np.broadcast_to(v.reshape(v.shape + (1,) * 0) if v.ndim else v, shape)
    return np.array(v, dtype=v.dtype)


def _scan(eqn: JaxprEqn, env: _Env, mask: np.ndarray) -> None:
    body = getattr(eqn.params["jaxpr"], "jaxpr", eqn.params["jaxpr"])
    nc = len(eqn.outvars)
    nconst = len(eqn.invars) - nc
    if eqn.params.get("reverse", False):
        raise EmitError("no reverse-mode scan support, use lax.fori_loop")
    n_carry = int(eqn.params.get("num_carry", nc))
    if nc != n_carry:
        raise EmitError("lax.scan with stacked ys not supported, use lax.fori_loop")
    if int(eqn.params.get("num_consts", nconst)) != nconst:
        raise EmitError("lax.scan with scanned xs not supported, use lax.fori_loop")
    consts = [env.read(a) for a in eqn.invars[:nconst]]
    carries = [_full(env.read(a), ov.aval, env.n) for a, ov in zip(eqn.invars[nconst:], eqn.outvars)]
    for _ in range(int(eqn.params["length"])):
        outs = _eval(body, env, consts + carries, mask)
        carries = [_full(o, ov.aval, env.n) for o, ov in zip(outs, eqn.outvars)]
    for ov, c in zip(eqn.outvars, carries):
        env.write(ov, c)


def _while(eqn: JaxprEqn, env: _Env, mask: np.ndarray) -> None:
    cn, bn = int(eqn.params["cond_nconsts"]), int(eqn.params["body_nconsts"])
    cj = getattr(eqn.params["cond_jaxpr"], "jaxpr", eqn.params["cond_jaxpr"])
    bj = getattr(eqn.params["body_jaxpr"], "jaxpr", eqn.params["body_jaxpr"])
    cconsts = [env.read(a) for a in eqn.invars[:cn]]
    bconsts = [env.read(a) for a in eqn.invars[cn : cn + bn]]
    carries = [_full(env.read(a), ov.aval, env.n) for a, ov in zip(eqn.invars[cn + bn :], eqn.outvars)]
    n = env.n
    while True:
        (p,) = _eval(cj, env, cconsts + carries, mask)
        active = mask & np.broadcast_to(np.asarray(p).reshape(n, -1)[:, 0], (n,))
        if not active.any():
            break
        outs = _eval(bj, env, bconsts + carries, active)
        new = []
        for c, o, ov in zip(carries, outs, eqn.outvars):
            o = _full(o, ov.aval, n)
            m = active.reshape((n,) + (1,) * (c.ndim - 1))
            new.append(np.where(m, o, c))
        carries = new
    for ov, c in zip(eqn.outvars, carries):
        env.write(ov, c)


def _cond(eqn: JaxprEqn, env: _Env, mask: np.ndarray) -> None:
    branches = eqn.params["branches"]
    n = env.n
    idx = np.asarray(env.read(eqn.invars[0])).reshape(n)
    ops = [env.read(a) for a in eqn.invars[1:]]
    nb = len(branches)
    idx = np.clip(idx, 0, nb - 1)
    results = None
    for i, br in enumerate(branches):
        m = mask & (idx == i)
        if not m.any():
            continue
        outs = _eval(getattr(br, "jaxpr", br), env, ops, m)
        outs = [_full(o, ov.aval, n) for o, ov in zip(outs, eqn.outvars)]
        if results is None:
            results = [np.zeros_like(o) for o in outs]
        for r, o in zip(results, outs):
            mm = m.reshape((n,) + (1,) * (o.ndim - 1))
            np.copyto(r, o, where=np.broadcast_to(mm, o.shape))
    if results is None:
        results = [np.zeros((n,) + tuple(ov.aval.shape), ov.aval.dtype) for ov in eqn.outvars]
    for ov, r in zip(eqn.outvars, results):
        env.write(ov, r)


def _grid_pids(grid: tuple[int, ...]) -> list[np.ndarray]:
    n = math.prod(grid)
    flat = np.arange(n, dtype=np.int64)
    pids = []
    rem = flat
    for g in reversed(grid):
        pids.append((rem % g).astype(np.int32))
        rem = rem // g
    return list(reversed(pids))


def eval_index_map(info: BlockInfo, pids: list[np.ndarray], n: int) -> list[np.ndarray]:
    """Block indices (units of blocks) per array dim for every instance."""
    imj = info.index_map_jaxpr.jaxpr
    env = _Env(n, pids, ())
    outs = _eval(imj, env, pids[: len(imj.invars)], np.ones(n, bool))
    return [np.broadcast_to(np.asarray(o).astype(np.int64).reshape(-1), (n,)) for o in outs]


def block_offsets(spec: KernelSpec, info: BlockInfo, pids: list[np.ndarray] | None = None) -> np.ndarray:
    """Element offset of each instance's block in the flat array."""
    n = spec.num_programs
    pids = pids if pids is not None else _grid_pids(tuple(spec.grid))
    full = info.full_block()
    strides = [math.prod(info.array_shape[d + 1 :]) for d in range(len(info.array_shape))]
    off = np.zeros(n, np.int64)
    for bi, b, s in zip(eval_index_map(info, pids, n), full, strides):
        off = off + bi * b * s
    return off


def _ragged_lane_operands(spec: KernelSpec) -> tuple[int, ...]:
    """Operands whose ragged last block the lane-parallel lowering handles
    (lanes past the array load a clamped row and store nothing)."""
    from palladium_amd.emit.lanes import lane_transform

    plan = lane_transform(spec)
    return plan.lane_operands if plan is not None and plan.rows is not None else ()


def check_block_bounds(spec: KernelSpec) -> None:
    """Raise EmitError if any instance's block extends past its array
    (ragged blocks are not lowered: they would read and write out of
    bounds on the device)."""
    pids = _grid_pids(tuple(spec.grid))
    ragged_ok = _ragged_lane_operands(spec)
    for k, info in enumerate(list(spec.inputs) + list(spec.outputs)):
        imj = info.index_map_jaxpr.jaxpr
        full = info.full_block()
        outs = eval_index_map(info, pids, spec.num_programs)
        for d, (bi, b, a) in enumerate(zip(outs, full, info.array_shape)):
            lo, hi = int(bi.min()), int(bi.max())
            if d == 0 and k in ragged_ok:
                continue  # a ragged tail the lane-parallel lowering masks
            if lo < 0 or (hi + 1) * b > a:
                raise EmitError(
                    f"operand {k}: the index map places a block of {b} along dim {d} at block index "
                    f"{lo if lo < 0 else hi}, past the array extent {a}; ragged or out-of-range blocks are "
                    "not supported (size the grid so blocks tile the array)"
                )
        del imj


def interpret_spec(spec: KernelSpec, *arrays: np.ndarray, math_mode: Any = None) -> tuple[np.ndarray, ...]:
    """Run a KernelSpec on the CPU. Float operations are IEEE, in the traced
    order (SAFE's semantics). With `math_mode` REPRODUCIBLE the program
    first goes through the emitter's rewrites for that mode (FAST's algebra,
    then the product contraction) and float32 division, power, log2 and exp2
    take that mode's forms (`palladium_amd.exact`), so the results are the
    device's bit for bit for everything but the other transcendentals."""
    from palladium_amd.runtime import REPRODUCIBLE_ORDINAL, math_mode_ordinal

    reproducible = math_mode is not None and math_mode_ordinal(math_mode) == REPRODUCIBLE_ORDINAL
    if reproducible:
        from palladium_amd.emit.optimize import contract_products, fast_rewrites

        spec = dataclasses.replace(spec, jaxpr=contract_products(fast_rewrites(spec.jaxpr)))
    n = spec.num_programs
    pids = _grid_pids(tuple(spec.grid))
    refs = []
    outs = []
    operands = list(spec.inputs) + list(spec.outputs)
    ragged = _ragged_lane_operands(spec)
    for k, info in enumerate(operands):
        shape = tuple(info.array_shape)
        if k in ragged:
            # Rows are independent in a ragged lane kernel: pad the tail
            # block with copies of the last row, drop its outputs after.
            shape = (spec.grid[0] * info.block_shape[0],) + shape[1:]
            info = dataclasses.replace(info, array_shape=shape)
        bf = is_bf16(info.dtype)
        if k < len(spec.inputs):
            arr = np.ascontiguousarray(arrays[k], dtype=info.dtype)
            if bf:
                arr = to_float(arr)
            if arr.shape != shape:
                arr = np.pad(arr, [(0, shape[0] - arr.shape[0])] + [(0, 0)] * (arr.ndim - 1), mode="edge")
            flat = arr.reshape(-1).copy()
        else:
            flat = np.zeros(math.prod(shape), np.float32 if bf else info.dtype)
            outs.append(flat)
        check_contiguous(info, f"operand {k}")
        bshape = tuple(info.block_shape) or (1,)
        strides = tuple(math.prod(bshape[d + 1 :]) for d in range(len(bshape)))
        refs.append(_Ref(flat, block_offsets(spec, info, pids), bshape, strides, k < len(spec.inputs)))
    env = _Env(n, pids, tuple(spec.grid), reproducible)
    _eval(spec.jaxpr, env, refs, np.ones(n, bool))
    return tuple(
        _to_storage(o[: math.prod(info.array_shape)].reshape(info.array_shape), info.dtype)
        for o, info in zip(outs, spec.outputs)
    )


def _to_storage(a: np.ndarray, dtype: Any) -> np.ndarray:
    """bfloat16 values are carried as float32 inside the interpreter."""
    return from_float(a) if is_bf16(dtype) else a


def interpret_call(call: Any, *args: Any, math_mode: Any = None) -> Any:
    """Run a staged pallas_call on the CPU interpreter."""
    arrays = [np.asarray(a) for a in args]
    spec = trace(call, *arrays)
    outs = interpret_spec(spec, *arrays, math_mode=math_mode)
    return outs if call.multiple_results else outs[0]
