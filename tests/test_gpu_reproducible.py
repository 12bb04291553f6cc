"""The REPRODUCIBLE math mode on the GPU against the C oracle, bit for bit:
its correctly rounded reciprocal on every float, division and the fast
deterministic pow on special and scattered operands, and the adaptive
BS3(2)+PI Van der Pol loop of config 2 at full size (final states and both
step counts), whose op sequence oracle/oracle.c:oracle_bs3_vdp_r restates
with C fmaf at the fused sites; the deterministic exp, log, sin and cos on
scattered and special operands, and the GBM Monte Carlo of config 3 path
by path against oracle_gbm_r."""

import dataclasses

import numpy as np
import pytest

import oracle
import palladium_amd as pa
from palladium_amd import runtime as rt
from palladium_amd.emit.prelude import PRELUDE
from palladium_amd.frontend import pl
from palladium_amd.workloads import BS3_CFG, bs3_inputs, bs3_vdp_call

pytestmark = pytest.mark.gpu

RCP_SRC = PRELUDE + r"""
extern "C" __global__ void __launch_bounds__(256)
rrcp_all(unsigned int* __restrict__ count, unsigned int* __restrict__ first)
{
    // 65536 workgroups x 256 lanes x 256 values: every 32-bit pattern once
    const unsigned int lane = blockIdx.x * 256u + threadIdx.x;
    for (unsigned int k = 0; k < 256u; ++k) {
        const unsigned int bits = (k << 24) | lane;
        const float b = __uint_as_float(bits);
        const float got = ph_rrcp(b);
        const float want = 1.0f / b;
        const bool same = (__float_as_uint(got) == __float_as_uint(want)) || (got != got && want != want);
        if (!same) {
            const unsigned int slot = atomicAdd(count, 1u);
            if (slot < 16u) first[slot] = bits;
        }
    }
}
"""


def test_rrcp_is_the_ieee_reciprocal_on_every_float():
    print("[reproducible] ph_rrcp over all 2^32 patterns", flush=True)
    k = rt.Kernel(RCP_SRC, "rrcp_all", "reproducible")
    count = rt.Buffer.from_numpy(np.zeros(1, np.uint32))
    first = rt.Buffer.from_numpy(np.zeros(16, np.uint32))
    rt.run(k, (65536,), [count, first])
    n = int(count.to_numpy()[0])
    bad = first.to_numpy()[: min(n, 16)]
    assert n == 0, f"{n} mismatches, e.g. b = {[hex(int(b)) for b in bad]}"


def _elementwise(fn, n):
    s = pl.BlockSpec((1,), lambda i: (i,))
    return pa.hip_call(fn, grid=(n,), in_specs=[s, s], out_specs=s,
                       out_shape=pl.ShapeDtypeStruct((n,), np.float32), math_mode="reproducible")


def _operands(seed, n):
    r = np.random.default_rng(seed)
    special = np.array([0.0, -0.0, 1.0, -1.0, 2.0, 0.5, np.inf, -np.inf, np.nan, 1e-45, -1e-45,
                        1.1754942e-38, 1.17549435e-38, 3.4028235e38, 8191.0, 8192.0, -8192.0, 0.23333333,
                        -0.13333334, 3.0, -3.0, 1e9, 1e-9], np.float32)
    xs = np.concatenate([
        r.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32),
        (10.0 ** r.uniform(-40, 38, n)).astype(np.float32),
        np.repeat(special, special.size),
    ])
    ys = np.concatenate([
        r.uniform(-4, 4, n).astype(np.float32),
        r.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32),
        np.tile(special, special.size),
    ])
    return xs, ys


def test_division_and_pow_match_the_oracle():
    xs, ys = _operands(3, 1 << 18)
    n = xs.size
    print(f"[reproducible] div and pow over {n} operand pairs", flush=True)

    def div(x_ref, y_ref, o_ref):
        o_ref[...] = x_ref[...] / y_ref[...]

    def power(x_ref, y_ref, o_ref):
        o_ref[...] = x_ref[...] ** y_ref[...]

    got_div = _elementwise(div, n)(xs, ys)
    want_div = np.array([oracle.rdiv(a, b) for a, b in zip(xs[:4096], ys[:4096])], np.float32)
    _assert_same_bits(got_div[:4096], want_div, "division (oracle_rdiv)")
    # the whole sample through the vectorised restatement of a * RN(1/b)
    with np.errstate(all="ignore"):
        want_all = xs * (np.float32(1.0) / ys)
    _assert_same_bits(got_div, want_all, "division")
    got_pow = _elementwise(power, n)(xs, ys)
    _assert_same_bits(got_pow, oracle.rpow(xs, ys), "pow")


def _assert_same_bits(got, want, what):
    """Bit-identical, except that any NaN matches any NaN."""
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    bad = np.flatnonzero(~same)
    assert bad.size == 0, f"{bad.size} {what} mismatches, first at {bad[:4]}: {got[bad[:4]]} != {want[bad[:4]]}"


def test_bs3_config2_states_and_counts_exact():
    n = BS3_CFG.n
    x0, v0, mu = bs3_inputs(n, seed=BS3_CFG.seed)
    print(f"[reproducible] bs3_vdp n={n} vs oracle_bs3_vdp_r", flush=True)
    got = bs3_vdp_call(n, math_mode="reproducible")(x0, v0, mu)
    want = oracle.bs3_vdp(x0, v0, mu, BS3_CFG, mode="reproducible")
    for g, w, name in zip(got, want, ["t", "x", "v", "accepted", "rejected"]):
        np.testing.assert_array_equal(g, w, err_msg=name)
    assert np.all(got[0] == np.float32(BS3_CFG.t1))


def test_bs3_attempt_cap_exact():
    cfg = dataclasses.replace(BS3_CFG, max_attempts=37)
    n = 1000
    x0, v0, mu = bs3_inputs(n, seed=9)
    got = bs3_vdp_call(n, cfg, math_mode="reproducible")(x0, v0, mu)
    want = oracle.bs3_vdp(x0, v0, mu, cfg, mode="reproducible")
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    assert np.all(got[3] + got[4] <= 37)


def test_lv_config1_reproducible_bit_exact():
    """Config 1 in full (10^6 trajectories, 4,000 steps, max|y|) under
    REPRODUCIBLE: FAST's common-factor and affine-shift rewrites with fused
    multiply-adds at the contraction's sites, equal bit for bit to
    oracle_lv_rk4_r, and within FAST's 1e-3 of the SAFE-order oracle."""
    from palladium_amd.workloads import LV_CFG1, lv_inputs, lv_rk4_call

    n = 1_000_000
    args = lv_inputs(n, 1)
    print(f"[reproducible] lv_rk4 n={n} steps={LV_CFG1.steps}", flush=True)
    got = lv_rk4_call(n, LV_CFG1.dt, LV_CFG1.steps, track_max=True, math_mode="reproducible")(*args)
    want = oracle.lv_rk4_r(*args, LV_CFG1.dt, LV_CFG1.steps)
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    safe = oracle.lv_rk4(*args[:], LV_CFG1.dt, LV_CFG1.steps, track_max=True)
    np.testing.assert_allclose(got[0], safe[0], rtol=1e-3)


def _transcendental_operands(seed):
    r = np.random.default_rng(seed)
    n = 1 << 22
    special = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 1.1754942e-38,
                        3.4028235e38, -3.4028235e38, 2.0 ** 19, -2.0 ** 19, 2.0 ** 20, -2.0 ** 20,
                        1048575.9, 88.72283, 88.72284, -103.97208, -87.33655, 0.7853982, 1.5707964,
                        3.1415927, 6.2831855, 1e30, -1e30], np.float32)
    return np.concatenate([
        # every exponent and sign, low bits scattered
        ((np.arange(n, dtype=np.uint64) << np.uint64(10)) | r.integers(0, 1024, n, dtype=np.uint64))
        .astype(np.uint32).view(np.float32),
        r.uniform(-10, 10, n).astype(np.float32),
        r.uniform(-110, 90, n).astype(np.float32),
        r.uniform(0, 2 * np.pi, n).astype(np.float32),
        special,
    ])


def test_exp_log_sin_cos_tanh_sqrt_match_the_oracle():
    """The REPRODUCIBLE exp, log, sin, cos and tanh (ph_dexpf, ph_dlogf,
    ph_dtrig, ph_dtanhf) equal oracle_dexpf/dlogf/dsinf/dcosf/dtanhf bit for bit on 16.8M
    operands (scattered bit patterns over every exponent, the working
    ranges of exp and of Box-Muller's angle, the large-argument reduction
    and the special values), and sqrtf under this mode's compile options is
    the correctly rounded square root."""
    from palladium_amd.frontend import jnp

    xs = _transcendental_operands(5)
    n = xs.size
    print(f"[reproducible] exp/log/sin/cos/sqrt over {n} operands", flush=True)
    s = pl.BlockSpec((1,), lambda i: (i,))
    outs = tuple(pl.ShapeDtypeStruct((n,), np.float32) for _ in range(6))

    def k(x_ref, e_ref, l_ref, s_ref, c_ref, t_ref, q_ref):
        x = x_ref[...]
        e_ref[...] = jnp.exp(x)
        l_ref[...] = jnp.log(x)
        s_ref[...] = jnp.sin(x)
        c_ref[...] = jnp.cos(x)
        t_ref[...] = jnp.tanh(x)
        q_ref[...] = jnp.sqrt(x)

    got = pa.hip_call(k, grid=(n,), in_specs=[s], out_specs=[s] * 6, out_shape=outs,
                      math_mode="reproducible")(xs)
    for g, name in zip(got[:5], ("dexpf", "dlogf", "dsinf", "dcosf", "dtanhf")):
        _assert_same_bits(g, getattr(oracle, name)(xs), name)
    with np.errstate(all="ignore"):
        _assert_same_bits(got[5], np.sqrt(xs), "sqrtf")


def test_gbm_config3_reproducible_bit_exact():
    """Config 3's GBM kernel under REPRODUCIBLE, path by path equal to
    oracle_gbm_r (Threefry, JAX's uniform conversion, Box-Muller with the
    deterministic log, cos and exp, 252 steps) on the first 1M paths and
    the last 64K, and within FAST's tolerance of the IEEE oracle."""
    from palladium_amd.frontend import random
    from palladium_amd.workloads import GBM_CFG, gbm_call

    cfg = GBM_CFG
    print(f"[reproducible] gbm_paths n={cfg.n_paths} steps={cfg.n_steps}", flush=True)
    got = gbm_call(cfg, math_mode="reproducible")(random.key(cfg.seed))
    head = 1 << 20
    tail = 1 << 16
    _assert_same_bits(got[:head], oracle.gbm(cfg, head, mode="reproducible"), "gbm head")
    _assert_same_bits(got[-tail:], oracle.gbm(cfg, tail, first_path=cfg.n_paths - tail, mode="reproducible"),
                      "gbm tail")
    ieee = oracle.gbm(cfg, head)
    np.testing.assert_allclose(got[:head], ieee, atol=2e-2, rtol=1e-3)


@pytest.mark.parametrize("narrow", ["bfloat16", "float16"])
def test_narrow_float_transcendentals_bit_exact_with_the_interpreter(narrow):
    """bfloat16 and float16 exp, log, sin, cos and tanh under REPRODUCIBLE: the
    device computes them in float32 with the deterministic forms and rounds,
    and the interpreter does the same, so every bit pattern of the format
    (NaNs aside, compared as NaN) gives the same result on both."""
    from palladium_amd import dtypes
    from palladium_amd.frontend import jnp

    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    if narrow == "bfloat16":
        dt = dtypes.bfloat16
        x = dtypes.from_float((bits.astype(np.uint32) << 16).view(np.float32))
    else:
        dt = np.dtype(np.float16)
        x = bits.view(np.float16)
    n = 1 << 16
    print(f"[reproducible] {narrow} exp/log/sin/cos over all {n} patterns", flush=True)
    s = pl.BlockSpec((1,), lambda i: (i,))

    def k(x_ref, e_ref, l_ref, s_ref, c_ref, t_ref):
        v = x_ref[...]
        e_ref[...] = jnp.exp(v)
        l_ref[...] = jnp.log(v)
        s_ref[...] = jnp.sin(v)
        c_ref[...] = jnp.cos(v)
        t_ref[...] = jnp.tanh(v)

    call = pa.hip_call(k, grid=(n,), in_specs=[s], out_specs=[s] * 5,
                       out_shape=tuple(pl.ShapeDtypeStruct((n,), dt) for _ in range(5)), math_mode="reproducible")
    got = call(x)
    want = call.interpret(x)
    for g, w, name in zip(got, want, ("exp", "log", "sin", "cos", "tanh")):
        gf = dtypes.to_float(g) if dtypes.is_bf16(g.dtype) else np.asarray(g, np.float32)
        wf = dtypes.to_float(w) if dtypes.is_bf16(w.dtype) else np.asarray(w, np.float32)
        _assert_same_bits(gf.astype(np.float32), wf.astype(np.float32), f"{narrow} {name}")


def _butterfly_block_sums(v: np.ndarray, block: int) -> np.ndarray:
    """The device's cross-lane sum of each block of `block` float32 values:
    a __shfl_xor butterfly inside each 64-lane wavefront (lane i adds lane
    i ^ off, off = 32 .. 1), then the wavefronts' partials added in order."""
    w = v.reshape(-1, block // 64, 64)
    off = 32
    while off >= 1:
        w = w[..., :off] + w[..., off:2 * off]
        off //= 2
    parts = w[..., 0]
    acc = parts[:, 0].copy()
    for k in range(1, parts.shape[1]):
        acc = acc + parts[:, k]
    return acc


def test_gbm_block_sums_config3_reproducible_bit_exact():
    """Config 3's stated output (the discounted payoff summed per block of
    256 paths, the paths spread over the block's lanes) under REPRODUCIBLE:
    all 16,384 block sums equal oracle_gbm_r's payoffs, discounted and summed
    in the device's cross-lane order, bit for bit."""
    import math

    from palladium_amd.frontend import random
    from palladium_amd.workloads import GBM_CFG, gbm_block_call

    cfg = GBM_CFG
    block = 256
    print(f"[reproducible] gbm_block_sums n={cfg.n_paths} block={block}", flush=True)
    got = gbm_block_call(cfg, block=block, math_mode="reproducible")(random.key(cfg.seed))
    payoff = oracle.gbm(cfg, cfg.n_paths, mode="reproducible")
    disc = np.float32(math.exp(-cfg.r * cfg.t))
    want = _butterfly_block_sums(disc * payoff, block)
    _assert_same_bits(np.asarray(got, np.float32), want.astype(np.float32), "gbm block sums")


def test_gray_scott_reproducible_bit_exact_vs_interpreter():
    """Config 4's per-step kernel under REPRODUCIBLE (FAST's algebra, fused
    multiply-adds at the contraction's sites) on a 128 x 128 grid, 20 steps
    chained on the device and in the interpreter, bit for bit."""
    from palladium_amd.workloads import gray_scott_call, gray_scott_initial

    n = 128
    u, v = gray_scott_initial(n)
    call = gray_scott_call(size=n, math_mode="reproducible")
    src = call.bound(u, v).hip_source
    assert "__builtin_fmaf" in src[src.index('extern "C"'):]
    du, dv = u, v
    hu, hv = u, v
    for _ in range(20):
        du, dv = call(du, dv)
        hu, hv = call.interpret(hu, hv)
    np.testing.assert_array_equal(du, hu)
    np.testing.assert_array_equal(dv, hv)


def test_lv_config0_blocks_reproducible_bit_exact():
    """Config 0 (N = 100,000, dt = 0.01, 1,000 steps, 256-trajectory blocks
    spread over lanes, the last block ragged) under REPRODUCIBLE: final
    states equal oracle_lv_rk4_r's bit for bit."""
    from palladium_amd.workloads import LV_CFG0, lv_inputs, lv_rk4_call

    cfg = LV_CFG0
    args = lv_inputs(cfg.n, cfg.seed)
    print(f"[reproducible] lv_rk4 config 0 n={cfg.n} blocks of 256", flush=True)
    got = lv_rk4_call(cfg.n, cfg.dt, cfg.steps, track_max=False, block=256, math_mode="reproducible")(*args)
    want = oracle.lv_rk4_r(*args, cfg.dt, cfg.steps)
    np.testing.assert_array_equal(got[0], want[0])
    np.testing.assert_array_equal(got[1], want[1])
