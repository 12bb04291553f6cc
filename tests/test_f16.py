"""float16 kernels: staging, lowering and interpretation (CPU)."""

import numpy as np

from f16_cases import arithmetic, inputs, transcendental
from palladium_amd import runtime as rt
from palladium_amd.emit import emit_hip
from palladium_amd.frontend import pl
from palladium_amd.trace import trace


def test_promotion_follows_jax():
    seen = {}

    def kernel(h_ref, f_ref, i_ref, o_ref):
        h, f, i = h_ref[...], f_ref[...], i_ref[...]
        seen["h+1.5"] = (h + 1.5).dtype
        seen["h+f"] = (h + f).dtype
        seen["h+i"] = (h + i).dtype
        o_ref[...] = f

    call = pl.pallas_call(kernel, out_shape=pl.ShapeDtypeStruct((4,), np.float32))
    trace(call, np.zeros(4, np.float16), np.zeros(4, np.float32), np.zeros(4, np.int32))
    assert seen == {"h+1.5": np.float16, "h+f": np.float32, "h+i": np.float16}


def test_interpreter_close_to_float64():
    x, y = inputs()
    o, c, i = arithmetic().interpret(x, y)
    assert o.dtype == np.float16
    xd, yd = x.astype(np.float64), y.astype(np.float64)
    z = xd * yd + np.float16(0.1) * xd - yd / (xd * xd + 1.0)
    z = np.where(z > 0, z * 3.0, np.abs(z) - 0.5)
    z = z + np.maximum(xd, yd) - np.minimum(xd, -yd) + yd**3
    ok = np.isfinite(z) & (np.abs(z) < 6e4)
    np.testing.assert_allclose(o[ok], z[ok], rtol=1e-2, atol=2e-2)
    np.testing.assert_array_equal(i, np.trunc((y * np.float16(100)).astype(np.float64)).astype(np.int32))


def test_literals_are_float16_rounded():
    spec = trace(arithmetic()._staged, *inputs())
    src = emit_hip(spec)
    assert "0.0999755859375f" in src  # float16(0.1), not float32(0.1)
    assert "_Float16" in src


def test_sources_compile_for_gfx950():
    x, y = inputs()
    for f, args in ((arithmetic(), (x, y)), (transcendental(), (x,))):
        spec = trace(f._staged, *args)
        for mode in ("safe", "fast"):
            rt.compile_code_object(emit_hip(spec, math_mode=mode), spec.name, mode)


def test_transcendental_interpreter_in_float16():
    x, _ = inputs()
    o, s = transcendental().interpret(x)
    xd = x.astype(np.float64)
    with np.errstate(over="ignore"):
        z = np.exp(xd * 0.5) + np.log(np.abs(xd) + 1.0) + np.sin(xd) + np.sqrt(np.abs(xd))
    ok = np.abs(z) < 6e4
    np.testing.assert_allclose(o[ok], z[ok], rtol=5e-3, atol=5e-3)
    assert s.dtype == np.float16 and s.shape == (x.size // 64,)
