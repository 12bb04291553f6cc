"""The in-order loop latency model (palladium_amd.isa) on synthetic
disassembly and on this build's own BS3 code object (CPU: hiprtc compiles
without a GPU)."""

import os

import pytest

from palladium_amd import isa

_SYNTH = """
\tv_mov_b32_e32 v1, 0                                  // 000000000000: 00000000
\tv_fma_f32 v1, v1, v2, v3                             // 000000000004: 00000000
\tv_fma_f32 v1, v1, v2, v3                             // 00000000000C: 00000000
\tv_exp_f32_e32 v1, v1                                 // 000000000014: 00000000
\tv_add_f32_e32 v4, v5, v6                             // 000000000018: 00000000
\ts_branch 65530                                       // 00000000001C: BF82FFFA
\ts_endpgm                                             // 000000000020: BF810000
"""


def test_parse_reads_operands_and_branch_target():
    ins = isa.parse(_SYNTH)
    assert [i.op for i in ins][:3] == ["v_mov_b32_e32", "v_fma_f32", "v_fma_f32"]
    assert ins[1].dst == ("v1",) and set(ins[1].src) >= {"v1", "v2", "v3"}
    # offset -6 dwords from the next instruction (0x20) -> 0x08... relative to 0x1C + 4
    assert ins[5].target == 0x1C + 4 - 24


def test_dependent_chain_sets_the_iteration_time():
    # body: from 0x08 (the second fma) to the branch: fma -> exp -> (next) fma ...
    asm = _SYNTH.replace("65530", "65529")  # target 0x04: both fmas, the exp, the add
    m = isa.loop_model(asm, lat_valu=4.0, lat_trans=10.0, issue=1.0)
    assert m.transcendental == 1 and m.valu == 4
    assert m.cycles_per_iteration == pytest.approx(4 + 4 + 10)
    # with latencies below the issue interval, issue bounds it
    m = isa.loop_model(asm, lat_valu=0.5, lat_trans=0.5, issue=1.0)
    assert m.cycles_per_iteration == pytest.approx(5.0)


def test_independent_work_overlaps_the_chain():
    asm = _SYNTH.replace("65530", "65529")
    a = isa.loop_model(asm, 4.0, 10.0, 1.0).cycles_per_iteration
    extra = _SYNTH.replace("\tv_add_f32_e32 v4, v5, v6                             // 000000000018: 00000000",
                           "\tv_add_f32_e32 v4, v5, v6  // 000000000018: 0\n\tv_add_f32_e32 v7, v8, v9  // 00000000001A: 0").replace("65530", "65529")
    assert len(isa.loop_body(isa.parse(extra))) == len(isa.loop_body(isa.parse(asm))) + 1
    assert isa.loop_model(extra, 4.0, 10.0, 1.0).cycles_per_iteration == a


@pytest.mark.skipif(not os.path.exists(isa.OBJDUMP), reason="ROCm llvm-objdump absent")
def test_bs3_fast_loop_has_one_exp_and_no_branches_inside():
    import palladium_amd as pa  # noqa: F401
    from palladium_amd import runtime as rt
    from palladium_amd.emit import emit_hip
    from palladium_amd.trace import trace
    from palladium_amd.workloads import bs3_inputs, bs3_vdp_call

    n = 4096
    spec = trace(bs3_vdp_call(n)._staged, *bs3_inputs(n))
    code = rt.compile_code_object(emit_hip(spec, math_mode="fast"), spec.name, "fast")
    body = isa.loop_body(isa.parse(isa.disassemble(code)))
    ops = [b.op for b in body]
    # the compacted loop's machine loop runs several attempts per pass
    from palladium_amd.emit.compact import iterations_per_pass

    u = iterations_per_pass(emit_hip(spec, math_mode="fast"))
    assert u == 32
    assert sum(o.startswith("v_exp_") for o in ops) == u
    # log2(err) only: log2(prev) is carried (emit/optimize.py:carry_logs)
    assert sum(o.startswith("v_log_") for o in ops) == u
    # the two divisions of the error norm; 1 / err no longer feeds a carry
    assert sum(o.startswith("v_rcp_") for o in ops) == 2 * u
    assert not any("saveexec" in o for o in ops), "a pow slow path still branches inside the loop"
    m = isa.loop_model(code, 4.0, 12.0, 1.0)
    assert 50 * u < m.valu < 120 * u
    assert m.cycles_per_iteration > m.instructions  # latency, not issue, sets it


@pytest.mark.skipif(not os.path.exists(isa.OBJDUMP), reason="ROCm llvm-objdump absent")
def test_issue_slots_divide_by_the_unroll_factor():
    from palladium_amd import runtime as rt
    from palladium_amd.emit import emit_hip
    from palladium_amd.trace import trace
    from palladium_amd.workloads import lv_inputs, lv_rk4_call

    spec = trace(lv_rk4_call(4096, 0.005, 4000, track_max=True)._staged, *lv_inputs(8, 1))
    code = rt.compile_code_object(emit_hip(spec, math_mode="fast"), spec.name, "fast")
    body = isa.loop_body(isa.parse(isa.disassemble(code)))
    k = isa.unroll_factor(body)
    slots, hist = isa.issue_slots(code, {})
    # one RK4 step of the 58 staged float ops is ~28 VALU instructions after
    # contraction and factoring, however many steps the machine loop holds
    assert 24 <= slots <= 34
    assert sum(b.op.startswith("v_") for b in body) == pytest.approx(slots * k)
    costs = {"v_fma_f32": 1.0, "v_mul_f32": 2.0}
    assert isa.issue_slots(code, costs)[0] == pytest.approx(slots + hist.get("v_mul_f32_e32", 0))


@pytest.mark.skipif(not os.path.exists(isa.OBJDUMP), reason="ROCm llvm-objdump absent")
def test_register_stencil_slots_per_machine_iteration():
    """The register Gray-Scott loop's induction step counts rows, not source
    iterations: per machine iteration its slots are the whole group's."""
    from palladium_amd import runtime as rt
    from palladium_amd import stencil

    code = rt.compile_code_object(stencil.register_source(4096, 6, 64, .16, .08, .037, .097, 1.0, group=4),
                                  "gray_scott_regs", "fast")
    whole, hist = isa.issue_slots(code, {}, per_machine_iteration=True)
    # 4 rows x 6 steps of ~15 float ops per cell, plus addressing
    assert 360 <= whole <= 480 and hist.get("v_add_f32_dpp", 0) == 96
