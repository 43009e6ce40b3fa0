"""The load-time validator through the C-ABI (seeml_hip_validate_instruction),
with the reference's own cases (test/runtime/validator/validator_test.cc)."""
import pytest

from helpers import NULL, RO, compile_workload, instr, validate
from seeml_amd import planner

A, R = 1024, 256  # arena / rodata sizes of the reference test fixture
OP = planner.OP


def ok(ins, arena=A, rodata=R, version=7):
    rc, msg = validate(ins, arena, rodata, version)
    assert rc == 0, msg


def bad(ins, arena=A, rodata=R, version=7, contains=None):
    rc, msg = validate(ins, arena, rodata, version)
    assert rc == 1
    assert msg.startswith("PlanValidator: ")
    if contains:
        assert contains in msg, msg
    return msg


def add_ew(x, y, o, n):
    return instr(OP["AddEW"], [x, y, o], [n])


def test_accepts_in_bounds_operands():
    ok(add_ew(0, 256, 512, 64))


def test_transformer_opcodes_are_version_gated():
    attn = instr(OP["AttnFwd"], [0, 64 * 4, 128 * 4, 192 * 4], [256 * 4, (1 << 32) | 4, (2 << 32) | 4])
    ok(attn, arena=2048)
    bad(attn, arena=2048, version=5, contains="pre-v6 plan")
    bad(instr(OP["AttnFwd"], [0, 256, 512, 0], [1024, (1 << 32) | 4, (2 << 32) | 4]), arena=2048)
    bad(instr(OP["AttnFwd"], [0, 256, 512, 768], [1024, (1 << 32) | 4, 4]), arena=2048)


def test_rmsnorm_backward_proves_the_stats_ref():
    ok(instr(OP["RmsNormBwd"], [0, 128, 256, 512], [768, (4 << 32) | 8]))
    bad(instr(OP["RmsNormBwd"], [0, 128, 256, 512], [A - 4, (4 << 32) | 8]))


def test_attention_backward_extents_are_proven():
    ok(instr(OP["AttnDP"], [0, 128, 256], [(1 << 32) | 4, (2 << 32) | 4]))
    bad(instr(OP["AttnDP"], [0, 128, A - 64], [(1 << 32) | 4, (2 << 32) | 4]))
    bad(instr(OP["AttnDP"], [0, 128, 64], [(1 << 32) | 4, (2 << 32) | 4]))


def test_softmax_rows_backward_overflow_is_rejected():
    bad(instr(OP["SoftmaxRowsBwd"], [0, 256, 512], [(0xFFFFFFFF << 32) | 0xFFFFFFFF]))


def test_embed_proves_buffers_and_demands_rodata_table():
    emb = [0, RO | 0, 64]
    ok(instr(OP["EmbedFwd"], emb, [4, (8 << 32) | 4]))
    bad(instr(OP["EmbedFwd"], [0, 256, 64], [4, (8 << 32) | 4]))
    bad(instr(OP["EmbedFwd"], emb, [4, (8 << 32) | 4]), version=6, contains="token opcode")
    bad(instr(OP["EmbedFwd"], [0, RO, A - 32], [4, (8 << 32) | 4]))
    bad(instr(OP["EmbedFwd"], [0, RO, 0], [4, (8 << 32) | 4]))


def test_rope_requires_even_head_width():
    bad(instr(OP["RopeFwd"], [0, 96], [(1 << 32) | 2, (2 << 32) | 3]))
    ok(instr(OP["RopeFwd"], [0, 512], [(1 << 32) | 2, (2 << 32) | 4]))


def test_rejects_reads_past_the_arena():
    bad(add_ew(900, 0, 256, 64), contains="instruction operand out of bounds")


def test_rejects_writes_into_rodata():
    bad(add_ew(0, 256, RO | 0, 16))
    bad(instr(OP["Fill"], [RO | 0], [16]))


def test_rejects_null_refs_and_unknown_opcodes():
    bad(add_ew(NULL, 0, 256, 16))
    bad(instr(0xFFFF), contains="unknown opcode")


def test_quantized_weights_must_live_in_rodata():
    bad(instr(OP["GemmNNQ8"], [0, 64, 512], [2, 2, 2]))
    ok(instr(OP["GemmNNQ8"], [0, RO, 512], [2, 2, 2]))


def test_write_ranges_must_not_alias():
    bad(add_ew(0, 512, 128, 64), contains="alias")
    ok(add_ew(0, 0, 512, 64))
    bad(add_ew(0, 256, 32, 16))


def test_in_place_optimizer_steps_alias_only_through_one_ref():
    ok(instr(OP["SgdStep"], [0, 256], [64]))
    bad(instr(OP["SgdStep"], [0, 128], [64]))
    ok(instr(OP["AdamWStep"], [0, 256, 512, 768], [64]))
    bad(instr(OP["AdamWStep"], [0, 256, 512, 512], [64]))


def test_bounds_math_is_overflow_safe():
    bad(add_ew(0, 0, 0, (1 << 64) // 2 - 1))


def gemm(a, b, c, m, n, k, flags=0, bias=NULL):
    return instr(OP["GemmNN"], [a, b, c, bias], [m, n, k], flags)


def test_flag_discipline():
    g = gemm(0, 64, 512, 4, 4, 4, flags=1, bias=256)
    bad(g, version=4, contains="flags")
    bad(gemm(0, 64, 512, 4, 4, 4, flags=1 << 15), contains="flags")
    bad(instr(OP["AddEW"], [0, 256, 512], [16], flags=1 << 1))
    ok(gemm(0, 64, 512, 4, 4, 4, flags=1 | (2 << 1), bias=256))
    bad(gemm(0, 64, 512, 4, 4, 4, flags=1 | (2 << 1), bias=1020))
    bad(gemm(0, 64, 512, 4, 4, 4, flags=1 | (2 << 1), bias=512), contains="alias")
    ok(instr(OP["GemmNNQ8"], [0, RO, 512], [2, 2, 2], flags=3 << 1))
    bad(instr(OP["GemmNNQ8"], [0, RO, 512], [2, 2, 2], flags=1 | (3 << 1)))


def test_zero_extent_and_misaligned_operands():
    bad(instr(OP["SoftmaxXEntFwd"], [0, 256, 512, 640], [4, 0]))
    ok(instr(OP["SoftmaxXEntFwd"], [0, 256, 512, 640], [4, 4]))
    bad(add_ew(0, 256, 512, 0))
    bad(add_ew(2, 256, 512, 16))
    ok(instr(OP["GemmNNQ8"], [0, RO | 3, 512], [2, 2, 2]))


@pytest.mark.parametrize("name", ["c1", "c3s", "c5s"])
def test_every_compiled_instruction_validates(name):
    w, p = compile_workload(name)
    h = p.header
    for prog in (p.train, p.merge, p.eval):
        for ins in prog:
            word = planner.INSTR.pack(ins["opcode"], ins["flags"], 0, *ins["inp"], *ins["out"])
            ok(word, arena=h["arena_size"], rodata=h["rodata_size"])
