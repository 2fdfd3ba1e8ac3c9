"""Lowering of formal Programs onto the rocm kernels (CPU: authoring,
pattern matching and compile-time selection from specs; no device work)."""
import pytest

from affon_amd import TensorSpec, lowering, program, quantized_matmul
from affon_amd.decoder import DecoderShape
from affon_amd.ops import add, fused_select_for_specs, mul, silu

BITS, GROUP = 4, 64


def weights(p, name, n, k):
    return (p.argument(f"{name}.packed", TensorSpec.u32([n, k * BITS // 32])),
            p.argument(f"{name}.scales", TensorSpec.bf16([n, k // GROUP])),
            p.argument(f"{name}.biases", TensorSpec.bf16([n, k // GROUP])))


def qmm(x, w):
    return quantized_matmul(x, *w, bits=BITS, group_size=GROUP)


def steps_of(source):
    return lowering.lower(source.nodes, source.outputs)


def test_feed_forward_lowers_to_silu_gate_then_down():
    def body(p):
        h = p.argument("h", TensorSpec.bf16([1, 256]))
        gated = mul(silu(qmm(h, weights(p, "gate", 512, 256))), qmm(h, weights(p, "up", 512, 256)))
        return qmm(gated, weights(p, "down", 256, 512))
    steps = steps_of(program("ffn", body))
    assert [s.kind for s in steps] == ["silu_gate", "quantized_matmul"]
    assert len(steps[0].operands) == 7 and len(steps[0].absorbed) == 3
    assert steps[1].operands[0] == steps[0].node  # down reads the fused product


def test_mul_operand_order_and_bias_either_side():
    def body(p):
        h = p.argument("h", TensorSpec.bf16([2, 128]))
        up = qmm(h, weights(p, "up", 64, 128))
        gated = mul(up, silu(qmm(h, weights(p, "gate", 64, 128))))
        biased = add(p.argument("bias", TensorSpec.f32([64])), qmm(h, weights(p, "o", 64, 128)))
        return [gated, biased]
    source = program("two", body)
    assert source.multiple and len(source.outputs) == 2
    assert [s.kind for s in steps_of(source)] == ["silu_gate", "bias"]


def test_projections_of_one_input_are_grouped_four_at_a_time():
    def body(p):
        h = p.argument("h", TensorSpec.bf16([1, 128]))
        other = p.argument("other", TensorSpec.bf16([1, 128]))
        outs = [qmm(h, weights(p, n, 64, 128)) for n in ("q", "k", "v", "a", "b")]
        outs.append(add(qmm(h, weights(p, "c", 32, 128)), p.argument("c.bias", TensorSpec.f32([32]))))
        outs.append(qmm(other, weights(p, "o", 64, 128)))
        return outs
    steps = steps_of(program("qkv", body))
    assert [s.kind for s in steps] == ["grouped", "grouped", "quantized_matmul"]
    assert [len(s.members) for s in steps[:2]] == [4, 2]
    assert [m.kind for m in steps[1].members] == ["quantized_matmul", "bias"]
    first = [m.node for m in steps[0].members]
    assert first == sorted(first)


def test_grouped_selection_from_specs():
    from affon_amd.ops import grouped_select_for_specs
    opts = {"bits": 4, "group_size": 64}

    def member(m, n):
        return [TensorSpec.bf16([m, 4096]), TensorSpec.u32([n, 512]), TensorSpec.bf16([n, 64]),
                TensorSpec.bf16([n, 64])]
    qkv = [member(1, 4096), member(1, 1024), member(1, 1024)]
    assert grouped_select_for_specs(qkv, opts, "backend_equivalent") == "rocm_quantized_matmul.gemv[grouped:3]"
    biased = [qkv[0] + [TensorSpec.bf16([4096])], qkv[1] + [TensorSpec.bf16([1024])], qkv[2]]
    assert grouped_select_for_specs(biased, opts, "backend_equivalent") == "rocm_quantized_matmul.gemv[grouped:3,bias]"
    batch = [member(2, 4096), member(2, 1024)]  # the virtual-row kernels take no groups
    assert grouped_select_for_specs(batch, opts, "backend_equivalent") == \
        "rocm_quantized_matmul.gemv_mfma;rocm_quantized_matmul.gemv_mfma"
    batch = [member(32, 4096), member(32, 1024), member(32, 1024)]  # the LDS-tiled kernel does
    assert grouped_select_for_specs(batch, opts, "backend_equivalent") == "rocm_quantized_matmul.gemv_mfma[grouped:3]"

    def member_g32(m, n):
        return [TensorSpec.bf16([m, 4096]), TensorSpec.u32([n, 512]), TensorSpec.bf16([n, 128]),
                TensorSpec.bf16([n, 128])]
    # Groups of 32 past M = 4 run on the group-32 GEMM, which takes no groups.
    batch = [member_g32(8, 4096), member_g32(8, 1024)]
    assert grouped_select_for_specs(batch, {"bits": 4, "group_size": 32}, "backend_equivalent") == \
        "rocm_quantized_matmul.gemv_mfma;rocm_quantized_matmul.gemv_mfma"

    def member_b8(m, n):
        return [TensorSpec.bf16([m, 4096]), TensorSpec.u32([n, 1024]), TensorSpec.bf16([n, 64]),
                TensorSpec.bf16([n, 64])]
    # At 8 bits the tiled kernel takes M = 2.
    batch = [member_b8(2, 4096), member_b8(2, 1024)]
    assert grouped_select_for_specs(batch, {"bits": 8, "group_size": 64}, "backend_equivalent") == \
        "rocm_quantized_matmul.gemv_mfma[grouped:2]"


@pytest.mark.parametrize("case", ["silu_alone", "shared_gate", "gate_is_output", "bias_matrix", "different_inputs",
                                  "mul_plain", "add_two_projections"])
def test_unfusable_elementwise_nodes_are_rejected(case):
    def body(p):
        h = p.argument("h", TensorSpec.bf16([1, 128]))
        g = qmm(h, weights(p, "gate", 64, 128))
        u = qmm(h, weights(p, "up", 64, 128))
        if case == "silu_alone":
            return silu(g)
        if case == "shared_gate":
            return [mul(silu(g), u), g]
        if case == "gate_is_output":
            s = silu(g)
            return [mul(s, u), s]
        if case == "bias_matrix":
            return add(g, p.argument("bias", TensorSpec.f32([1, 64])))
        if case == "different_inputs":
            h2 = p.argument("h2", TensorSpec.bf16([1, 128]))
            return mul(silu(g), qmm(h2, weights(p, "up2", 64, 128)))
        if case == "mul_plain":
            return mul(g, u)
        return add(g, u)
    with pytest.raises(TypeError, match="unsupported operation on rocm"):
        steps_of(program("bad", body))


def test_elementwise_ops_are_formal_only():
    with pytest.raises(TypeError, match="no rocm kernel"):
        add(1, 2)
    with pytest.raises(TypeError, match="no rocm kernel"):
        silu(3)
    with pytest.raises(TypeError, match="do not broadcast"):
        program("bad", lambda p: add(p.argument("a", TensorSpec.f32([2, 3])), p.argument("b", TensorSpec.f32([2]))))


def test_fused_selection_from_specs():
    """M = 1 pairs gate and up rows in the decode kernel; M = 2 takes the MFMA
    decode kernel twice; a bias keeps the plain pick."""
    x1, x2 = TensorSpec.bf16([1, 4096]), TensorSpec.bf16([2, 4096])
    w = [TensorSpec.u32([14336, 512]), TensorSpec.bf16([14336, 64]), TensorSpec.bf16([14336, 64])]
    opts = {"bits": 4, "group_size": 64}
    assert fused_select_for_specs("silu_gate", [x1, *w, *w], opts, "backend_equivalent") == \
        "rocm_quantized_matmul.gemv[silu_gate]"
    assert fused_select_for_specs("silu_gate", [x2, *w, *w], opts, "backend_equivalent") == \
        "rocm_quantized_matmul.gemv_mfma;rocm_quantized_matmul.gemv_mfma[gate_mul]"
    assert fused_select_for_specs("silu_gate", [x1, *w, *w], opts, "exact_only") == \
        "rocm_quantized_matmul.generic;rocm_quantized_matmul.generic[gate_mul]"
    assert fused_select_for_specs("bias", [x1, *w, TensorSpec.f32([14336])], opts, "backend_equivalent") == \
        "rocm_quantized_matmul.gemv[bias]"


def test_decoder_shape_checks():
    shape = DecoderShape(4096, 14336, 32, 8)
    assert shape.kv_width == 1024
    assert shape.features("key") == (1024, 4096) and shape.features("down") == (4096, 14336)
    for bad in [(4096, 14336, 32, 5), (4096, 14336, 3, 1), (10, 20, 2, 1), (0, 1, 1, 1)]:
        with pytest.raises(TypeError, match="Invalid Llama dimensions"):
            DecoderShape(*bad)
