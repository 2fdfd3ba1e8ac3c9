"""GPU parity of the quantized decoder-block projections (Programs over a
checkpoint in the Hugging Face module layout) against the CPU oracle.

Tolerances: each projection of a bf16 input is within rtol 1e-2 / atol
1e-2*rms of the oracle's ordered loop; the feed-forward output, whose down
projection reads the f32 SiLU-gated product, is within rtol 2e-3 / atol 1e-4
(the f32-input matmul tolerance) of the oracle's down projection applied to
the same product, which the fused gate/up call returns bit for bit.
"""
import json

import numpy as np
import pytest

import affon_amd as A
from affon_amd.decoder import DecoderShape, PROJECTIONS, QuantizedDecoderBlock
from oracle import oracle as O
from tests.helpers import assert_close_rtol_atol
from tests.test_checkpoint import write_file
from tests.test_gpu_parity import check_against_oracle, dtype_of, upload

pytestmark = pytest.mark.gpu

SHAPE = DecoderShape(width=256, inner_width=768, heads=4, kv_heads=2)
BITS, GROUP = 4, 64


def block_checkpoint(tmp_path, index=3, with_biases=True):
    """A quantized block in MLX-affine form: packed/scales/biases per
    projection (quantized from seeded N(0, 0.02) weights by the oracle) and,
    like Qwen2-style attention, output biases on query/key/value."""
    entries, arrays = [], {}
    for seed, (field, module, _, _) in enumerate(PROJECTIONS):
        out, inp = SHAPE.features(field)
        wf, wb = O.randn(100 + seed, out * inp, 0.0, 0.02)
        packed, s, b = O.quantize(wb.reshape(out, inp), BITS, GROUP, "bf16")
        name = f"model.layers.{index}.{module}"
        arrays[field] = (packed, s, b)
        entries += [(name + ".weight", "U32", list(packed.shape), packed.tobytes()),
                    (name + ".scales", "BF16", list(s.shape), s.tobytes()),
                    (name + ".biases", "BF16", list(b.shape), b.tobytes())]
        if with_biases and field in ("query", "key", "value"):
            bias = O.bf16_from_f32(O.randn(200 + seed, out, 0.0, 0.5)[0])
            arrays[field + ".bias"] = bias
            entries.append((name + ".bias", "BF16", [out], bias.tobytes()))
    path = write_file(tmp_path / "block.safetensors", entries, metadata={"format": "mlx"})
    return str(path), arrays


@pytest.mark.parametrize("M", [1, 2, 32])
def test_decoder_block_programs_against_oracle(session, tmp_path, M):
    path, arrays = block_checkpoint(tmp_path)
    block = QuantizedDecoderBlock.from_checkpoint(session, path, 3, SHAPE, bits=BITS, group_size=GROUP)
    assert sorted(block.output_biases) == ["key", "query", "value"]
    h = O.randn(7, M * SHAPE.width)[1].reshape(M, SHAPE.width)
    ht = upload(session, h, "bf16")

    q, k, v = block.attention(ht)
    for field, out in zip(("query", "key", "value"), (q, k, v)):
        expected = O.add_output_bias(O.quantized_matmul(h, *arrays[field], BITS, GROUP), arrays[field + ".bias"])
        rms = float(np.sqrt(np.mean(expected.astype(np.float64) ** 2)))
        assert_close_rtol_atol(out.numpy(), expected, rtol=1e-2, atol=1e-2 * rms)

    a = O.randn(8, M * SHAPE.width)[1].reshape(M, SHAPE.width)
    o = block.attention_output(upload(session, a, "bf16")).numpy()
    check_against_oracle(o, a, *arrays["attentionOutput"], BITS, GROUP, True)

    y = block.feed_forward(ht).numpy()
    gate = tuple(block.layers["gate"].__dict__[k] for k in ("packed", "scales", "biases"))
    up = tuple(block.layers["up"].__dict__[k] for k in ("packed", "scales", "biases"))
    product = A.quantized_silu_gate(ht, gate, up, bits=BITS, group_size=GROUP).numpy()
    check_against_oracle(y, product, *arrays["down"], BITS, GROUP, False)

    explained = session.compile(block.feed_forward_program(M, "bf16")).explain()["executable"]["physical_nodes"]
    assert [n["op"] for n in explained] == ["quantized_matmul+silu+quantized_matmul+mul", "quantized_matmul"]
    if M == 1:
        assert explained[0]["implementation_id"] == "rocm_quantized_matmul.gemv[silu_gate]"
    else:
        assert explained[0]["implementation_id"].endswith("[gate_mul]")
    attention_nodes = session.compile(block.attention_program(M, "bf16")).explain()["executable"]["physical_nodes"]
    assert [n["op"] for n in attention_nodes] == ["grouped(" + ",".join(["quantized_matmul+add"] * 3) + ")"]
    impl = attention_nodes[0]["implementation_id"]
    if M == 1:
        assert impl == "rocm_quantized_matmul.gemv[grouped:3,bias]", impl
    else:  # one grouped launch on the LDS-tiled kernel, or three launches
        assert impl == "rocm_quantized_matmul.gemv_mfma[grouped:3,bias]" or \
            (impl.count(";") == 2 and impl.endswith("[bias]")), impl


def test_decoder_block_rejects_mismatched_layers(session, tmp_path):
    path, _ = block_checkpoint(tmp_path, with_biases=False)
    block = QuantizedDecoderBlock.from_checkpoint(session, path, 3, SHAPE, bits=BITS, group_size=GROUP)
    assert block.output_biases == {}
    layers = dict(block.layers)
    layers["key"], layers["value"] = layers["query"], layers["key"]  # [256,256] where [128,256] belongs
    with pytest.raises(TypeError, match="key must be"):
        QuantizedDecoderBlock(SHAPE, layers)
    with pytest.raises(TypeError, match="gate and up output biases"):
        QuantizedDecoderBlock(SHAPE, block.layers, {"gate": session.empty("f32", (SHAPE.inner_width,))})
    with pytest.raises(Exception, match="needs .weight"):
        QuantizedDecoderBlock.from_checkpoint(session, path, 4, SHAPE, bits=BITS, group_size=GROUP)
