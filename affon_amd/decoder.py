"""Quantized projections of a Llama-style decoder block, authored as Programs.

The reference Llama (packages/@affon/models/src/llama/model.ts:64-87) gives
each block seven projections: query, key, value and attentionOutput around
attention, and gate, up and down in the feed-forward
``down(mul(silu(gate(h)), up(h)))``. It stores them dense as ``[in, out]``
matrices for ``matmul``. Quantized checkpoints keep the Hugging Face
``[out, in]`` orientation (packages/@affon/huggingface/src/adapters/llama.ts:27-33),
which is exactly quantized_matmul's packed ``[N, K/P]`` row layout, so here each
projection is one quantized_matmul over ``[out, in]`` packed weights.

Each part of the block is a Program whose weights are arguments:
* ``attention_program``: normalized ``[M, width]`` -> (query, key, value), with
  each projection's output bias when the checkpoint has one
  (``add(quantized_matmul(..), bias)``, lowered into the kernel's epilogue);
* ``output_program``: attention ``[M, width]`` -> attentionOutput;
* ``feed_forward_program``: normalized ``[M, width]`` ->
  ``down(mul(silu(gate), up))``, whose gate/up pair lowers to one fused step
  (one launch at M = 1).
Norms, RoPE, attention and the residual adds are other ops, not part of this
path.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Mapping

from . import checkpoint as ckpt
from .core import Program, Session, Tensor, TensorSpec, program
from .ops import add, mul, quantized_matmul, silu

# (block field of LlamaWeights, Hugging Face module, input side, output side)
PROJECTIONS = (
    ("query", "self_attn.q_proj", "width", "width"),
    ("key", "self_attn.k_proj", "width", "kv_width"),
    ("value", "self_attn.v_proj", "width", "kv_width"),
    ("attentionOutput", "self_attn.o_proj", "width", "width"),
    ("gate", "mlp.gate_proj", "width", "inner_width"),
    ("up", "mlp.up_proj", "width", "inner_width"),
    ("down", "mlp.down_proj", "inner_width", "width"),
)


@dataclass(frozen=True)
class DecoderShape:
    """The dimensions create_llama checks (model.ts:17-20)."""
    width: int
    inner_width: int
    heads: int
    kv_heads: int

    def __post_init__(self):
        dims = (self.width, self.inner_width, self.heads, self.kv_heads)
        if any(not isinstance(d, int) or isinstance(d, bool) or d <= 0 for d in dims):
            raise TypeError("Invalid Llama dimensions, RoPE or normalization")
        if self.width % self.heads or self.heads % self.kv_heads or (self.width // self.heads) % 2:
            raise TypeError("Invalid Llama dimensions, RoPE or normalization")

    @property
    def kv_width(self) -> int:
        return self.kv_heads * (self.width // self.heads)

    def features(self, name: str) -> tuple[int, int]:
        """(out, in) of a projection."""
        for field, _, side_in, side_out in PROJECTIONS:
            if field == name:
                return getattr(self, side_out), getattr(self, side_in)
        raise KeyError(name)


class QuantizedDecoderBlock:
    """The seven quantized projections of one block, with optional output
    biases, and the Programs that run them."""

    def __init__(self, shape: DecoderShape, layers: Mapping[str, ckpt.QuantizedLinear],
                 output_biases: Mapping[str, Tensor] | None = None):
        output_biases = dict(output_biases or {})
        names = [p[0] for p in PROJECTIONS]
        if sorted(layers) != sorted(names):
            raise TypeError(f"a decoder block needs the projections {names}")
        first = layers[names[0]]
        session = first.packed.session
        for name in names:
            layer = layers[name]
            out_features, in_features = shape.features(name)
            if (layer.out_features, layer.in_features) != (out_features, in_features):
                raise TypeError(f"{name} must be [{out_features}, {in_features}] (out, in), got "
                                f"[{layer.out_features}, {layer.in_features}]")
            if (layer.bits, layer.group_size) != (first.bits, first.group_size):
                raise TypeError("every projection of a block must share bits and group_size")
            if layer.packed.session is not session:
                raise TypeError("every projection of a block must belong to the same Session")
        for name, bias in output_biases.items():
            if name not in names:
                raise TypeError(f"unknown projection {name}")
            if name in ("gate", "up"):
                raise TypeError("gate and up output biases are not supported (the SiLU-gated product fuses them)")
            if bias.dtype not in ("f32", "bf16") or bias.shape != (shape.features(name)[0],):
                raise TypeError(f"{name} output bias must be an f32/bf16 [{shape.features(name)[0]}] tensor")
        self.shape = shape
        self.layers = dict(layers)
        self.output_biases = output_biases
        self.bits = first.bits
        self.group_size = first.group_size
        self.session: Session = session
        self._programs: dict[tuple[str, int, str], Program] = {}

    # ---- construction from a checkpoint ----

    @classmethod
    def from_checkpoint(cls, session: Session, path: str, index: int, shape: DecoderShape, *, bits: int,
                        group_size: int, prefix: str = "model.layers") -> "QuantizedDecoderBlock":
        """Binds block ``index`` of an MLX-affine checkpoint: ``<prefix>.<index>.
        <module>.weight`` (U32) with ``.scales`` / ``.biases`` per projection,
        and ``<module>.bias`` as the output bias where present."""
        base = f"{prefix}.{index}"
        modules = {field: f"{base}.{module}" for field, module, _, _ in PROJECTIONS}
        bound = ckpt.quantized_linears(session, path, bits=bits, group_size=group_size, prefixes=modules.values())
        header = ckpt.inspect(path)
        bias_names = [m + ".bias" for m in modules.values() if m + ".bias" in header]
        loaded = ckpt.load(session, path, bias_names) if bias_names else {}
        layers = {field: bound[module] for field, module in modules.items()}
        biases = {field: loaded[module + ".bias"] for field, module in modules.items() if module + ".bias" in loaded}
        return cls(shape, layers, biases)

    # ---- Programs ----

    def _weights(self, p, name: str):
        layer = self.layers[name]
        return (p.argument(f"{name}.packed", layer.packed.spec), p.argument(f"{name}.scales", layer.scales.spec),
                p.argument(f"{name}.biases", layer.biases.spec))

    def _project(self, p, name: str, x):
        y = quantized_matmul(x, *self._weights(p, name), bits=self.bits, group_size=self.group_size)
        bias = self.output_biases.get(name)
        if bias is not None:
            y = add(y, p.argument(f"{name}.bias", bias.spec))
        return y

    def _program(self, part: str, rows: int, dtype: str) -> Program:
        key = (part, rows, dtype)
        if key not in self._programs:
            width = self.shape.width
            if part == "attention":
                body = lambda p: self._attention_body(p, rows, dtype)
            elif part == "output":
                body = lambda p: self._project(p, "attentionOutput", p.argument("attention",
                                                                                 TensorSpec(dtype, (rows, width))))
            else:
                body = lambda p: self._feed_forward_body(p, rows, dtype)
            self._programs[key] = program(f"quantized_decoder_{part}", body)
        return self._programs[key]

    def _attention_body(self, p, rows: int, dtype: str):
        h = p.argument("normalized", TensorSpec(dtype, (rows, self.shape.width)))
        return [self._project(p, name, h) for name in ("query", "key", "value")]

    def _feed_forward_body(self, p, rows: int, dtype: str):
        h = p.argument("normalized", TensorSpec(dtype, (rows, self.shape.width)))
        gated = mul(silu(self._project(p, "gate", h)), self._project(p, "up", h))
        return self._project(p, "down", gated)

    def attention_program(self, rows: int, dtype: str = "bf16") -> Program:
        return self._program("attention", rows, dtype)

    def output_program(self, rows: int, dtype: str = "bf16") -> Program:
        return self._program("output", rows, dtype)

    def feed_forward_program(self, rows: int, dtype: str = "bf16") -> Program:
        return self._program("feed_forward", rows, dtype)

    def weight_arguments(self) -> dict[str, Tensor]:
        args: dict[str, Tensor] = {}
        for name, layer in self.layers.items():
            args[f"{name}.packed"], args[f"{name}.scales"], args[f"{name}.biases"] = (layer.packed, layer.scales,
                                                                                   layer.biases)
        for name, bias in self.output_biases.items():
            args[f"{name}.bias"] = bias
        return args

    # ---- running ----

    def _run(self, source: Program, inputs: Mapping[str, Tensor], **options):
        executable = self.session.compile(source, **options)
        arguments = self.weight_arguments()
        needed = {n["name"] for n in source.nodes if n["kind"] == "argument"}
        arguments = {k: v for k, v in arguments.items() if k in needed}
        arguments.update(inputs)
        return executable.run(arguments)

    def attention(self, normalized: Tensor, **options) -> list[Tensor]:
        """(query, key, value) of normalized activations [M, width]."""
        return self._run(self.attention_program(normalized.shape[0], normalized.dtype), {"normalized": normalized},
                         **options)

    def attention_output(self, attention: Tensor, **options) -> Tensor:
        return self._run(self.output_program(attention.shape[0], attention.dtype), {"attention": attention},
                         **options)

    def feed_forward(self, normalized: Tensor, **options) -> Tensor:
        """down(silu(gate(h)) * up(h)) of normalized activations [M, width]."""
        return self._run(self.feed_forward_program(normalized.shape[0], normalized.dtype), {"normalized": normalized},
                         **options)
