"""Lowering of a formal Program onto the rocm quantized-linear kernels.

The reference compiler maps every Program node to one physical implementation
and names it in the executable explanation (src/js/compute/native.zig:1314-1322).
On the rocm device the only kernels are quantized_matmul's, so the element-wise
nodes a decoder block authors after its projections
(packages/@affon/models/src/llama/model.ts:82, docs/core/quantized-inference.md:37-42)
are absorbed into the projection kernel's output epilogue:

* ``add(quantized_matmul(x, W), bias)`` with ``bias`` an ``[N]`` argument
  becomes one ``bias`` step;
* ``mul(silu(quantized_matmul(x, Wg)), quantized_matmul(x, Wu))`` (either
  operand order), with both projections reading the same input with the same
  options and weight specs, becomes one ``silu_gate`` step.

Plain and bias steps that read the same input with the same options (a
block's query, key and value) are then gathered, up to four at a time, into
one ``grouped`` step: one launch where the M = 1 kernel takes them all.

An absorbed node must have exactly one user and must not be a Program output.
Any element-wise node that does not fit a pattern has no rocm kernel and is
rejected at compile time, as the reference compiler rejects an operation its
backend lacks.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Sequence

ELEMENTWISE = ("add", "mul", "silu")
# Ops with a rocm kernel of their own: one step each.
STANDALONE = ("rms_norm", "softmax", "index_select")


@dataclass
class Step:
    """One launch sequence: ``kind`` is "quantized_matmul", "bias",
    "silu_gate" or "grouped"; ``node`` the node whose value it produces;
    ``operands`` the node ids it reads (x, packed, scales, biases, then the
    bias or the up projection's packed, scales, biases); ``absorbed`` the node
    ids folded in; a grouped step's ``members`` are plain and bias steps."""
    kind: str
    node: int
    operands: list[int]
    options: dict[str, Any]
    absorbed: list[int] = field(default_factory=list)
    members: list["Step"] = field(default_factory=list)

    @property
    def nodes(self) -> list[int]:
        """Every node the step computes or absorbs."""
        if self.members:
            return sorted(n for m in self.members for n in m.nodes)
        return sorted(self.absorbed + [self.node])


MAX_GROUP = 4


def _users(nodes: Sequence[dict[str, Any]]) -> dict[int, list[int]]:
    users: dict[int, list[int]] = {n["id"]: [] for n in nodes}
    for n in nodes:
        for o in n.get("operands", []):
            users[o].append(n["id"])
    return users


def lower(nodes: Sequence[dict[str, Any]], outputs: Sequence[int]) -> list[Step]:
    by_id = {n["id"]: n for n in nodes}
    users = _users(nodes)
    outs = set(outputs)

    def op(i: int) -> str | None:
        n = by_id[i]
        return n["op"] if n["kind"] == "operation" else None

    def private(i: int, user: int) -> bool:
        """Node i feeds only `user` and is not an output."""
        return users[i] == [user] and i not in outs

    def reject(node: dict[str, Any], why: str) -> TypeError:
        return TypeError(f"unsupported operation on rocm: {node['op']} ({why})")

    steps: list[Step] = []
    absorbed: set[int] = set()
    pending: dict[int, Step] = {}  # quantized_matmul nodes not yet emitted
    for n in nodes:
        if n["kind"] != "operation":
            continue
        i = n["id"]
        if n["op"] == "quantized_matmul":
            pending[i] = Step("quantized_matmul", i, list(n["operands"]), dict(n["options"]))
            continue
        if n["op"] in STANDALONE:
            steps.append(Step(n["op"], i, list(n["operands"]), dict(n["options"])))
            continue
        if n["op"] == "silu":
            (src,) = n["operands"]
            if op(src) != "quantized_matmul" or not private(src, i) or len(users[i]) != 1 or i in outs \
                    or op(users[i][0]) != "mul":
                raise reject(n, "silu is lowered only as the gate of mul(silu(quantized_matmul), quantized_matmul)")
            continue  # handled with its mul
        if n["op"] == "add":
            a, b = n["operands"]
            q, bias = (a, b) if op(a) == "quantized_matmul" else (b, a)
            qn, bn = by_id[q], by_id[bias]
            if op(q) != "quantized_matmul" or not private(q, i):
                raise reject(n, "add is lowered only as an output bias of a quantized_matmul used nowhere else")
            if bn["kind"] != "argument" or len(bn["spec"].shape) != 1 or bn["spec"].shape[0] != qn["spec"].shape[1] \
                    or bn["spec"].dtype not in ("f32", "bf16"):
                raise reject(n, "the bias must be an f32/bf16 [N] argument")
            step = pending.pop(q)
            steps.append(Step("bias", i, step.operands + [bias], step.options, [q]))
            absorbed.add(q)
            continue
        if n["op"] == "mul":
            a, b = n["operands"]
            s_node, u = (a, b) if op(a) == "silu" else (b, a)
            if op(s_node) != "silu" or op(u) != "quantized_matmul" or not private(s_node, i) or not private(u, i):
                raise reject(n, "mul is lowered only as mul(silu(quantized_matmul), quantized_matmul)")
            g = by_id[s_node]["operands"][0]
            gn, un = by_id[g], by_id[u]
            same_input = gn["operands"][0] == un["operands"][0]
            same_weights = all(by_id[x]["spec"] == by_id[y]["spec"] for x, y in zip(gn["operands"][1:], un["operands"][1:]))
            if not (same_input and same_weights and gn["options"] == un["options"]):
                raise reject(n, "gate and up must read the same input with the same options and weight shapes")
            gate, up = pending.pop(g), pending.pop(u)
            steps.append(Step("silu_gate", i, gate.operands + up.operands[1:], gate.options, [g, s_node, u]))
            absorbed.update((g, s_node, u))
            continue
        raise reject(n, "no rocm kernel")
    # quantized_matmul nodes that were not absorbed run on their own, in
    # Program order relative to each other and before any step that reads them.
    ordered: list[Step] = []
    for n in nodes:
        if n["id"] in pending:
            ordered.append(pending[n["id"]])
        ordered.extend(s for s in steps if s.node == n["id"])
    return _group(ordered, by_id)


def _group(steps: list[Step], by_id: dict[int, dict[str, Any]]) -> list[Step]:
    """Gathers plain and bias steps with the same input and options into
    grouped steps, placed where the first member was. Members' other operands
    must be Program arguments, so no step in between can produce them."""
    def groupable(s: Step) -> bool:
        return s.kind in ("quantized_matmul", "bias") and all(by_id[o]["kind"] == "argument" for o in s.operands[1:])

    result: list[Step] = []
    taken: set[int] = set()
    for i, s in enumerate(steps):
        if i in taken:
            continue
        members = [s]
        if groupable(s):
            for j in range(i + 1, len(steps)):
                t = steps[j]
                if len(members) == MAX_GROUP:
                    break
                if j not in taken and groupable(t) and t.operands[0] == s.operands[0] and t.options == s.options:
                    members.append(t)
                    taken.add(j)
        if len(members) == 1:
            result.append(s)
        else:
            result.append(Step("grouped", s.node, [s.operands[0]], s.options, members=members))
    return result
