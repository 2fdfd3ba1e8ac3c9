"""The counted waits of the tiled kernels' transfer plans (lds_pipeline.h
Plan::wait_own for the decode-batch kernel, Plan::wait and the prologue
wait for the prefill GEMM, RePlan::wait for the reassociated prefill GEMM)
against an independent simulation of the issue stream.

The simulation lists every transfer instruction the kernels issue, in
order, with the K steps whose data it carries (parameter windows, packed
words, activations), from the kernels' schedules as their comments state
them -- not from the plan's counting formulas. At the start of iteration t
a wave may leave in flight exactly the transfers issued after the last one
that carries data that iteration reads, because the load counter drains in
issue order. Every bound the plan computes must be at most that (a larger
one would let the iteration read LDS before its data landed), and in the
steady state equal to it (a smaller one waits for transfers it does not
need). The plan's values come from a host program compiled with hipcc.
"""
import pathlib
import shutil
import subprocess

import pytest

REPO = pathlib.Path(__file__).resolve().parents[1]
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

# (name, BITS, PT bytes, activation transfers per step, PWHOLE, steps per
# word transfer, activations issued first) of every plan the kernels
# instantiate: the decode-batch kernel (8, 16, 32 activation rows = 1, 2, 4
# transfers per step; 8-bit words two steps at a time up to 16 rows) ...
SKINNY = []
for bits in (2, 4, 8):
    for pt in (2, 4):
        for aloads in (1, 2, 4):
            for whole in (False, True):
                ws = (2 if aloads <= 2 else 1) if bits == 8 else 4
                SKINNY.append((f"skinny_b{bits}_p{pt}_a{aloads}_w{int(whole)}", bits, pt, aloads, whole, ws, True))
# ... and the prefill GEMM (four 8-row activation transfers per step).
GEMM = [(f"gemm_b{bits}_p{pt}", bits, pt, 4, False, 1 if bits == 8 else 4, False) for bits in (2, 4, 8) for pt in (2, 4)]

DUMP = r"""
#include <cstdio>
#include "lds_pipeline.h"
using namespace affon;
using namespace affon::pipeline;
template <class P>
void dump(const char* name) {
  std::printf("%s", name);
  for (int j = 0; j < 4; ++j) std::printf(" %d", P::wait_own(j));
  for (int j = 0; j < 4; ++j) std::printf(" %d", P::wait(j));
  std::printf(" %d\n", P::ops_after(0, 4, 1));
}
int main() {
@CALLS@
  std::printf("replan");
  for (int j = 0; j < 4; ++j) std::printf(" %d", RePlan::wait(j));
  std::printf(" %d %d %d\n", RePlan::kAOps, RePlan::kWOps, RePlan::kSOps);
  return 0;
}
"""


def plan_type(bits, pt, aloads, whole, ws, afirst):
    ptype = "BF16" if pt == 2 else "F32"
    return f"Plan<{bits}, {ptype}, {aloads}, {str(whole).lower()}, {ws}, {str(afirst).lower()}>"


@pytest.fixture(scope="module")
def plan_values(tmp_path_factory):
    if not pathlib.Path(HIPCC).exists():
        pytest.skip("hipcc is not available")
    d = tmp_path_factory.mktemp("plan")
    calls = "\n".join(f'  dump<{plan_type(*c[1:])}>("{c[0]}");' for c in SKINNY + GEMM)
    src = d / "plan_dump.cpp"
    src.write_text(DUMP.replace("@CALLS@", calls))
    exe = d / "plan_dump"
    cmd = [HIPCC, "--offload-arch=gfx950", "-std=c++17", "-x", "hip", f"-I{REPO / 'include'}",
           f"-I{REPO / 'affon_amd' / 'csrc'}", str(src), "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    values = {}
    for line in out.splitlines():
        name, *nums = line.split()
        nums = list(map(int, nums))
        if name == "replan":
            values[name] = {"wait": nums[0:4], "aops": nums[4], "wops": nums[5], "sops": nums[6]}
        else:
            values[name] = {"own": nums[0:4], "wait": nums[4:8], "prologue": nums[8]}
    return values


def issue_stream(bits, aloads, whole, ws, afirst, iterations):
    """Transfers in issue order as (iteration, kind, covered steps)."""
    w_loads = 64 * (8 * bits * ws) // 1024  # 16-byte transfers per packed-word transfer of 64 columns
    ahead = 3 if ws == 2 else 4
    ops = []
    if whole:  # the whole range's parameters, before every other transfer
        ops += [(-5, "p", None)] * (2 * 64 * 32 // 256)
    for u in range(-4, iterations):
        j = u % 4
        if j == 0 and not whole:  # parameter window of the four steps u+4 .. u+7
            ops += [(u, "p", set(range(u + 4, u + 8)))] * 8
        words = []
        if (ws == 2 and j % 2 == 1) or ws == 1 or (ws == 4 and j == 0):
            words = [(u, "w", set(range(u + ahead, u + ahead + ws)))] * w_loads
        # activations of step u+3; the first prologue iteration repeats step 0
        acts = [(u, "a", {max(u + 3, 0)})] * aloads
        ops += acts + words if afirst else words + acts
    return ops


def allowed_in_flight(ops, before_iteration, needs):
    """Transfers issued before `before_iteration` that may still be in flight
    when every transfer carrying one of `needs` = {(kind, step)} has landed."""
    issued = [o for o in ops if o[0] < before_iteration]
    last = -1
    for i, (_, kind, steps) in enumerate(issued):
        if any(k == kind and (steps is None or s in steps) for k, s in needs):
            last = i
    assert last >= 0, (before_iteration, needs)
    return len(issued) - 1 - last


@pytest.mark.parametrize("case", SKINNY, ids=[c[0] for c in SKINNY])
def test_decode_batch_waits_cover_exactly_the_step(plan_values, case):
    name, bits, pt, aloads, whole, ws, afirst = case
    ops = issue_stream(bits, aloads, whole, ws, afirst, 40)
    own = plan_values[name]["own"]
    assert max(own) < 64  # s_waitcnt vmcnt range
    for t in range(0, 32):
        needs = {("a", t), ("w", t), ("p", t)}
        sim = allowed_in_flight(ops, t, needs)
        assert own[t % 4] <= sim, (t, own[t % 4], sim)
        if t >= 8:
            assert own[t % 4] == sim, (t, own[t % 4], sim)


@pytest.mark.parametrize("case", GEMM, ids=[c[0] for c in GEMM])
def test_prefill_gemm_waits(plan_values, case):
    name, bits, pt, aloads, whole, ws, afirst = case
    ops = issue_stream(bits, aloads, whole, ws, afirst, 40)
    values = plan_values[name]
    # Before iteration 0: the packed words of step 0 (decoded in the prologue).
    sim0 = allowed_in_flight(ops, 0, {("w", 0)})
    assert values["prologue"] <= sim0 and values["prologue"] == sim0
    # Iteration t reads its step's activations and decodes step t+1.
    for t in range(0, 32):
        needs = {("a", t), ("w", t + 1), ("p", t + 1)}
        sim = allowed_in_flight(ops, t, needs)
        assert values["wait"][t % 4] <= sim, (t, values["wait"][t % 4], sim)
        if t >= 8:
            assert values["wait"][t % 4] == sim, (t, values["wait"][t % 4], sim)


def test_simulation_detects_a_wait_one_too_large(plan_values):
    """The check has teeth: the 4-bit plan's bound plus one fails it."""
    name, bits, pt, aloads, whole, ws, afirst = SKINNY[[c[0] for c in SKINNY].index("skinny_b4_p2_a2_w1")]
    ops = issue_stream(bits, aloads, whole, ws, afirst, 40)
    own = plan_values[name]["own"]
    sim = allowed_in_flight(ops, 12, {("a", 12), ("w", 12), ("p", 12)})
    assert own[0] == sim and not (own[0] + 1 <= sim)


def re_issue_stream(aops, wops, sops, iterations):
    """The reassociated prefill GEMM (gemm_re.hip), one wave, in issue order:
    the K range's scales; the packed words of steps 0..3; the activations of
    steps 0 and 1; then iteration t issues the activations of step t+2 and, at
    t % 4 == 0, the packed words of steps t+4 .. t+7."""
    ops = [(-3, "p", None)] * sops + [(-3, "w", {0, 1, 2, 3})] * wops
    ops += [(-2, "a", {0})] * aops + [(-1, "a", {1})] * aops
    for t in range(iterations):
        ops += [(t, "a", {t + 2})] * aops
        if t % 4 == 0:
            ops += [(t, "w", set(range(t + 4, t + 8)))] * wops
    return ops


def test_reassociated_gemm_waits(plan_values):
    v = plan_values["replan"]
    ops = re_issue_stream(v["aops"], v["wops"], v["sops"], 40)
    # Before the loop the kernel decodes step 0's packed words after waiting
    # for all but the two activation transfers (2 * aops).
    assert 2 * v["aops"] == allowed_in_flight(ops, 0, {("w", 0), ("p", 0)})
    # Iteration t reads step t's activations, packed words and scales, and the
    # next step's packed words (decoded one step ahead).
    for t in range(0, 32):
        needs = {("a", t), ("w", t), ("w", t + 1), ("p", t)}
        sim = allowed_in_flight(ops, t, needs)
        assert v["wait"][t % 4] <= sim, (t, v["wait"][t % 4], sim)
        if t >= 4:
            assert v["wait"][t % 4] == sim, (t, v["wait"][t % 4], sim)
