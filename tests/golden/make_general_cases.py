"""Writes general_checker_cases.npz: the 192 random cases of the reference's
general quantized checker (test/parity/reference/check-cuda-quantized-general.py:34-59).

The cases come from the reference checker itself: its ``cases()`` and
``view()`` are imported from the reference tree (build container only; the
reference does not travel to the GPU box), so the draw order, seed
(20261105) and layouts are the checker's own. Stored per case, as the
checker's ``view()`` hands them to its worker: the logical activations,
scales and biases (f32; already rounded to bf16 in the bf16 cases), and the
codes recovered from the packed words. Layouts and dtypes stay encoded in
the case ids as in the reference.

Run: python tests/golden/make_general_cases.py [--check]
"""
import argparse
import importlib.util
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
REFERENCE_CHECKER = pathlib.Path("/root/reference/test/parity/reference/check-cuda-quantized-general.py")
SEED = 20261105


def reference_checker():
    spec = importlib.util.spec_from_file_location("reference_general_checker", REFERENCE_CHECKER)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def logical_cases(checker, seed=SEED):
    """(id|group, x, q, s, b) per reference case, logical (un-strided) values."""
    import torch

    result = []
    for case in checker.cases(seed):
        bits, group = case["bits"], case["group_size"]
        per_word = 32 // bits
        inputs = {name: checker.view(value) for name, value in case["inputs"].items()}
        shifts = torch.arange(per_word) * bits
        codes = ((inputs["w"].unsqueeze(-1) >> shifts) & ((1 << bits) - 1)).flatten(1)
        result.append((f"{case['id']}|{group}", inputs["x"].float().contiguous().numpy(),
                       codes.to(torch.uint8).contiguous().numpy(), inputs["s"].float().contiguous().numpy(),
                       inputs["b"].float().contiguous().numpy()))
    return result


def main():
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--check", action="store_true", help="compare with the committed file instead of writing it")
    args = parser.parse_args()
    arrays, ids = {}, []
    for i, (case_id, x, q, s, b) in enumerate(logical_cases(reference_checker())):
        ids.append(case_id)
        arrays[f"x{i}"], arrays[f"q{i}"], arrays[f"s{i}"], arrays[f"b{i}"] = x, q, s, b
    arrays["ids"] = np.array(ids)
    target = HERE / "general_checker_cases.npz"
    if args.check:
        old = np.load(target)
        same = list(old["ids"]) == ids and all(
            np.array_equal(old[k], arrays[k]) for k in arrays if k != "ids")
        print(f"{len(ids)} cases; committed file {'matches' if same else 'DIFFERS'}")
        return 0 if same else 1
    np.savez_compressed(target, **arrays)
    print(len(ids), "cases")
    return 0


if __name__ == "__main__":
    sys.exit(main())
