"""Writes general_checker_cases.npz: the 192 random cases of the reference's
general quantized checker (test/parity/reference/check-cuda-quantized-general.py:34-59),
regenerated with the same torch generator, seed (20261105) and draw order.

Values only (inputs in f32 and codes); layouts and dtypes are encoded in the
case ids as in the reference. Run: python tests/golden/make_general_cases.py
"""
import pathlib

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent


def cases(seed=20261105):
    rng = torch.Generator().manual_seed(seed)
    result = []
    for bits in (2, 4, 8):
        per_word = 32 // bits
        factor = int(torch.randint(1, 34, (), generator=rng))
        dims = [(1, per_word * 3, 5, 3), (3, per_word * 17, 19, per_word),
                (int(torch.randint(1, 13, (), generator=rng)), per_word * factor,
                 int(torch.randint(1, 24, (), generator=rng)), factor), (7, per_word * 31, 3, 31)]
        for x_dtype in ("f32", "bf16"):
            for p_dtype in ("f32", "bf16"):
                for index, (rows, inner, columns, group) in enumerate(dims):
                    for layout in ("dense", "offset", "strided", "transposed"):
                        x = torch.rand((rows, inner), generator=rng) - 0.5
                        q = torch.randint(0, 1 << bits, (columns, inner), generator=rng)
                        scales = torch.rand((columns, inner // group), generator=rng) / (1 << bits)
                        biases = (torch.rand((columns, inner // group), generator=rng) - 0.5) / 4
                        result.append((f"q{bits}/{x_dtype}/{p_dtype}/{index}/{layout}", group, x.numpy(),
                                       q.numpy().astype(np.uint8), scales.numpy(), biases.numpy()))
    return result


def main():
    arrays = {}
    ids = []
    for i, (case_id, group, x, q, s, b) in enumerate(cases()):
        ids.append(f"{case_id}|{group}")
        arrays[f"x{i}"], arrays[f"q{i}"], arrays[f"s{i}"], arrays[f"b{i}"] = x, q, s, b
    arrays["ids"] = np.array(ids)
    np.savez_compressed(HERE / "general_checker_cases.npz", **arrays)
    print(len(ids), "cases")


if __name__ == "__main__":
    main()
