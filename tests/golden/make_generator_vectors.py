"""Writes tests/golden/generator_vectors.json: the reference's own seeded
generator run under node, for the generator checks in tests/test_oracle.py.

Runs in the build container only (it reads the reference checkout). It
extracts two functions from src/js/compute/program.ts at run time --
`seededRandom` (:1385-1394, mulberry32) and the `normal` closure of
`initializedValue` (:1396-1413, Box-Muller with a cached spare) -- strips
their TypeScript annotations, and runs them under node (v12 here). Nothing of
the reference's source is kept: the committed file holds only the numbers.

For each seed the vectors hold the first 64 uniforms, and the first 65
`normal()` values (an odd count, so the cached spare is exercised) with their
f32 roundings of mean + std * normal() for (mean, std) = (0, 1) and
(0, 0.02) (`Math.fround`, the f64 -> f32 conversion of a Float32Array
element). Numbers are JS shortest round-trip strings, which Python's float()
reads back exactly.
"""
from __future__ import annotations

import json
import pathlib
import re
import subprocess

PROGRAM = pathlib.Path("/root/reference/src/js/compute/program.ts")
OUT = pathlib.Path(__file__).resolve().parent / "generator_vectors.json"
SEEDS = [0, 1, 2, 3, 7, 42, 20261105, 4294967295, -1, 2**32 + 5, 2**53, 1.5]


def block_from(text: str, start: int) -> str:
    """The text from `start` through the brace that closes the first '{' after it."""
    open_at = text.index("{", start)
    depth = 0
    for i in range(open_at, len(text)):
        depth += {"{": 1, "}": -1}.get(text[i], 0)
        if depth == 0:
            return text[start:i + 1]
    raise ValueError("unbalanced braces")


def extract(text: str) -> tuple[str, str]:
    seeded = block_from(text, text.index("function seededRandom("))
    seeded = seeded.replace("function seededRandom(seed: number): () => number {", "function seededRandom(seed) {", 1)
    spare = text.index("let spareNormal")
    normal_start = text.index("const normal = () =>", spare)
    normal = text[spare:normal_start] + block_from(text, normal_start)
    normal = re.sub(r"let spareNormal: number \| undefined", "let spareNormal", normal)
    for js in (seeded, normal):
        if re.search(r":\s*(number|string|boolean)\b|=>\s*number", js.split("{", 1)[1]):
            raise ValueError("a type annotation survived stripping")
    return seeded, normal


def main() -> None:
    seeded, normal = extract(PROGRAM.read_text())
    harness = f"""
'use strict';
{seeded}
function makeNormal(random) {{
  {normal}
  return normal;
}}
const seeds = {json.dumps(SEEDS)};
const out = [];
for (const seed of seeds) {{
  const r = seededRandom(seed);
  const uniforms = [];
  for (let i = 0; i < 64; i++) uniforms.push(String(r()));
  const n = makeNormal(seededRandom(seed));
  const normals = [], f32_std1 = [], f32_std002 = [];
  for (let i = 0; i < 65; i++) {{
    const v = n();
    normals.push(String(v));
    f32_std1.push(String(Math.fround(0 + 1 * v)));
    f32_std002.push(String(Math.fround(0 + 0.02 * v)));
  }}
  out.push({{seed: String(seed), uniforms, normals, f32_std1, f32_std002}});
}}
process.stdout.write(JSON.stringify({{node: process.version, cases: out}}));
"""
    result = subprocess.run(["node", "-e", harness], capture_output=True, text=True, check=True)
    data = json.loads(result.stdout)
    data["source"] = ("src/js/compute/program.ts seededRandom (:1385-1394) and initializedValue's normal() "
                      "(:1396-1413), run under node " + data["node"])
    OUT.write_text(json.dumps(data, indent=1) + "\n")
    print(f"wrote {OUT} ({len(data['cases'])} seeds, node {data['node']})")


if __name__ == "__main__":
    main()
