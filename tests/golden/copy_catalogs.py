"""Copies the reference's quantized parity catalogs (case lists: ids, shapes,
bits, group sizes; no values) and its decode-step op catalog (ids, ops,
dtypes, shapes, index shapes and axes) into tests/golden/ as data fixtures.

Run in the build container, where the reference tree is mounted:
    python tests/golden/copy_catalogs.py
Sources: test/parity/catalogs/metal-quantized-grid-128.json and
test/parity/catalogs/metal-quantized-views-128.json and
test/parity/catalogs/cuda-apertus-decode-ops.json. Values are produced at
test time by the deterministic fixture formulas of
test/parity/fixtures/quantized_fixture.py:4-18 and
test/parity/reference/probe-capabilities.py:111-125,170-176.
"""
import json
import pathlib

REFERENCE = pathlib.Path("/root/reference/test/parity/catalogs")
HERE = pathlib.Path(__file__).resolve().parent

for name in ("metal-quantized-grid-128.json", "metal-quantized-views-128.json"):
    data = json.loads((REFERENCE / name).read_text())
    cases = [{k: case[k] for k in ("id", "dtype", "shape", "bits", "group_size")} for case in data["cases"]]
    (HERE / name).write_text(json.dumps({"source": f"test/parity/catalogs/{name}", "cases": cases}, indent=1) + "\n")
    print(name, len(cases))

name = "cuda-apertus-decode-ops.json"
data = json.loads((REFERENCE / name).read_text())
keys = ("id", "op", "dtype", "shape", "index_shape", "index_axis")
cases = [{k: case[k] for k in keys if k in case} for case in data["cases"]]
(HERE / name).write_text(json.dumps({"source": f"test/parity/catalogs/{name}", "cases": cases}, indent=1) + "\n")
print(name, len(cases))
