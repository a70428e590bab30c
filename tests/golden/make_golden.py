"""Write a subset of the reference's own seeded golden cases as test fixtures.

Runs only in the build container, where the reference is mounted read-only: it imports the
reference's case generator (code/tests/golden/generate_golden.py) and calls its
``generate_case`` for the cases below.  The cases come from its CASES table
(generate_golden.py:37-257): inputs from its seeded ``build_case`` (:461-506) and outputs
from its ``run_reference`` (:350-436).  That function is the contest's "O2" recurrence
(fp16 saturation, bf16 state; docs/problem.txt:81-185), which no check of this repository
pins otherwise.

The files it writes are the reference's own on-disk format (generate_golden.py:582-658):
raw little-endian ``input_*.bin`` / ``golden_*.bin`` (bf16 as 16-bit storage) and a
``manifest.json`` with shapes, dtypes, byte counts and SHA-256 digests.  Only these data
files are committed; nothing under tests/ imports the reference.

    python tests/golden/make_golden.py [--out tests/golden/cases]
"""

from __future__ import annotations

import argparse
import importlib.util
import pathlib
import sys

REFERENCE_GENERATOR = pathlib.Path(
    "/root/reference/ChunkGatedDeltaRuleFwdH_problem_290_template/code/tests/golden/generate_golden.py")

# Small cases (about 4.5 MB together): partial, boundary and single-token chunks, packed
# varlen sequences, grouped heads, K = V in {32, 128, 256}, with and without initial state.
SELECTED = (
    "smoke_single_partial",
    "boundary_63_64_65",
    "boundary_127_128_129",
    "grouped_heads_packed",
    "two_chunk_single",
    "two_v_tiles",
    "four_v_tiles",
    "without_initial_state",
    "single_token",
    "heads_equal_hk_hv",
    "no_state_long",
    "long_1024_single",
)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", type=pathlib.Path, default=pathlib.Path(__file__).parent / "cases")
    args = ap.parse_args()
    spec = importlib.util.spec_from_file_location("reference_generate_golden", REFERENCE_GENERATOR)
    gen = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = gen   # its dataclasses resolve their module by name
    spec.loader.exec_module(gen)
    by_name = {case.name: case for case in gen.CASES}
    for name in SELECTED:
        summary = gen.generate_case(by_name[name], args.out)
        print(name, summary["total_tokens"], summary["total_chunks"])


if __name__ == "__main__":
    main()
