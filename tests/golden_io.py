"""Reader for the reference's golden-case directories (tests/golden/cases/<name>/).

Format (the reference's own, code/tests/golden/generate_golden.py:582-658): raw C-order
little-endian ``input_*.bin`` / ``golden_*.bin`` (bf16 stored as its 16-bit pattern, fp32,
int64) and a ``manifest.json`` giving each file's shape, dtype, element and byte counts and
SHA-256.  Layouts are the contest's head-major ones: k [1,T,HK,K], w [1,HV,T,K],
u [1,HV,T,V], g [1,HV,T], initial_state [N,HV,K,V] -> h [1,HV,NT,K,V], v [1,HV,T,V],
final_state [N,HV,K,V] (bf16).
"""

from __future__ import annotations

import hashlib
import json
import pathlib

import numpy as np

CASES_DIR = pathlib.Path(__file__).resolve().parent / "golden" / "cases"

_DTYPES = {"bfloat16": np.uint16, "float32": np.float32, "int64": np.int64}


def case_dirs() -> list[pathlib.Path]:
    return sorted(p for p in CASES_DIR.iterdir() if (p / "manifest.json").exists())


def load_case(case_dir: pathlib.Path, verify: bool = True) -> tuple[dict, dict[str, np.ndarray]]:
    """(manifest, arrays): bf16 tensors come back as float32 holding the exact bf16 values."""
    manifest = json.loads((case_dir / "manifest.json").read_text())
    arrays = {}
    for key, meta in manifest["tensors"].items():
        raw = (case_dir / meta["file"]).read_bytes()
        if verify:
            assert len(raw) == meta["bytes"], (case_dir.name, key)
            assert hashlib.sha256(raw).hexdigest() == meta["sha256"], (case_dir.name, key)
        a = np.frombuffer(raw, dtype=_DTYPES[meta["dtype"]])
        if meta["dtype"] == "bfloat16":
            a = (a.astype(np.uint32) << 16).view(np.float32)
        a = a.reshape(meta["shape"]).copy()
        assert a.size == meta["elements"], (case_dir.name, key)
        arrays[key] = a
    return manifest, arrays


def token_major_inputs(arrays: dict[str, np.ndarray]) -> dict:
    """Oracle (token-major) keyword inputs of a case."""
    return dict(
        k=arrays["input_k"],
        w=arrays["input_w"].transpose(0, 2, 1, 3),
        u=arrays["input_u"].transpose(0, 2, 1, 3),
        g=arrays["input_g"].transpose(0, 2, 1),
        initial_state=arrays.get("input_initial_state"),
        cu_seqlens=arrays["input_cu_seqlens"],
    )


def head_major_outputs(h, v, f):
    """Token-major (h [B,NT,H,K,V], v [B,T,H,V], final) -> the golden head-major layouts."""
    return h.transpose(0, 2, 1, 3, 4), v.transpose(0, 2, 1, 3), f
