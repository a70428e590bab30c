"""The reference's own golden cases (tests/golden/cases, written by tests/golden/make_golden.py
from the reference's seeded generator and its "O2" reference recurrence).

Tolerances, written per check:
  * first h snapshot of every sequence == initial_state (or 0): bit-exact;
  * h, v_new, final_state: max |error| <= 1% of the tensor's max |golden|.  O2 keeps the state
    in bf16 between chunks (docs/problem.txt:137-167) where the Triton kernel, this oracle and
    this build keep it in fp32, so h and final differ from the golden by about one bf16 ulp of
    the state; v_new additionally within rtol=2e-2, atol=2e-3 for all but 0.1% of elements.
"""

import hashlib
import json
import os
import shutil
import subprocess

import numpy as np
import pytest
import torch

from cgdr_amd import _abi
from golden_io import case_dirs, head_major_outputs, load_case, token_major_inputs
from oracle import cgdr_oracle as O

CASES = case_dirs()
IDS = [c.name for c in CASES]


def _check_against_golden(name, arrays, h, v, f):
    gh, gv, gf = arrays["golden_h"], arrays["golden_v"], arrays["golden_final_state"]
    h = np.asarray(h, np.float64); v = np.asarray(v, np.float64); f = np.asarray(f, np.float64)
    # first snapshot of each sequence is the initial state (bf16) or zero
    offs = O.prepare_chunk_offsets(arrays["input_cu_seqlens"])
    h0 = arrays.get("input_initial_state")
    for n in range(len(offs) - 1):
        want = np.zeros_like(gh[0, :, offs[n]]) if h0 is None else h0[n]
        assert np.array_equal(gh[0, :, offs[n]], want), (name, "golden first snapshot")
        assert np.array_equal(h[0, :, offs[n]], want), (name, "first snapshot", n)
    for out, got, ref in (("h", h, gh), ("v_new", v, gv), ("final_state", f, gf)):
        err = np.abs(got - ref)
        scale = max(np.abs(ref).max(), 1e-30)
        assert err.max() <= 1e-2 * scale, f"{name} {out}: max err {err.max():.3e} > 1% of {scale:.3e}"
    bad = np.abs(v - gv) > 2e-3 + 2e-2 * np.abs(gv)
    assert bad.mean() <= 1e-3, f"{name} v_new: {bad.sum()}/{bad.size} outside rtol=2e-2, atol=2e-3"


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_manifest_and_files(case):
    manifest, arrays = load_case(case)          # sizes and SHA-256 verified on load
    spec = manifest["case"]
    T, HV, HK, D = manifest["total_tokens"], spec["hv"], spec["hk"], spec["dim"]
    assert arrays["input_k"].shape == (1, T, HK, D)
    assert arrays["golden_h"].shape == (1, HV, manifest["total_chunks"], D, D)
    assert list(arrays["input_cu_seqlens"]) == list(np.concatenate([[0], np.cumsum(spec["seq_lens"])]))
    assert np.array_equal(arrays["input_chunk_indices"], O.prepare_chunk_indices(arrays["input_cu_seqlens"]))


@pytest.mark.parametrize("rounding", [None, "bf16"])
@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_oracle_matches_reference_golden(case, rounding):
    """The oracle (exact, and the bf16 rounding model) against the reference's own outputs."""
    _, arrays = load_case(case)
    h, v, f = O.fwd_h(**token_major_inputs(arrays), rounding=rounding)
    _check_against_golden(case.name, arrays, *head_major_outputs(h, v, f))


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_kernel_matches_reference_golden(dev, case):
    """cgdr_amd.run (the contest's head-major signature) on the golden inputs."""
    import cgdr_amd
    print(f"[golden] {case.name}", flush=True)
    _, arrays = load_case(case)
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(device=dev, dtype=dt)
    h0 = arrays.get("input_initial_state")
    S, v, f = cgdr_amd.run(t(arrays["input_k"], torch.bfloat16), t(arrays["input_w"], torch.bfloat16),
                           t(arrays["input_u"], torch.bfloat16), t(arrays["input_g"], torch.float32),
                           None if h0 is None else t(h0, torch.bfloat16),
                           t(arrays["input_cu_seqlens"], torch.int64), t(arrays["input_chunk_indices"], torch.int64))
    torch.cuda.synchronize()
    got = [x.float().cpu().numpy() for x in (S, v, f)]
    _check_against_golden(case.name, arrays, *got)
    # and against the oracle's model of the same rounding points: within rtol=2e-2, atol=2e-3
    # for all but 0.1% of elements and within 1% of the tensor's scale everywhere.  Over many
    # chunks a one-ulp difference in a bf16 operand (fp32 sums in another order) carries into
    # the state, and a stored bf16 snapshot near a power of two then differs by one ulp of it.
    ref = head_major_outputs(*O.fwd_h(**token_major_inputs(arrays), rounding="bf16"))
    for out, a, b in zip(("h", "v_new", "final_state"), got, ref):
        if out == "final_state":
            b = O.bf16_round(b)          # run() returns the final state in u's dtype
        err = np.abs(a - b)
        scale = max(np.abs(b).max(), 1e-30)
        bad = err > 2e-3 + 2e-2 * np.abs(b)
        print(f"  {out}: max err {err.max():.3e} = {err.max() / scale:.2e} of scale; "
              f"{bad.sum()}/{bad.size} outside rtol=2e-2, atol=2e-3", flush=True)
        assert bad.mean() <= 1e-3, f"{case.name} {out}: {bad.sum()}/{bad.size} outside rtol=2e-2, atol=2e-3 of the model"
        assert err.max() <= 1e-2 * scale, f"{case.name} {out}: max err {err.max():.3e} > 1% of {scale:.3e}"


# ----------------------------------------------------------------- the C++ golden-case runner
RUNNER = os.path.join(os.path.dirname(_abi.LIB_PATH), "cgdr_golden_runner")


def _runner(*args, timeout=120):
    assert os.path.exists(RUNNER), f"{RUNNER} not built (cgdr_amd.build.build_all)"
    return subprocess.run([RUNNER, *map(str, args)], capture_output=True, text=True, timeout=timeout)


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_runner_dry_run_verifies_case(case):
    """Manifest parse, SHA-256 of every file, chunk_indices and host-side planning; no device call."""
    r = _runner(case, "--dry-run")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "Dry run: inputs verified" in r.stdout


def test_runner_rejects_tampered_files(tmp_path):
    src = CASES[0]
    for victim, expect in (("input_u.bin", "SHA-256"), ("input_chunk_indices.bin", "chunk_indices")):
        dst = tmp_path / victim.split(".")[0]
        shutil.copytree(src, dst)
        raw = bytearray((dst / victim).read_bytes())
        if victim == "input_u.bin":
            raw[7] ^= 0x40
        else:                      # a consistent manifest but a wrong chunk row
            raw[8] ^= 0x01
            m = json.loads((dst / "manifest.json").read_text())
            m["tensors"]["input_chunk_indices"]["sha256"] = hashlib.sha256(bytes(raw)).hexdigest()
            (dst / "manifest.json").write_text(json.dumps(m))
        (dst / victim).write_bytes(bytes(raw))
        r = _runner(dst, "--dry-run")
        assert r.returncode == 2 and expect in r.stderr, (victim, r.stdout, r.stderr)
    r = _runner(tmp_path / "missing", "--dry-run")
    assert r.returncode == 2 and "cannot open" in r.stderr
    assert _runner().returncode == 2                      # usage


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_runner_replays_case(dev, case, tmp_path):
    """The runner's outputs pass its own golden check and equal cgdr_amd.run's bit for bit."""
    import cgdr_amd
    print(f"[runner] {case.name}", flush=True)
    r = _runner(case, "--out", tmp_path, "--check")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "Case passed" in r.stdout
    manifest, arrays = load_case(case)
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(device=dev, dtype=dt)
    h0 = arrays.get("input_initial_state")
    outs = cgdr_amd.run(t(arrays["input_k"], torch.bfloat16), t(arrays["input_w"], torch.bfloat16),
                        t(arrays["input_u"], torch.bfloat16), t(arrays["input_g"], torch.float32),
                        None if h0 is None else t(h0, torch.bfloat16),
                        t(arrays["input_cu_seqlens"], torch.int64), t(arrays["input_chunk_indices"], torch.int64))
    torch.cuda.synchronize()
    for name, x in zip(("h", "v", "final_state"), outs):
        got = np.fromfile(tmp_path / f"actual_{name}.bin", dtype=np.uint16)
        want = x.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).ravel()
        assert got.shape == want.shape and np.array_equal(got, want), f"{case.name} {name}"
