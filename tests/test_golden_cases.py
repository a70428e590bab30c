"""The reference's own golden cases (tests/golden/cases, written by tests/golden/make_golden.py
from the reference's seeded generator and its "O2" reference recurrence).

Tolerances, written per check:
  * first h snapshot of every sequence == initial_state (or 0): bit-exact;
  * h, v_new, final_state: max |error| <= 1% of the tensor's max |golden|.  O2 keeps the state
    in bf16 between chunks (docs/problem.txt:137-167) where the Triton kernel, this oracle and
    the default numerics of the library keep it in fp32, so h and final differ from the golden by about one bf16 ulp of
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


# ----------------------------------------------------------------------------- O2 ("contest") numerics

def _contest_ok(got, ref):
    """The contest comparison (code/examples/compare_npu_output.py:14-15,54-73): bit-equal, or
    |err| <= 1e-6, or |err| <= 1e-5 |golden|."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    return (got == ref) | (err <= 1e-6) | (err <= 1e-5 * np.abs(ref)) | (np.isnan(got) & np.isnan(ref))


# bit-exact fractions the oracle reaches against the reference's goldens; the misses are
# single bf16 ulps from 1-ulp differences of torch's float32 exp (not correctly rounded)
# that flip a fp16 gate now and then, carried on by the bf16 state
O2_MIN_EXACT = 0.985


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_o2_oracle_matches_reference_golden(case):
    _, a = load_case(case)
    h, v, f = O.fwd_h_o2(a["input_k"], a["input_w"], a["input_u"], a["input_g"], a.get("input_initial_state"),
                         a["input_cu_seqlens"])
    for name, got, ref in (("h", h, a["golden_h"]), ("v", v, a["golden_v"]), ("final", f, a["golden_final_state"])):
        exact = (got == ref).mean()
        assert exact >= O2_MIN_EXACT and _contest_ok(got, ref).mean() >= O2_MIN_EXACT, (case.name, name, exact)
        assert np.abs(got - ref).max() <= 1e-2 * np.abs(ref).max(), (case.name, name)


def test_f16_casts_special_values():
    x = np.array([70000.0, -70000.0, 65519.0, 65520.0, np.inf, -np.inf, np.nan, 1e-8, 3.0e-5, -0.0, 1.0009765625],
                 np.float32)
    sat = O.f16_sat(x).astype(np.float32)
    want = np.array([65504, -65504, 65504, 65504, np.inf, -np.inf, np.nan, 0.0, 2.998e-05, -0.0, 1.0],
                    np.float32)
    assert np.array_equal(np.isnan(sat), np.isnan(want))
    m = ~np.isnan(want)
    np.testing.assert_allclose(sat[m], want[m], rtol=1e-3)
    assert sat[3] == 65504          # 65520 rounds to inf in fp16; the finite input saturates
    assert np.signbit(sat[9])
    n2n = O.f16_nan_to_num(np.array([np.nan, 70000.0, -np.inf, 2.5], np.float32)).astype(np.float32)
    assert n2n[0] == 0 and n2n[1] == np.inf and n2n[2] == -np.inf and n2n[3] == 2.5


def test_contest_numerics_validation():
    import ctypes
    a = _abi.FwdHArgs()
    fake = 1 << 24
    a.k = a.w = a.u = a.h = fake
    T, H, K, V = 128, 2, 128, 128
    a.B, a.T, a.H, a.Hg, a.K, a.V, a.N, a.NT, a.chunk_size = 1, T, H, H, K, V, 1, 2, 64
    a.stride_k[:] = a.stride_w[:] = [T * H * K, H * K, K]
    a.stride_u[:] = [T * H * V, H * V, V]
    a.stride_h[:] = [2 * H * K * V, H * K * V, K * V]
    a.numerics = _abi.CGDR_NUMERICS_CONTEST
    assert _abi.get_plan(a).kernel == 2
    a.K = 256
    a.stride_k[:] = a.stride_w[:] = [T * H * 256, H * 256, 256]
    a.stride_h[:] = [2 * H * 256 * V, H * 256 * V, 256 * V]
    assert _abi.get_plan(a).kernel == 2
    a.numerics = 2
    n = ctypes.c_size_t()
    assert _abi.load().cgdr_fwd_h_workspace_size(ctypes.byref(a), ctypes.byref(n)) == _abi.CGDR_ERR_INVALID
    a.numerics = _abi.CGDR_NUMERICS_CONTEST
    a.in_dtype = _abi.CGDR_F32
    assert _abi.load().cgdr_fwd_h_workspace_size(ctypes.byref(a), ctypes.byref(n)) == _abi.CGDR_ERR_UNSUPPORTED


def _run_contest(dev, a):
    import cgdr_amd
    t = lambda x, dt: torch.from_numpy(np.ascontiguousarray(x)).to(device=dev, dtype=dt)
    h0 = a.get("input_initial_state")
    S, v, f = cgdr_amd.run(t(a["input_k"], torch.bfloat16), t(a["input_w"], torch.bfloat16),
                           t(a["input_u"], torch.bfloat16), t(a["input_g"], torch.float32),
                           None if h0 is None else t(h0, torch.bfloat16),
                           t(a["input_cu_seqlens"], torch.int64), None, numerics="contest")
    torch.cuda.synchronize()
    return [x.float().cpu().numpy() for x in (S, v, f)]


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_contest_kernel_matches_reference_golden(dev, case):
    """numerics="contest" against the reference's own O2 outputs and against the O2 oracle."""
    print(f"[contest] {case.name}", flush=True)
    _, a = load_case(case)
    got = _run_contest(dev, a)
    ref_o = O.fwd_h_o2(a["input_k"], a["input_w"], a["input_u"], a["input_g"], a.get("input_initial_state"),
                       a["input_cu_seqlens"])
    for name, g_, gold, orc in zip(("h", "v", "final"), got, (a["golden_h"], a["golden_v"], a["golden_final_state"]),
                                   ref_o):
        eg, eo = (g_ == gold).mean(), (g_ == orc).mean()
        print(f"  {name}: bit-exact vs golden {eg:.5f}, vs O2 oracle {eo:.5f}; contest tolerance vs golden "
              f"{_contest_ok(g_, gold).mean():.5f}", flush=True)
        assert eg >= O2_MIN_EXACT and _contest_ok(g_, gold).mean() >= O2_MIN_EXACT, (case.name, name)
        assert eo >= O2_MIN_EXACT, (case.name, name)
        assert np.abs(g_ - gold).max() <= 1e-2 * np.abs(gold).max(), (case.name, name)


@pytest.mark.gpu
def test_contest_kernel_saturation(dev):
    """u beyond the fp16 range: saturation to +-65504 and the nan_to_num of an overflowing W S
    follow the oracle; grouped heads, a partial chunk and K = 256."""
    print("[contest] saturation", flush=True)
    rng = np.random.default_rng(5)
    T, HV, HK, D = 150, 2, 1, 256
    k = O.bf16_round((rng.random((1, T, HK, D)) * 2 - 1).astype(np.float32))
    w = O.bf16_round(((rng.random((1, HV, T, D)) * 2 - 1) / D).astype(np.float32))
    u = O.bf16_round(((rng.random((1, HV, T, D)) * 2 - 1) * 1.2e5).astype(np.float32))
    g = (-0.02 * np.tile(np.arange(1, T + 1, dtype=np.float32), (1, HV, 1))).astype(np.float32)
    cu = np.array([0, 100, 150], np.int64)
    for i0, i1 in ((0, 64), (64, 100), (100, 150)):
        g[..., i0:i1] = -0.02 * np.arange(1, i1 - i0 + 1, dtype=np.float32)
    a = dict(input_k=k, input_w=w, input_u=u, input_g=g, input_cu_seqlens=cu)
    got = _run_contest(dev, a)
    ref = O.fwd_h_o2(k, w, u, g, None, cu)
    assert (np.abs(ref[1]) == 65536).any()          # saturated: bf16(65504) = 65536 in v
    for name, x, r in zip(("h", "v", "final"), got, ref):
        same = (x == r) | (np.isnan(x) & np.isnan(r))
        assert same.mean() >= O2_MIN_EXACT, (name, same.mean())


@pytest.mark.gpu
@pytest.mark.parametrize("D", [48, 96, 160, 192, 33, 100])
def test_contest_kernel_padded_head_dims(dev, D):
    """Contest numerics at key dims between the kernels' instantiated 32/64/128/256 (zero-padded
    tiles and state rows on chip): against the O2 oracle, with the generator's distributions
    (generate_golden.py: k, u in [-1, 1), w in [-1, 1)/D, a linear chunk-local gate), grouped
    heads and two sequences, one ending in a partial chunk."""
    print(f"[contest] D={D}", flush=True)
    rng = np.random.default_rng(100 + D)
    T, HV, HK = 200, 4, 2
    k = O.bf16_round((rng.random((1, T, HK, D)) * 2 - 1).astype(np.float32))
    w = O.bf16_round(((rng.random((1, HV, T, D)) * 2 - 1) / D).astype(np.float32))
    u = O.bf16_round((rng.random((1, HV, T, D)) * 2 - 1).astype(np.float32))
    h0 = O.bf16_round((rng.random((2, HV, D, D)) * 2 - 1).astype(np.float32))
    cu = np.array([0, 128, 200], np.int64)
    g = np.zeros((1, HV, T), np.float32)
    for i0, i1 in ((0, 64), (64, 128), (128, 192), (192, 200)):
        g[..., i0:i1] = -0.02 * np.arange(1, i1 - i0 + 1, dtype=np.float32)
    a = dict(input_k=k, input_w=w, input_u=u, input_g=g, input_initial_state=h0, input_cu_seqlens=cu)
    got = _run_contest(dev, a)
    ref = O.fwd_h_o2(k, w, u, g, h0, cu)
    for name, x, r in zip(("h", "v", "final"), got, ref):
        exact = (x == r).mean()
        assert exact >= O2_MIN_EXACT, (D, name, exact)
        assert np.abs(x - r).max() <= 1e-2 * np.abs(r).max(), (D, name)


@pytest.mark.gpu
def test_contest_kernel_subnormal_updates(dev):
    """u of order 1e-5: v16, the gated vd and the state updates K^T vd sit in fp16's subnormal
    range (below 6.1e-5), where the fast pass's mixed fp16/fp32 additions and conversions must
    keep every bit; against the O2 oracle, with a decaying gate, grouped heads and an initial
    state of the same order."""
    print("[contest] subnormal updates", flush=True)
    rng = np.random.default_rng(21)
    T, HV, HK, D = 300, 4, 2, 128
    k = O.bf16_round((rng.random((1, T, HK, D)) * 2 - 1).astype(np.float32))
    w = O.bf16_round(((rng.random((1, HV, T, D)) * 2 - 1) / D).astype(np.float32))
    u = O.bf16_round(((rng.random((1, HV, T, D)) * 2 - 1) * 2e-5).astype(np.float32))
    h0 = O.bf16_round((rng.standard_normal((2, HV, D, D)) * 1e-5).astype(np.float32))
    cu = np.array([0, 180, 300], np.int64)
    g = np.zeros((1, HV, T), np.float32)
    for i0, i1 in ((0, 64), (64, 128), (128, 180), (180, 244), (244, 300)):
        g[..., i0:i1] = -0.02 * np.arange(1, i1 - i0 + 1, dtype=np.float32)
    a = dict(input_k=k, input_w=w, input_u=u, input_g=g, input_initial_state=h0, input_cu_seqlens=cu)
    got = _run_contest(dev, a)
    ref = O.fwd_h_o2(k, w, u, g, h0, cu)
    sub = (np.abs(ref[1]) > 0) & (np.abs(ref[1]) < 6.1e-5)
    assert sub.mean() > 0.5, sub.mean()             # most v_new values are fp16 subnormals
    for name, x, r in zip(("h", "v", "final"), got, ref):
        exact = (x == r).mean()
        assert exact >= O2_MIN_EXACT, (name, exact)
        assert np.abs(x - r).max() <= 1e-2 * np.abs(r).max(), name


@pytest.mark.gpu
def test_contest_kernel_without_v_new_output(dev):
    """Token-major calls, u beyond the fp16 range on one head: that shows first in the staged
    v_new, which the fast pass checks whether or not v_new is an output.  With v_new requested
    the saturated values (bf16(65504) = 65536, where the fast pass alone would leave inf) follow
    the oracle; without it, h and the final state are bit for bit the same."""
    import cgdr_amd
    print("[contest] no v_new output", flush=True)
    rng = np.random.default_rng(9)
    T, HV, HK, D = 150, 2, 1, 128
    k = O.bf16_round((rng.random((1, T, HK, D)) * 2 - 1).astype(np.float32))
    w = O.bf16_round(((rng.random((1, T, HV, D)) * 2 - 1) / D).astype(np.float32))
    u = O.bf16_round((rng.random((1, T, HV, D)) * 2 - 1).astype(np.float32))
    u[0, 70:90, 1] *= 1.2e5                 # head 1: u beyond the fp16 range
    g = np.zeros((1, T, HV), np.float32)
    for i0, i1 in ((0, 64), (64, 128), (128, 150)):
        g[0, i0:i1] = -0.02 * np.arange(1, i1 - i0 + 1, dtype=np.float32)[:, None]
    t = lambda x, dt: torch.from_numpy(np.ascontiguousarray(x)).to(device=dev, dtype=dt)

    def call(save_v):
        out = cgdr_amd.chunk_gated_delta_rule_fwd_h(
            t(k, torch.bfloat16), t(w, torch.bfloat16), t(u, torch.bfloat16), g=t(g, torch.float32),
            output_final_state=True, save_new_value=save_v, final_state_dtype=torch.bfloat16,
            numerics="contest")
        torch.cuda.synchronize()
        return out

    h1, v1, f1 = call(True)
    h0, v0, f0 = call(False)
    assert v0 is None
    hm = lambda x: np.ascontiguousarray(x.transpose(0, 2, 1, 3))   # [1,T,H,D] -> [1,H,T,D]
    ref = O.fwd_h_o2(k, hm(w), hm(u), np.ascontiguousarray(g.transpose(0, 2, 1)), None, None)
    gv = hm(v1.float().cpu().numpy())
    assert (np.abs(gv[0, 1]) == 65536).any() and not np.isinf(gv).any()
    same = (gv == ref[1]) | (np.isnan(gv) & np.isnan(ref[1]))
    assert same.mean() >= O2_MIN_EXACT, same.mean()
    # the snapshots before the saturated tokens reach the state follow the oracle (chunk 2 holds
    # states of ~1e6 built from +-65504 values, where the GEMMs' fp32 summation order shows)
    gh = h1.float().cpu().numpy().transpose(0, 2, 1, 3, 4)          # [1,NT,H,K,V] -> [1,H,NT,K,V]
    assert (gh[:, :, :2] == ref[0][:, :, :2]).mean() >= O2_MIN_EXACT
    assert torch.equal(h0.view(torch.int16), h1.view(torch.int16))
    assert torch.equal(f0.view(torch.int16), f1.view(torch.int16))


@pytest.mark.gpu
def test_contest_kernel_rising_gates_and_large_state(dev):
    """Gates above 1 (g rising inside a chunk) on one head, an initial state beyond the fp16
    range on another, ordinary values on the third: the heads that need the saturating casts
    are recomputed with them, and all three follow the oracle."""
    print("[contest] rising gates, large state", flush=True)
    rng = np.random.default_rng(7)
    T, HV, HK, D = 200, 3, 3, 128
    k = O.bf16_round((rng.standard_normal((1, T, HK, D)) / np.sqrt(D)).astype(np.float32))
    w = O.bf16_round((rng.standard_normal((1, HV, T, D)) / np.sqrt(D)).astype(np.float32))
    u = O.bf16_round(rng.standard_normal((1, HV, T, D)).astype(np.float32))
    g = np.zeros((1, HV, T), np.float32)
    for i0 in range(0, T, 64):
        n = min(64, T - i0)
        g[0, :, i0:i0 + n] = -0.05 * np.arange(1, n + 1, dtype=np.float32)
    g[0, 0, :] *= -0.2                   # head 0: rising g, gates up to e^0.6
    h0 = O.bf16_round((rng.standard_normal((1, HV, D, D)) * 0.1).astype(np.float32))
    h0[0, 1, :4, :4] = 7.0e4             # head 1: state entries above 65504
    cu = np.array([0, T], np.int64)
    a = dict(input_k=k, input_w=w, input_u=u, input_g=g, input_cu_seqlens=cu, input_initial_state=h0)
    got = _run_contest(dev, a)
    ref = O.fwd_h_o2(k, w, u, g, h0, cu)
    for name, x, r in zip(("h", "v", "final"), got, ref):
        same = (x == r) | (np.isnan(x) & np.isnan(r))
        assert same.mean() >= O2_MIN_EXACT, (name, same.mean())


@pytest.mark.gpu
def test_contest_kernel_full_length(dev):
    """Contest numerics over the headline's sequence length, T = 32768 (512 chunks), on four
    heads, with the headline's plan (32-column tiles, helper workgroups, two compute waves per 16
    columns), against the O2 oracle.  The first 64 chunks are held to the golden cases' bit-exact
    share.  Further on, the two bf16 GEMMs of a chunk accumulate in a different order on the MFMAs
    than in the oracle's (or the reference's) CPU GEMM, the resulting 1-ulp differences pass
    through the bf16 state, and the exact share falls slowly (measured on MI355X: h 100 % at chunk
    8, 99.2 % at 64, 95.6 % at 511); the deviation stays bounded: every element within 1 % of the
    tensor's largest magnitude, and at least 95 % of them bit-exact."""
    print("[contest] T=32768 H=4", flush=True)
    inp = O.make_inputs(81, 1, 32768, 4, 128, 128, gate="linear", with_h0=True, profile="golden")
    h0 = O.bf16_round(inp["initial_state"])
    w = np.swapaxes(inp["w"], 1, 2).copy()
    u = np.swapaxes(inp["u"], 1, 2).copy()
    g = np.swapaxes(inp["g"], 1, 2).copy()
    cu = np.array([0, 32768], np.int64)
    a = dict(input_k=inp["k"], input_w=w, input_u=u, input_g=g, input_cu_seqlens=cu, input_initial_state=h0)
    got = _run_contest(dev, a)
    ref = O.fwd_h_o2(inp["k"], w, u, g, h0, cu)
    early = (got[0][0, :, :64] == ref[0][0, :, :64]).mean()
    print(f"  h, first 64 chunks: bit-exact {early:.5f}", flush=True)
    assert early >= O2_MIN_EXACT, early
    assert (got[1][0, :, :4096] == ref[1][0, :, :4096]).mean() >= O2_MIN_EXACT
    for name, x, r in zip(("h", "v", "final"), got, ref):
        same = (x == r).mean()
        err = np.abs(x - r).max() / np.abs(r).max()
        print(f"  {name}: bit-exact {same:.5f}, max |err| / max |ref| {err:.3e}", flush=True)
        assert np.isfinite(x).all(), name
        assert same >= 0.95, (name, same)
        assert err <= 0.01, (name, err)


@pytest.mark.gpu
@pytest.mark.parametrize("case", [c for c in CASES if c.name in ("long_1024_single", "grouped_heads_packed")],
                         ids=lambda c: c.name)
def test_runner_contest_mode(dev, case, tmp_path):
    print(f"[runner contest] {case.name}", flush=True)
    r = _runner(case, "--out", tmp_path, "--check", "--contest")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "contest_tolerance" in r.stdout and "Case passed" in r.stdout
