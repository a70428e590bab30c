"""Pins for the CPU oracle (oracle/cgdr_oracle.py), all on the CPU.

The chunked recurrence is checked against things that do not share its code:
  * the token-by-token Gated DeltaNet recurrence fed through the WY producer
    (fixes operand order, signs, the gate placement exp(g_last - g), state decay,
    partial chunks, varlen boundaries, GQA head mapping and h0 handling);
  * closed forms (w = 0, k = 0, g = None), exact linearity and decomposition identities;
  * the reference's worked varlen example for chunk metadata
    (docs/problem_understanding.md:173-190: cu_seqlens [0,61,64] -> indices [[0,0],[1,0]],
    offsets [0,1,2]);
  * torch's float->bfloat16 conversion for the rounding helper.
"""

import glob
import os

import numpy as np
import pytest
import torch

import o1_probe
from oracle import cgdr_oracle as O


def _wy_case(seed, B, T, H, K, V, Hg=None, cu=None, with_h0=True, decay_shift=4.0):
    rng = np.random.default_rng(seed)
    Hg = H if Hg is None else Hg
    kg = rng.standard_normal((B, T, Hg, K))
    kg /= np.linalg.norm(kg, axis=-1, keepdims=True)
    kfull = np.repeat(kg, H // Hg, axis=2)
    v = rng.standard_normal((B, T, H, V))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H))))
    a = -np.logaddexp(0.0, -(rng.standard_normal((B, T, H)) + decay_shift))   # mild log-decay
    N = B if cu is None else len(cu) - 1
    h0 = rng.standard_normal((N, H, K, V)) if with_h0 else None
    return kg, kfull, v, beta, a, h0


@pytest.mark.parametrize("case", [
    dict(B=2, T=150, H=2, K=8, V=6),                    # fixed length, partial last chunk
    dict(B=1, T=200, H=4, K=8, V=4, Hg=2),               # GQA head mapping
    dict(B=1, T=0, H=2, K=6, V=5, cu=[0, 1, 64, 129, 200]),  # varlen, chunk boundaries
])
def test_chunked_equals_tokenwise_recurrence(case):
    cu = case.get("cu")
    if cu is not None:
        case = dict(case, T=cu[-1])
        cu = np.asarray(cu, np.int64)
    kg, kfull, v, beta, a, h0 = _wy_case(11, case["B"], case["T"], case["H"], case["K"], case["V"],
                                         case.get("Hg"), cu)
    w, u, g = O.wy_prepare(kfull, v, beta, a, cu_seqlens=cu)
    h, vn, fin = O.fwd_h(kg, w, u, g, h0, cu_seqlens=cu, compute_dtype=np.float64)
    st, ft = O.gated_delta_rule_tokenwise(kfull, v, beta, a, h0, cu_seqlens=cu)
    scale = max(1.0, np.abs(ft).max())
    assert np.abs(h - st).max() <= 1e-10 * scale
    assert np.abs(fin - ft).max() <= 1e-10 * scale
    # sanity: the decay is mild enough that states really propagate across chunks
    assert np.abs(st[:, 1:]).max() > 0.1


def test_tokenwise_pin_catches_plausible_mistakes():
    """A transposed gate, a dropped state decay or a sign flip in U - W S must all break the pin."""
    kg, kfull, v, beta, a, h0 = _wy_case(3, 1, 130, 2, 6, 5)
    w, u, g = O.wy_prepare(kfull, v, beta, a)
    _, ft = O.gated_delta_rule_tokenwise(kfull, v, beta, a, h0)
    good = O.fwd_h(kg, w, u, g, h0, compute_dtype=np.float64)[2]
    bad_gate = O.fwd_h(kg, w, u, -g, h0, compute_dtype=np.float64)[2]          # exp(g - g_last)
    bad_sign = O.fwd_h(kg, -w, u, g, h0, compute_dtype=np.float64)[2]          # U + W S
    assert np.abs(good - ft).max() < 1e-9
    assert np.abs(bad_gate - ft).max() > 1e-3
    assert np.abs(bad_sign - ft).max() > 1e-3


def test_w_zero_gives_u_and_closed_form_state():
    inp = O.make_inputs(1, 1, 130, 2, 16, 8, dtype="f32", gate="linear")
    inp["w"] = np.zeros_like(inp["w"])
    h, vn, fin = O.fwd_h(**inp)
    assert np.array_equal(vn, inp["u"])
    # S_{c+1} = e^{g_last} S_c + K_c^T (gamma * U_c), computed by hand for head 0
    S = inp["initial_state"][0, 0].astype(np.float64)
    for c, t0 in enumerate(range(0, 130, 64)):
        t1 = min(t0 + 64, 130)
        assert np.allclose(h[0, c, 0], S, rtol=1e-5, atol=1e-6)
        gc = inp["g"][0, t0:t1, 0].astype(np.float64)
        gam = np.exp(gc[-1] - gc)
        S = np.exp(gc[-1]) * S + inp["k"][0, t0:t1, 0].astype(np.float64).T @ (gam[:, None] * inp["u"][0, t0:t1, 0])
    assert np.allclose(fin[0, 0], S, rtol=1e-5, atol=1e-5)


def test_k_zero_state_only_decays():
    inp = O.make_inputs(2, 1, 200, 2, 8, 8, dtype="f32", gate="logsigmoid", gate_shift=3.0)
    inp["k"] = np.zeros_like(inp["k"])
    h, _, fin = O.fwd_h(**inp, compute_dtype=np.float64)
    decay = np.ones(2)
    for c, t0 in enumerate(range(0, 200, 64)):
        assert np.allclose(h[0, c], inp["initial_state"][0] * decay[:, None, None], rtol=1e-12)
        t1 = min(t0 + 64, 200)
        decay = decay * np.exp(inp["g"][0, t1 - 1].astype(np.float64))
    assert np.allclose(fin[0], inp["initial_state"][0] * decay[:, None, None], rtol=1e-12)


def test_no_gate_equals_zero_gate():
    inp = O.make_inputs(3, 1, 150, 2, 16, 16, dtype="f32", gate=None)
    a = O.fwd_h(**inp)
    b = O.fwd_h(**dict(inp, g=np.zeros((1, 150, 2), np.float32)))
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


@pytest.mark.parametrize("rounding", [None, "bf16"])
def test_linearity_is_exact(rounding):
    inp = O.make_inputs(4, 1, 140, 2, 32, 16, dtype="bf16", gate="linear")
    a = O.fwd_h(**inp, rounding=rounding)
    inp2 = dict(inp, u=inp["u"] * 2, initial_state=inp["initial_state"] * 2)
    b = O.fwd_h(**inp2, rounding=rounding)
    for x, y in zip(a, b):
        assert np.array_equal(2 * x, y)


def test_varlen_equals_separate_sequences():
    cu = np.array([0, 5, 69, 133, 300], np.int64)
    inp = O.make_inputs(5, 1, 300, 2, 16, 16, dtype="bf16", gate="linear", cu_seqlens=cu)
    h, vn, fin = O.fwd_h(**inp, rounding="bf16")
    offs = O.prepare_chunk_offsets(cu)
    for n in range(4):
        b, e = cu[n], cu[n + 1]
        sub = dict(k=inp["k"][:, b:e], w=inp["w"][:, b:e], u=inp["u"][:, b:e], g=inp["g"][:, b:e],
                   initial_state=inp["initial_state"][n:n + 1])
        hs, vs, fs = O.fwd_h(**sub, rounding="bf16")
        assert np.array_equal(h[0, offs[n]:offs[n + 1]], hs[0])
        assert np.array_equal(vn[0, b:e], vs[0])
        assert np.array_equal(fin[n], fs[0])
        assert np.array_equal(h[0, offs[n]], bf16_or_same(inp["initial_state"][n]))


def bf16_or_same(x):
    return O.bf16_round(x)


def test_gqa_equals_repeated_keys():
    inp = O.make_inputs(6, 1, 130, 4, 16, 16, Hg=2, dtype="bf16", gate="linear")
    a = O.fwd_h(**inp, rounding="bf16")
    b = O.fwd_h(**dict(inp, k=np.repeat(inp["k"], 2, axis=2)), rounding="bf16")
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_first_snapshot_is_initial_state():
    inp = O.make_inputs(7, 2, 100, 2, 16, 16, dtype="f32", gate="linear")
    h, _, _ = O.fwd_h(**inp)
    assert np.array_equal(h[:, 0], inp["initial_state"])


@pytest.mark.parametrize("gate,shift", [("linear", 0.0), ("logsigmoid", 0.0), ("logsigmoid", 3.0)])
def test_bf16_rounding_model_close_to_exact(gate, shift):
    """The bf16-operand rounding model stays within 1% of the exact recurrence's scale.

    Elementwise rtol=2e-2/atol=2e-3 does NOT hold for it: near-zero elements of
    U - W bf16(S) carry absolute errors of a few 1e-3 from the bf16 rounding of S
    (measured worst ratio to the elementwise bound: ~8 for the mild linear gate at T=512).
    """
    inp = O.make_inputs(8, 1, 512, 4, 64, 64, dtype="bf16", gate=gate, gate_shift=shift)
    e = O.fwd_h(**inp, compute_dtype=np.float64)
    r = O.fwd_h(**inp, rounding="bf16")
    for x, y in zip(e, r):
        assert np.abs(x - y).max() <= 1e-2 * np.abs(x).max()
        assert np.linalg.norm(x - y) <= 5e-3 * np.linalg.norm(x)


def test_safe_exp():
    x = np.array([-np.inf, -100.0, -1.0, 0.0, 1e-30, 5.0], np.float32)
    got = O.safe_exp(x)
    assert got[0] == 0 and got[3] == 1 and got[4] == 0 and got[5] == 0
    assert np.isclose(got[2], np.exp(-1.0))


def test_chunk_metadata_worked_example():
    cu = np.array([0, 61, 64], np.int64)
    assert O.prepare_chunk_indices(cu).tolist() == [[0, 0], [1, 0]]
    assert O.prepare_chunk_offsets(cu).tolist() == [0, 1, 2]
    cu = np.array([0, 63, 127, 192], np.int64)  # 63, 64, 65 tokens
    assert O.prepare_chunk_offsets(cu).tolist() == [0, 1, 2, 4]
    assert O.prepare_chunk_indices(cu).tolist() == [[0, 0], [1, 0], [2, 0], [2, 1]]


def test_head_major_round_trip():
    inp = O.make_inputs(9, 1, 100, 2, 16, 16, dtype="f32", gate="linear")
    w_hm, u_hm, g_hm = np.swapaxes(inp["w"], 1, 2), np.swapaxes(inp["u"], 1, 2), np.swapaxes(inp["g"], 1, 2)
    w_t, u_t, g_t = O.to_token_major(w_hm, u_hm, g_hm)
    assert np.array_equal(w_t, inp["w"]) and np.array_equal(u_t, inp["u"]) and np.array_equal(g_t, inp["g"])


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(50000) * 10.0 ** rng.uniform(-30, 30, 50000)).astype(np.float32)
    ties = ((np.arange(2000, dtype=np.uint32) << 16) | 0x8000).view(np.float32)
    x = np.concatenate([x, ties, -ties, np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 3.4e38], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    got = O.bf16_round(x)
    same = (ref.view(np.uint32) == got.view(np.uint32)) | (np.isnan(ref) & np.isnan(got))
    assert same.all()


def test_gate_generators():
    rng = np.random.default_rng(0)
    cu = np.array([0, 70, 200], np.int64)
    for kind in ("logsigmoid", "linear"):
        g = O.make_gate(rng, 1, 200, 3, kind, cu)
        for b0, b1 in ((0, 64), (64, 70), (70, 134), (134, 198), (198, 200)):
            seg = g[0, b0:b1]
            assert np.all(seg < 0)
            assert np.all(np.diff(seg, axis=0) <= 0)


def test_varlen_lengths_avoid_chunk_multiples():
    cu = O.varlen_cu_seqlens(0, 16, 64, 8192)
    lens = np.diff(cu)
    assert len(lens) == 16 and np.all(lens % 64 != 0) and lens.min() >= 64 and lens.max() <= 8192


# ---------------------------------------------------------------- O1 rounding points

O1_MISTAKES = ("mm1_fp32_state", "gate_rounded_v_new", "mm2_fp32_operand", "bf16_state")


@pytest.mark.parametrize("K,V,n_chunks,H", [(32, 32, 3, 2), (128, 128, 4, 2), (64, 48, 3, 1)])
def test_o1_rounding_points_closed_form(K, V, n_chunks, H):
    """The bf16 model equals, bit for bit, the closed form of the Triton kernel's four rounding
    rules on one-hot W and K rows (tests/o1_probe.py; docs/problem.txt:356-405): bf16(S) into
    W @ S, v_new from the fp32 Vn before gating, bf16(Vn gamma) into K^T @ ., fp32 state."""
    inp = o1_probe.probe_inputs(K, V, n_chunks, H=H, seed=1)
    assert o1_probe.gamma_margin_ok(inp)
    for name, want, got in zip(("h", "v_new", "final"), o1_probe.closed_form(inp), O.fwd_h(**inp, rounding="bf16")):
        assert np.array_equal(want, got), name


@pytest.mark.parametrize("mistake", O1_MISTAKES)
def test_o1_closed_form_catches_moved_rounding_points(mistake):
    """Each plausible misplacement of one rounding point breaks the closed form."""
    inp = o1_probe.probe_inputs(32, 32, 3, H=2, seed=1)
    want = o1_probe.closed_form(inp)
    got = O.fwd_h(**inp, rounding="bf16", mistake=mistake)
    assert any(not np.array_equal(a, b) for a, b in zip(want, got)), mistake


def test_o1_probe_distinguishes_each_rule():
    """The probe's values really exercise the rules: bf16 cannot hold the fp32 state rows,
    the MM1 operand rounding changes v_new, and gamma differs from 1 on the gated tokens."""
    inp = o1_probe.probe_inputs(32, 32, 2, H=1, seed=1)
    h0 = inp["initial_state"]
    assert (O.bf16_round(h0[0, 0, :16]) != h0[0, 0, :16]).all()
    g = inp["g"][0, :16, 0]
    assert (g > 0).all() and (inp["g"][0, 16:64, 0] == 0).all()
    h, v_new, final = o1_probe.closed_form(inp)
    assert np.array_equal(final[0, 0, :16], h0[0, 0, :16])          # fp32 state carried
    u0 = inp["u"][0, 16:32, 0]
    assert not np.array_equal(v_new[0, 16:32, 0], O.bf16_round(u0 - h0[0, 0, :16]))


# ----------------------------------------------------------------------------- bf16-state benchmark

BF16_STATE_CASES = sorted(os.path.basename(f)[:-4] for f in glob.glob(os.path.join(
    os.path.dirname(__file__), "golden", "bf16_state", "*.npz")))


def _bf16_state_case(name):
    a = np.load(os.path.join(os.path.dirname(__file__), "golden", "bf16_state", name + ".npz"))
    cu = a["cu_seqlens"] if len(a["cu_seqlens"]) > 2 else None
    return a, cu


@pytest.mark.parametrize("name", BF16_STATE_CASES)
def test_bf16_state_oracle_matches_reference_vectors(name):
    """fwd_h_bf16_state against the vectors the reference's own stage1_opt/stage2_opt wrote
    (tests/golden/make_bf16_state_golden.py): v_new bit for bit; the final state bit for bit
    but for a float32 accumulation-order residue of at most one bf16 ulp (1 of 1,024
    elements on the 10-chunk case)."""
    a, cu = _bf16_state_case(name)
    _, v, fin = O.fwd_h_bf16_state(a["k"], a["w"], a["u"], a["g"], a["h0"], cu_seqlens=cu)
    assert np.array_equal(v, a["v_new"]), name
    assert (fin == a["final"]).mean() >= 0.998, name
    ulp = np.abs(a["final"]) * 2.0 ** -7 + 1e-30
    assert (np.abs(fin - a["final"]) <= ulp).all(), name


@pytest.mark.parametrize("name", BF16_STATE_CASES)
def test_bf16_state_vectors_tell_the_rounding_models_apart(name):
    """The same vectors reject the other rounding models: the Triton kernel's (fp32 state,
    gate on v_new) and the exact recurrence both miss v_new or the final state, so the
    fixtures pin where the benchmark rounds, not only its scale."""
    a, cu = _bf16_state_case(name)
    for rounding in ("bf16", None):
        _, v, fin = O.fwd_h(a["k"], a["w"], a["u"], a["g"], a["h0"], cu_seqlens=cu, rounding=rounding)
        v = O.bf16_round(v)
        fin = O.bf16_round(fin)
        assert (v != a["v_new"]).any() or (fin != a["final"]).mean() > 0.01, (name, rounding)


def test_accuracy_gate_restatement():
    """tests/accuracy_gate.py follows compare.py's rules (compare.py:32-35,55-196): equal
    outputs pass; a device whose max relative error is 6x the benchmark's fails on that ratio
    alone; errors below 2^-7 pass whatever the ratio; the benchmark's errors are floored at
    2^-8; a small golden value the device misses counts in smra."""
    import accuracy_gate as G
    rng = np.random.default_rng(0)
    g = rng.uniform(0.5, 1.0, 4096).astype(np.float32)
    assert G.cross_check(g, g, g)["passed"]
    bench = g.copy()
    bench[0] += 0.05 * (g[0] + 1e-3)              # benchmark max_re 0.05
    npu = g.copy()
    npu[1] += 0.30 * (g[1] + 1e-3)                # device max_re 0.30 = 6x, mean and rmse tiny
    r = G.cross_check(npu, g, bench)
    assert not r["passed"] and r["ratios"]["max_re"] == pytest.approx(6.0, rel=1e-3)
    assert r["ratios"]["avg_re"] < 1.5 and r["ratios"]["rmse"] < 1.5
    npu = g.copy()
    npu[1] += 0.006 * (g[1] + 1e-3)               # below 2^-7: passes although 6x a tiny bench
    tiny = g.copy()
    tiny[0] += 0.001 * (g[0] + 1e-3)
    assert G.cross_check(npu, g, tiny)["passed"]
    # a benchmark error below 2^-8 counts as 2^-8, so a device max_re of 4 * 2^-8 passes;
    # against an exact benchmark any device error is an infinite ratio
    npu = g.copy()
    npu[2] += 4 * 2.0 ** -8 * (g[2] + 1e-3)
    r = G.cross_check(npu, g, tiny)
    assert r["ratios"]["max_re"] == pytest.approx(4.0, rel=1e-3) and r["passed"]
    r = G.cross_check(npu, g, g)
    assert r["ratios"]["max_re"] == float("inf") and not r["passed"]
    # small golden values (|g| < 2^-10): 3 of 4 missed
    gs = np.full(4, 2.0 ** -12, np.float32)
    assert G.errors(gs + np.array([0, 1e-5, 1e-5, 1e-5], np.float32), gs)["smra"] == pytest.approx(0.75)
