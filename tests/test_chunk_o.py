"""Chunk output o, the consumer of FwdH's h and v_new.

CPU (oracle pins):
  * wy_prepare -> fwd_h -> chunk_o (float64) equals the token-by-token Gated DeltaNet output
    ``o_t = scale S_t^T q_t`` to 1e-10 relative (fixed length, varlen, grouped heads); a
    planted omission of the intra-chunk term misses it by orders of magnitude;
  * closed forms: k = 0 gives ``scale e^{g_i} q_i . h_c``; h = 0 and one-token chunks give
    ``scale (q_i . k_i) v_i``; g = None equals g = 0;
  * the bf16 rounding model stays within 1% of the tensor's scale of the exact output.
CPU (host side): validation of cgdr_chunk_o_args and the V-tile plan.
GPU (tolerances written per check): the HIP kernel vs the bf16 rounding model elementwise
  rtol=2e-2, atol=2e-3; vs the exact output within 1% of the tensor's scale; device-derived
  chunk mapping and the given chunk_indices bit-identical; V-tile invariance and head-major
  strides bit-exact; fwd_h -> chunk_o on the GPU against the tokenwise recurrence.
"""

import ctypes

import numpy as np
import pytest
import torch

from cgdr_amd import _abi
from oracle import cgdr_oracle as O

BF16_TOL = dict(rtol=2e-2, atol=2e-3)


def make_o_inputs(seed, B, T, H, K, V, Hg=None, gate="logsigmoid", shift=3.0, cu=None, dtype="bf16"):
    """q, k ~ L2-normalised randn over K; v_new ~ randn; h ~ 0.3 randn; chunk-local g."""
    rng = np.random.default_rng(seed)
    Hg = H if Hg is None else Hg
    _, NT = O.sequence_bounds(B, T, cu)
    q = rng.standard_normal((B, T, Hg, K)).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k = rng.standard_normal((B, T, Hg, K)).astype(np.float32)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, T, H, V)).astype(np.float32)
    h = (rng.standard_normal((B, NT, H, K, V)) * 0.3).astype(np.float32)
    g = None if gate is None else O.make_gate(rng, B, T, H, gate, cu, shift=shift)
    if dtype == "bf16":
        q, k, v, h = (O.bf16_round(x) for x in (q, k, v, h))
    return dict(q=q, k=k, v_new=v, h=h, g=g, cu_seqlens=cu)


def _tokenwise_case(seed, B, T, H, K, V, Hg, cu):
    rng = np.random.default_rng(seed)
    N = B if cu is None else len(cu) - 1
    k = rng.standard_normal((B, T, Hg, K))
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    q = rng.standard_normal((B, T, Hg, K))
    v = rng.standard_normal((B, T, H, V))
    beta = 1 / (1 + np.exp(-rng.standard_normal((B, T, H))))
    a = -np.logaddexp(0, -(rng.standard_normal((B, T, H)) + 2.0))
    h0 = rng.standard_normal((N, H, K, V)) * 0.3
    kf, qf = np.repeat(k, H // Hg, axis=2), np.repeat(q, H // Hg, axis=2)
    _, _, o_tok = O.gated_delta_rule_tokenwise(kf, v, beta, a, initial_state=h0, cu_seqlens=cu, q=qf, scale=0.6)
    w, u, g = O.wy_prepare(kf, v, beta, a, cu_seqlens=cu)
    h, vn, _ = O.fwd_h(k, w, u, g=g, initial_state=h0, cu_seqlens=cu, compute_dtype=np.float64)
    return dict(q=q, k=k, v_new=vn, h=h, g=g, cu=cu, o_tok=o_tok, w=w, u=u, h0=h0)


TOKENWISE = [
    (1, 130, 2, 16, 8, 2, None),
    (2, 70, 2, 8, 12, 1, None),
    (1, 150, 4, 16, 16, 2, np.array([0, 1, 65, 150])),
    (1, 64, 1, 32, 32, 1, None),
]


@pytest.mark.parametrize("B,T,H,K,V,Hg,cu", TOKENWISE)
def test_oracle_chain_matches_tokenwise_output(B, T, H, K, V, Hg, cu):
    c = _tokenwise_case(11, B, T, H, K, V, Hg, cu)
    o = O.chunk_o(c["q"], c["k"], c["v_new"], c["h"], g=c["g"], scale=0.6, cu_seqlens=cu,
                  compute_dtype=np.float64)
    scale = np.abs(c["o_tok"]).max()
    assert np.abs(o - c["o_tok"]).max() <= 1e-10 * scale
    # a planted omission (no intra-chunk term) is caught by a wide margin
    o_bad = O.chunk_o(c["q"], c["k"], np.zeros_like(c["v_new"]), c["h"], g=c["g"], scale=0.6,
                      cu_seqlens=cu, compute_dtype=np.float64)
    assert np.abs(o_bad - c["o_tok"]).max() > 1e-3 * scale


def test_oracle_closed_forms():
    inp = make_o_inputs(3, 1, 150, 2, 32, 16, dtype="f32")
    q, k, v, h, g = inp["q"], inp["k"], inp["v_new"], inp["h"], inp["g"]
    sc = 0.37
    # k = 0: only the inter-chunk term
    o = O.chunk_o(q, np.zeros_like(k), v, h, g=g, scale=sc, compute_dtype=np.float64)
    for t in (0, 63, 64, 149):
        c = t // 64
        ref = sc * np.exp(g[0, t, :, None].astype(np.float64)) * np.einsum("hk,hkv->hv", q[0, t].astype(np.float64), h[0, c])
        np.testing.assert_allclose(o[0, t], ref, rtol=1e-12, atol=1e-14)
    # h = 0 and one-token chunks: scale (q_i.k_i) v_i
    cu = np.arange(0, 9, dtype=np.int64)
    i8 = make_o_inputs(4, 1, 8, 2, 32, 16, dtype="f32", cu=cu)
    o = O.chunk_o(i8["q"], i8["k"], i8["v_new"], np.zeros_like(i8["h"]), g=i8["g"], scale=sc,
                  cu_seqlens=cu, compute_dtype=np.float64)
    qk = np.einsum("thk,thk->th", i8["q"][0].astype(np.float64), i8["k"][0].astype(np.float64))
    np.testing.assert_allclose(o[0], sc * qk[:, :, None] * i8["v_new"][0], rtol=1e-12, atol=1e-14)
    # g = None is g = 0
    a = O.chunk_o(q, k, v, h, g=None, scale=sc)
    b = O.chunk_o(q, k, v, h, g=np.zeros_like(g), scale=sc)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("shift", [3.0, -2.0])
def test_oracle_bf16_model_near_exact(shift):
    inp = make_o_inputs(5, 2, 200, 2, 64, 64, shift=shift)
    ex = O.chunk_o(**inp)
    r1 = O.chunk_o(**inp, rounding="bf16")
    assert np.abs(r1 - ex).max() <= 1e-2 * np.abs(ex).max()


# ----------------------------------------------------------------------------- host-side ABI

def _oargs(B=1, T=256, H=4, Hg=2, K=128, V=128, varlen=None):
    a = _abi.ChunkOArgs()
    fake = 1 << 24
    a.q = a.k = a.v_new = a.h = a.o = fake
    a.B, a.T, a.H, a.Hg, a.K, a.V = B, T, H, Hg, K, V
    if varlen is None:
        a.N, a.NT = B, (T + 63) // 64
    else:
        a.cu_seqlens = fake
        a.N, a.NT = len(varlen) - 1, int(O.prepare_chunk_offsets(np.asarray(varlen))[-1])
    a.chunk_size, a.scale, a.in_dtype = 64, 1.0, _abi.CGDR_BF16
    a.stride_q[:] = a.stride_k[:] = [T * Hg * K, Hg * K, K]
    a.stride_v[:] = a.stride_o[:] = [T * H * V, H * V, V]
    a.stride_h[:] = [a.NT * H * K * V, H * K * V, K * V]
    return a


def _status(a):
    vt, wg = ctypes.c_int32(0), ctypes.c_int64(0)
    return _abi.load().cgdr_chunk_o_get_plan(ctypes.byref(a), ctypes.byref(vt), ctypes.byref(wg))


def test_chunk_o_plan():
    assert _abi.chunk_o_plan(_oargs()) == (128, 1 * 4 * 4)
    assert _abi.chunk_o_plan(_oargs(K=256, V=256)) == (64, 4 * 4 * 4)
    assert _abi.chunk_o_plan(_oargs(V=96, Hg=4)) == (32, 4 * 4 * 3)
    assert _abi.chunk_o_plan(_oargs(B=1, T=32768, H=32, Hg=32)) == (128, 512 * 32)
    assert _abi.chunk_o_plan(_oargs(T=300, varlen=[0, 100, 300])) == (128, 6 * 4)


@pytest.mark.parametrize("mutate,status", [
    (lambda a: setattr(a, "q", None), _abi.CGDR_ERR_NULLPTR),
    (lambda a: setattr(a, "o", None), _abi.CGDR_ERR_NULLPTR),
    (lambda a: setattr(a, "h", None), _abi.CGDR_ERR_NULLPTR),
    (lambda a: setattr(a, "chunk_size", 128), _abi.CGDR_ERR_UNSUPPORTED),
    (lambda a: setattr(a, "in_dtype", _abi.CGDR_F32), _abi.CGDR_ERR_UNSUPPORTED),
    (lambda a: setattr(a, "in_dtype", 7), _abi.CGDR_ERR_INVALID),
    (lambda a: setattr(a, "K", 96), _abi.CGDR_ERR_UNSUPPORTED),
    (lambda a: setattr(a, "Hg", 3), _abi.CGDR_ERR_INVALID),
    (lambda a: setattr(a, "NT", 5), _abi.CGDR_ERR_INVALID),
    (lambda a: setattr(a, "N", 2), _abi.CGDR_ERR_INVALID),
    (lambda a: setattr(a, "chunk_indices", 1 << 24), _abi.CGDR_ERR_INVALID),
    (lambda a: a.stride_q.__setitem__(1, 100), _abi.CGDR_ERR_UNSUPPORTED),
    (lambda a: setattr(a, "o", (1 << 24) + 2), _abi.CGDR_ERR_UNSUPPORTED),
    (lambda a: a.stride_h.__setitem__(2, 100), _abi.CGDR_ERR_INVALID),
    (lambda a: setattr(a, "scale", float("nan")), _abi.CGDR_ERR_INVALID),
])
def test_chunk_o_validation(mutate, status):
    a = _oargs()
    mutate(a)
    assert _status(a) == status
    assert _abi.last_error()


def test_chunk_o_validation_v_and_varlen():
    a = _oargs(V=48)
    assert _status(a) == _abi.CGDR_ERR_UNSUPPORTED and "multiple of 32" in _abi.last_error()
    a = _oargs(T=300, varlen=[0, 100, 300])
    a.NT = 4
    assert _status(a) == _abi.CGDR_ERR_INVALID
    a = _oargs(B=2, T=300, varlen=[0, 100, 300])
    assert _status(a) == _abi.CGDR_ERR_INVALID


# ----------------------------------------------------------------------------- GPU parity

def _dev(inp, dev):
    t = lambda x, dt: None if x is None else torch.from_numpy(np.ascontiguousarray(x)).to(device=dev, dtype=dt)
    return (t(inp["q"], torch.bfloat16), t(inp["k"], torch.bfloat16), t(inp["v_new"], torch.bfloat16),
            t(inp["h"], torch.bfloat16), t(inp["g"], torch.float32),
            None if inp["cu_seqlens"] is None else torch.from_numpy(np.asarray(inp["cu_seqlens"], np.int64)).to(dev))


def _check(got, inp, scale):
    got = got.float().cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    r1 = O.chunk_o(**inp, scale=scale, rounding="bf16")
    ex = O.chunk_o(**inp, scale=scale)
    err = np.abs(got - r1)
    bad = err > BF16_TOL["atol"] + BF16_TOL["rtol"] * np.abs(r1)
    assert not bad.any(), f"{bad.sum()}/{bad.size} outside rtol=2e-2, atol=2e-3 of the bf16 model; max err {err.max():.3e}"
    assert np.abs(got - ex).max() <= 1e-2 * np.abs(ex).max()


CASES = [
    # B, T, H, Hg, K, V, gate, shift, varlen
    (1, 64, 1, 1, 128, 128, "logsigmoid", 3.0, None),
    (2, 200, 4, 2, 128, 128, "logsigmoid", 3.0, None),
    (1, 300, 2, 2, 64, 64, "logsigmoid", -2.0, None),
    (1, 130, 2, 1, 32, 32, "linear", 0.0, None),
    (1, 257, 2, 2, 256, 128, "logsigmoid", 3.0, None),
    (1, 100, 2, 2, 128, 96, None, 0.0, None),
    (1, 700, 2, 2, 128, 256, "logsigmoid", 3.0, np.array([0, 1, 64, 65, 129, 400, 700])),
]


@pytest.mark.gpu
@pytest.mark.parametrize("B,T,H,Hg,K,V,gate,shift,cu", CASES)
def test_chunk_o_kernel_matches_oracle(dev, B, T, H, Hg, K, V, gate, shift, cu):
    import cgdr_amd
    print(f"[chunk_o] B={B} T={T} H={H} Hg={Hg} K={K} V={V} gate={gate} varlen={cu is not None}", flush=True)
    inp = make_o_inputs(21, B, T, H, K, V, Hg=Hg, gate=gate, shift=shift, cu=cu)
    q, k, v, h, g, cud = _dev(inp, dev)
    o = cgdr_amd.chunk_fwd_o(q, k, v, h, g=g, scale=0.5, cu_seqlens=cud)
    torch.cuda.synchronize()
    _check(o, inp, 0.5)
    if cud is not None:   # cu_seqlens on the host (copied through pinned memory): the same bits
        o2 = cgdr_amd.chunk_fwd_o(q, k, v, h, g=g, scale=0.5, cu_seqlens=cud.cpu())
        torch.cuda.synchronize()
        assert torch.equal(o, o2)


def _abi_o(q, k, v, h, g, cu, ci, o, scale, N, NT):
    from cgdr_amd.chunk_o import _args
    a = _args(q, k, v, h, g, cu, ci, o, scale, N, NT)
    _abi.chunk_o_launch(a, torch.cuda.current_stream(q.device).cuda_stream)
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_chunk_o_device_chunk_mapping_equals_chunk_indices(dev):
    """cu_seqlens alone (the kernel scans it) and cu_seqlens + chunk_indices give the same bits;
    o starts as NaN, so every token must be written."""
    cu = np.array([0, 5, 69, 133, 134, 400], np.int64)
    print("[chunk_o] device chunk mapping", flush=True)
    inp = make_o_inputs(8, 1, 400, 2, 128, 128, cu=cu)
    q, k, v, h, g, cud = _dev(inp, dev)
    NT = int(O.prepare_chunk_offsets(cu)[-1])
    ci = torch.from_numpy(O.prepare_chunk_indices(cu).astype(np.int64)).to(dev)
    outs = []
    for cidx in (None, ci):
        o = torch.full((1, 400, 2, 128), float("nan"), dtype=torch.bfloat16, device=dev)
        _abi_o(q, k, v, h, g, cud, cidx, o, 0.3, len(cu) - 1, NT)
        outs.append(o)
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    _check(outs[0], inp, 0.3)


@pytest.mark.gpu
def test_chunk_o_vtile_and_layout_invariance(dev):
    """V = 128 (one tile) equals V = 256 (two tiles) column for column; head-major views of
    q, k, v, o give the token-major bits."""
    import cgdr_amd
    print("[chunk_o] invariance", flush=True)
    inp = make_o_inputs(9, 1, 192, 2, 128, 256)
    q, k, v, h, g, _ = _dev(inp, dev)
    o2 = cgdr_amd.chunk_fwd_o(q, k, v, h, g=g)
    o1 = cgdr_amd.chunk_fwd_o(q, k, v[..., :128].contiguous(), h[..., :128].contiguous(), g=g)
    assert torch.equal(o1.view(torch.int16), o2[..., :128].contiguous().view(torch.int16))
    # head-major storage, passed as strided views
    qh = q.transpose(1, 2).contiguous().transpose(1, 2)
    kh = k.transpose(1, 2).contiguous().transpose(1, 2)
    vh = v.transpose(1, 2).contiguous().transpose(1, 2)
    gh = g.transpose(1, 2).contiguous().transpose(1, 2)
    o3 = cgdr_amd.chunk_fwd_o(qh, kh, vh, h, g=gh)
    torch.cuda.synchronize()
    assert torch.equal(o3.view(torch.int16), o2.view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("cu", [None, np.array([0, 70, 200, 256])])
def test_fwd_h_then_chunk_o_matches_tokenwise(dev, cu):
    """The forward pass on the GPU: WY inputs (oracle) -> cgdr_fwd_h -> cgdr_chunk_o, against
    the token-by-token recurrence (float64) within 1% of the output's scale."""
    import cgdr_amd
    print(f"[chunk_o] end to end varlen={cu is not None}", flush=True)
    B, T, H, Hg, K, V = 1, 256, 2, 2, 128, 128
    c = _tokenwise_case(13, B, T, H, K, V, Hg, cu)
    t = lambda x, dt=torch.bfloat16: torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(device=dev, dtype=dt)
    k, q, g = c["k"], c["q"], c["g"]
    cud = None if cu is None else torch.from_numpy(cu.astype(np.int64)).to(dev)
    h, vn, _ = cgdr_amd.chunk_gated_delta_rule_fwd_h(t(k), t(c["w"]), t(c["u"]), g=t(g, torch.float32),
                                                     initial_state=t(c["h0"], torch.float32), cu_seqlens=cud)
    o = cgdr_amd.chunk_fwd_o(t(q), t(k), vn, h, g=t(g, torch.float32), scale=0.6, cu_seqlens=cud)
    torch.cuda.synchronize()
    got = o.float().cpu().numpy()
    ref = c["o_tok"]
    assert np.abs(got - ref).max() <= 1e-2 * np.abs(ref).max()
