"""WY producer of FwdH's w, u, g, and the full chunked forward built on it.

CPU (oracle pins):
  * wy_prepare -> fwd_h reproduces the token-by-token recurrence's states (tests/test_oracle.py)
    and, with chunk_o, its outputs (tests/test_chunk_o.py); here: the bf16 rounding model of
    wy_prepare stays within 1% of the exact w, u; its g is the float32 sequential cumsum;
    GQA equals repeating the keys.
CPU (host side): validation of cgdr_wy_args.
GPU (tolerances written per check): g_cumsum bit-exact against numpy's sequential float32
  cumsum; w, u elementwise within rtol=2e-2, atol=2e-3 of the bf16 rounding model and within
  1% of the tensor's scale of the exact float64 WY representation; bf16 and fp32 beta agree
  bit for bit when beta holds bf16 values; the GPU forward (WY -> FwdH -> chunk output)
  against the token-by-token recurrence within 1% of the output's scale.
"""

import numpy as np
import pytest
import torch

from cgdr_amd import _abi
from oracle import cgdr_oracle as O

BF16_TOL = dict(rtol=2e-2, atol=2e-3)


def make_wy_inputs(seed, B, T, H, K, V, Hg=None, shift=2.0, cu=None, gate=True):
    rng = np.random.default_rng(seed)
    Hg = H if Hg is None else Hg
    k = rng.standard_normal((B, T, Hg, K)).astype(np.float32)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, T, H, V)).astype(np.float32)
    beta = (1 / (1 + np.exp(-rng.standard_normal((B, T, H))))).astype(np.float32)
    a = (-np.logaddexp(0, -(rng.standard_normal((B, T, H)) + shift))).astype(np.float32) if gate else None
    return dict(k=O.bf16_round(k), v=O.bf16_round(v), beta=O.bf16_round(beta), a=a, cu=cu)


def test_oracle_wy_bf16_model_near_exact():
    inp = make_wy_inputs(1, 1, 200, 2, 64, 64, cu=np.array([0, 70, 200]))
    a = inp["a"]
    ex = O.wy_prepare(inp["k"], inp["v"], inp["beta"], a, cu_seqlens=inp["cu"])
    r1 = O.wy_prepare(inp["k"], inp["v"], inp["beta"], a, cu_seqlens=inp["cu"], rounding="bf16")
    for x, y in zip(ex[:2], r1[:2]):
        assert np.abs(x - y).max() <= 1e-2 * np.abs(x).max()
    # g of the rounding model is the float32 sequential cumsum, restarted per chunk and sequence
    g = r1[2]
    for (s0, s1) in ((0, 64), (64, 70), (70, 134), (134, 198), (198, 200)):
        np.testing.assert_array_equal(g[0, s0:s1], np.cumsum(a[0, s0:s1], axis=0, dtype=np.float32))


def test_oracle_wy_gqa_is_repeated_keys():
    inp = make_wy_inputs(2, 1, 130, 4, 32, 32, Hg=2)
    g1 = O.wy_prepare(inp["k"], inp["v"], inp["beta"], inp["a"])
    g2 = O.wy_prepare(np.repeat(inp["k"], 2, axis=2), inp["v"], inp["beta"], inp["a"])
    for x, y in zip(g1, g2):
        np.testing.assert_array_equal(x, y)


# ----------------------------------------------------------------------------- host-side ABI

def _wargs(B=1, T=256, H=4, Hg=2, K=128, V=128):
    a = _abi.WyArgs()
    fake = 1 << 24
    a.k = a.v = a.beta = a.w = a.u = fake
    a.B, a.T, a.H, a.Hg, a.K, a.V, a.N, a.NT = B, T, H, Hg, K, V, B, (T + 63) // 64
    a.chunk_size, a.in_dtype, a.beta_dtype = 64, _abi.CGDR_BF16, _abi.CGDR_F32
    a.stride_k[:] = [T * Hg * K, Hg * K, K]
    a.stride_v[:] = [T * H * V, H * V, V]
    a.stride_w[:] = [T * H * K, H * K, K]
    a.stride_u[:] = [T * H * V, H * V, V]
    a.stride_beta[:] = [T * H, H, 1]
    return a


@pytest.mark.parametrize("mutate,status", [
    (lambda a: setattr(a, "k", None), _abi.CGDR_ERR_NULLPTR),
    (lambda a: setattr(a, "beta", None), _abi.CGDR_ERR_NULLPTR),
    (lambda a: setattr(a, "u", None), _abi.CGDR_ERR_NULLPTR),
    (lambda a: setattr(a, "chunk_size", 32), _abi.CGDR_ERR_UNSUPPORTED),
    (lambda a: setattr(a, "in_dtype", _abi.CGDR_F32), _abi.CGDR_ERR_UNSUPPORTED),
    (lambda a: setattr(a, "beta_dtype", 5), _abi.CGDR_ERR_INVALID),
    (lambda a: setattr(a, "K", 96), _abi.CGDR_ERR_UNSUPPORTED),
    (lambda a: setattr(a, "V", 512), _abi.CGDR_ERR_UNSUPPORTED),
    (lambda a: setattr(a, "Hg", 3), _abi.CGDR_ERR_INVALID),
    (lambda a: setattr(a, "NT", 3), _abi.CGDR_ERR_INVALID),
    (lambda a: setattr(a, "chunk_indices", 1 << 24), _abi.CGDR_ERR_INVALID),
    (lambda a: a.stride_v.__setitem__(1, 4 * 128 + 4), _abi.CGDR_ERR_UNSUPPORTED),
    (lambda a: a.stride_beta.__setitem__(1, 0), _abi.CGDR_ERR_INVALID),
])
def test_wy_validation(mutate, status):
    """Rejected before any device call (the launch is never reached)."""
    a = _wargs()
    mutate(a)
    import ctypes
    assert _abi.load().cgdr_wy_launch(ctypes.byref(a), None) == status
    assert _abi.last_error()


# ----------------------------------------------------------------------------- GPU parity

def _dev(x, dev, dt):
    return None if x is None else torch.from_numpy(np.ascontiguousarray(x)).to(device=dev, dtype=dt)


CASES = [
    # B, T, H, Hg, K, V, varlen, gate, beta dtype
    (1, 64, 1, 1, 128, 128, None, True, torch.float32),
    (2, 200, 4, 2, 128, 128, None, True, torch.bfloat16),
    (1, 300, 2, 2, 64, 64, None, True, torch.float32),
    (1, 130, 2, 1, 32, 256, None, False, torch.float32),
    (1, 150, 2, 2, 256, 64, None, True, torch.float32),
    (1, 700, 2, 2, 128, 128, np.array([0, 1, 64, 65, 129, 400, 700]), True, torch.float32),
]


@pytest.mark.gpu
@pytest.mark.parametrize("B,T,H,Hg,K,V,cu,gate,bdt", CASES)
def test_wy_kernel_matches_oracle(dev, B, T, H, Hg, K, V, cu, gate, bdt):
    import cgdr_amd
    print(f"[wy] B={B} T={T} H={H} Hg={Hg} K={K} V={V} varlen={cu is not None} gate={gate} beta={bdt}", flush=True)
    inp = make_wy_inputs(31, B, T, H, K, V, Hg=Hg, cu=cu, gate=gate)
    cud = None if cu is None else torch.from_numpy(cu.astype(np.int64)).to(dev)
    w, u, gc = cgdr_amd.wy_fwd(_dev(inp["k"], dev, torch.bfloat16), _dev(inp["v"], dev, torch.bfloat16),
                               _dev(inp["beta"], dev, bdt), g=_dev(inp["a"], dev, torch.float32), cu_seqlens=cud)
    torch.cuda.synchronize()
    a = inp["a"] if gate else np.zeros((B, T, H), np.float32)
    r1 = O.wy_prepare(inp["k"], inp["v"], inp["beta"], a, cu_seqlens=cu, rounding="bf16")
    ex = O.wy_prepare(inp["k"], inp["v"], inp["beta"], a, cu_seqlens=cu)
    np.testing.assert_array_equal(gc.cpu().numpy(), r1[2].astype(np.float32))
    for name, got, m, x in (("w", w, r1[0], ex[0]), ("u", u, r1[1], ex[1])):
        got = got.float().cpu().numpy().astype(np.float64)
        assert np.isfinite(got).all()
        err = np.abs(got - m)
        bad = err > BF16_TOL["atol"] + BF16_TOL["rtol"] * np.abs(m)
        assert not bad.any(), f"{name}: {bad.sum()}/{bad.size} outside rtol=2e-2, atol=2e-3 of the model; max {err.max():.3e}"
        assert np.abs(got - x).max() <= 1e-2 * np.abs(x).max(), name


@pytest.mark.gpu
def test_wy_beta_dtypes_agree(dev):
    import cgdr_amd
    print("[wy] beta dtypes", flush=True)
    inp = make_wy_inputs(32, 1, 192, 2, 128, 128)
    k, v, g = _dev(inp["k"], dev, torch.bfloat16), _dev(inp["v"], dev, torch.bfloat16), _dev(inp["a"], dev, torch.float32)
    o1 = cgdr_amd.wy_fwd(k, v, _dev(inp["beta"], dev, torch.bfloat16), g=g)
    o2 = cgdr_amd.wy_fwd(k, v, _dev(inp["beta"], dev, torch.float32), g=g)
    torch.cuda.synchronize()
    for x, y in zip(o1, o2):
        assert torch.equal(x, y)


@pytest.mark.gpu
@pytest.mark.parametrize("cu", [None, np.array([0, 100, 130, 384])])
def test_full_forward_matches_tokenwise(dev, cu):
    """chunk_gated_delta_rule_fwd (WY -> FwdH -> chunk output, all on the GPU) against the
    token-by-token Gated DeltaNet recurrence in float64."""
    import cgdr_amd
    print(f"[wy] full forward varlen={cu is not None}", flush=True)
    rng = np.random.default_rng(41)
    B, T, H, Hg, K, V = 1, 384, 4, 2, 128, 128
    N = 1 if cu is None else len(cu) - 1
    inp = make_wy_inputs(41, B, T, H, K, V, Hg=Hg, cu=cu)
    q = O.bf16_round((rng.standard_normal((B, T, Hg, K)) / np.sqrt(K)).astype(np.float32))
    h0 = (rng.standard_normal((N, H, K, V)) * 0.3).astype(np.float32)
    kf, qf = np.repeat(inp["k"], H // Hg, axis=2), np.repeat(q, H // Hg, axis=2)
    _, fin, o_ref = O.gated_delta_rule_tokenwise(kf, inp["v"], inp["beta"], inp["a"], initial_state=h0,
                                                 cu_seqlens=cu, q=qf, scale=K ** -0.5)
    cud = None if cu is None else torch.from_numpy(cu.astype(np.int64)).to(dev)
    o, f = cgdr_amd.chunk_gated_delta_rule_fwd(
        _dev(q, dev, torch.bfloat16), _dev(inp["k"], dev, torch.bfloat16), _dev(inp["v"], dev, torch.bfloat16),
        _dev(inp["a"], dev, torch.float32), _dev(inp["beta"], dev, torch.float32),
        initial_state=_dev(h0, dev, torch.float32), output_final_state=True, cu_seqlens=cud)
    torch.cuda.synchronize()
    got_o, got_f = o.float().cpu().numpy(), f.cpu().numpy()
    assert np.abs(got_o - o_ref).max() <= 1e-2 * np.abs(o_ref).max()
    assert np.abs(got_f - fin).max() <= 1e-2 * np.abs(fin).max()
