"""Helpers for the GPU tests: device copies of oracle inputs, a direct C-ABI call with
NaN-canaried output buffers, and the tolerance check."""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from cgdr_amd import _abi
from oracle import cgdr_oracle as O


def dev_inputs(inp: dict, dtype: torch.dtype, device, h0_dtype=torch.float32) -> dict:
    """Oracle inputs (float32 arrays holding bf16 values for bf16 cases) on the device."""
    out = {}
    for k in ("k", "w", "u"):
        out[k] = torch.from_numpy(np.ascontiguousarray(inp[k])).to(device=device, dtype=dtype)
    out["g"] = None if inp.get("g") is None else torch.from_numpy(np.ascontiguousarray(inp["g"])).to(device)
    h0 = inp.get("initial_state")
    out["initial_state"] = None if h0 is None else torch.from_numpy(np.ascontiguousarray(h0)).to(device, h0_dtype)
    cu = inp.get("cu_seqlens")
    out["cu_seqlens"] = None if cu is None else torch.from_numpy(np.asarray(cu, np.int64)).to(device)
    return out


_DT = {torch.bfloat16: _abi.CGDR_BF16, torch.float32: _abi.CGDR_F32}


def abi_call(d: dict, save_new_value=True, output_final_state=True, final_dtype=torch.float32,
             canary=float("nan"), tuning: dict | None = None, numerics: int = 0, no_alloc: bool = False,
             v_pad: int = 0):
    """Token-major FwdH through the C ABI into output buffers pre-filled with `canary`;
    `tuning` (fields of cgdr_fwd_h_tuning) overrides the launch plan; `numerics` is a
    cgdr_numerics; `no_alloc` calls cgdr_fwd_h_launch_no_alloc (its static scratch) instead of
    cgdr_fwd_h_launch with a workspace; `v_pad` > 0 leaves that many elements between v_new's
    token rows (a token stride of H * V + v_pad)."""
    k, w, u, g, h0, cu = d["k"], d["w"], d["u"], d["g"], d["initial_state"], d["cu_seqlens"]
    B, T, Hg, K = k.shape
    H, V = u.shape[2], u.shape[3]
    if cu is None:
        N, NT, offs = B, (T + 63) // 64, None
    else:
        cu_h = cu.cpu().numpy()
        N = len(cu_h) - 1
        offs_h = O.prepare_chunk_offsets(cu_h)
        NT = int(offs_h[-1])
        offs = torch.from_numpy(offs_h).to(k.device)
    h = torch.full((B, NT, H, K, V), canary, dtype=k.dtype, device=k.device)
    v = None
    if save_new_value:
        vbuf = torch.full((B, T, H * V + v_pad), canary, dtype=u.dtype, device=k.device)
        v = vbuf.as_strided((B, T, H, V), (T * (H * V + v_pad), H * V + v_pad, V, 1))
    f = torch.full((N, H, K, V), canary, dtype=final_dtype, device=k.device) if output_final_state else None
    a = _abi.FwdHArgs()
    a.k, a.w, a.u = k.data_ptr(), w.data_ptr(), u.data_ptr()
    a.g = None if g is None else g.data_ptr()
    a.initial_state = None if h0 is None else h0.data_ptr()
    a.cu_seqlens = None if cu is None else cu.data_ptr()
    a.chunk_offsets = None if offs is None else offs.data_ptr()
    a.h = h.data_ptr()
    a.v_new = None if v is None else v.data_ptr()
    a.final_state = None if f is None else f.data_ptr()
    a.B, a.T, a.H, a.Hg, a.K, a.V, a.N, a.NT = B, T, H, Hg, K, V, N, NT
    a.chunk_size = 64
    a.in_dtype = _DT[k.dtype]
    a.h0_dtype = _DT[h0.dtype] if h0 is not None else _abi.CGDR_F32
    a.final_dtype = _DT[final_dtype]
    a.stride_k[:] = list(k.stride()[:3])
    a.stride_w[:] = list(w.stride()[:3])
    a.stride_u[:] = list(u.stride()[:3])
    if g is not None:
        a.stride_g[:] = list(g.stride())
    a.stride_h[:] = list(h.stride()[:3])
    if v is not None:
        a.stride_v[:] = list(v.stride()[:3])
    if h0 is not None:
        a.stride_h0[:] = list(h0.stride()[:2])
    if f is not None:
        a.stride_final[:] = list(f.stride()[:2])
    a.numerics = numerics
    if tuning:
        t = _abi.make_tuning(**tuning)
        a.tuning = ctypes.pointer(t)
    if no_alloc:
        _abi.launch_no_alloc(a, torch.cuda.current_stream(k.device).cuda_stream)
        torch.cuda.synchronize()
        return h, v, f
    nws = _abi.workspace_size(a)
    ws = torch.full((max(nws, 1),), 0xAB, dtype=torch.uint8, device=k.device)
    _abi.launch(a, torch.cuda.current_stream(k.device).cuda_stream, ws.data_ptr() if nws else 0, nws)
    torch.cuda.synchronize()
    return h, v, f


def np32(t):
    return None if t is None else t.float().cpu().numpy()


def assert_close(got, ref, rtol, atol, name=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{name}: non-finite values (unwritten canary or overflow)"
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    bad = err > bound
    if bad.any():
        i = np.unravel_index(np.argmax(err / bound), err.shape)
        raise AssertionError(f"{name}: {bad.sum()}/{bad.size} elements outside rtol={rtol}, atol={atol}; "
                             f"worst at {i}: got {got[i]!r}, ref {ref[i]!r}")


def assert_scale_close(got, ref, frac, name=""):
    """max|got - ref| <= frac * max|ref| (a bound relative to the tensor's scale)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    err = np.abs(got - ref).max()
    scale = max(np.abs(ref).max(), 1e-30)
    assert err <= frac * scale, f"{name}: max err {err:.3e} > {frac} * scale {scale:.3e}"
