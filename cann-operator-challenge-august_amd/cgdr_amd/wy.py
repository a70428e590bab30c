"""Python interface of the WY producer on MI355X, and the full chunked forward built from it.

``wy_fwd(k, v, beta, g=None, cu_seqlens=None, chunk_indices=None, chunk_size=64)`` returns
``(w, u, g_cumsum)``, FwdH's inputs, for token-major k ``[B,T,Hg,K]``, v ``[B,T,H,V]``, beta
``[B,T,H]`` and the per-token log-decay g ``[B,T,H]`` (``include/cgdr_wy.h``; the WY part of
``ref/chunk_gated_delta_rule/tests/pytest/chunk_gated_delta_rule_golden.py:102-124``, paths
relative to the reference's ``ChunkGatedDeltaRuleFwdH_problem_290_template/``).

``chunk_gated_delta_rule_fwd(q, k, v, g, beta, scale=None, initial_state=None,
output_final_state=False, cu_seqlens=None)`` returns ``(o, final_state)``: WY producer ->
FwdH -> chunk output, all three on the GPU.  It computes what the reference's full-operator
golden ``chunk_gated_delta_rule_npu`` / ``chunk_gated_delta_rule_native``
(``chunk_gated_delta_rule_golden.py:15-157``) computes, without its q/k L2 normalisation
switch (which that golden accepts and ignores, ``:81``).
"""

from __future__ import annotations

import torch

from . import _abi
from .chunk_o import chunk_fwd_o
from .fwd_h import CHUNK_SIZE, _prep_input, _ptr, _varlen_meta, chunk_gated_delta_rule_fwd_h


def wy_fwd(
    k: torch.Tensor,
    v: torch.Tensor,
    beta: torch.Tensor,
    g: torch.Tensor | None = None,
    cu_seqlens: torch.LongTensor | None = None,
    chunk_indices: torch.Tensor | None = None,
    chunk_size: int = CHUNK_SIZE,
):
    """``(w [B,T,H,K], u [B,T,H,V], g_cumsum [B,T,H] fp32)``; bf16 k and v.  g_cumsum is a
    head-major view (strides ``(H*T, 1, T)``)."""
    if chunk_size != CHUNK_SIZE:
        raise ValueError(f"chunk_size must be {CHUNK_SIZE}, but got {chunk_size}")
    for t, name in ((k, "k"), (v, "v")):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16 (got {t.dtype})")
        if t.device.type != "cuda":
            raise ValueError(f"{name} must be a HIP device tensor (got {t.device})")
    if k.dim() != 4 or v.dim() != 4:
        raise ValueError("k must be [B,T,Hg,K] and v [B,T,H,V]")
    B, T, Hg, K = k.shape
    H, V = v.shape[2], v.shape[3]
    if tuple(v.shape[:2]) != (B, T) or H % Hg != 0:
        raise ValueError(f"v must be [B,T,H,V] with H a multiple of Hg={Hg}, got {list(v.shape)}")
    if tuple(beta.shape) != (B, T, H):
        raise ValueError(f"beta must have shape [B,T,H]={[B, T, H]}, got {list(beta.shape)}")
    if beta.dtype not in (torch.bfloat16, torch.float32):
        beta = beta.float()
    if g is not None:
        if tuple(g.shape) != (B, T, H):
            raise ValueError(f"g must have shape [B,T,H]={[B, T, H]}, got {list(g.shape)}")
        if g.dtype != torch.float32:
            g = g.float()
    dev = k.device
    if cu_seqlens is None:
        if chunk_indices is not None:
            raise ValueError("chunk_indices requires cu_seqlens")
        N, NT, cu_dev, ci_dev = B, (T + CHUNK_SIZE - 1) // CHUNK_SIZE, None, None
    else:
        if B != 1:
            raise ValueError(f"cu_seqlens requires B == 1, got B={B}")
        N, NT, cu_dev, _ = _varlen_meta(cu_seqlens, T, chunk_indices, None, dev, want_offsets=False)
        ci_dev = None
    k, v = _prep_input(k, "k", 16), _prep_input(v, "v", 16)
    w = torch.empty(B, T, H, K, dtype=torch.bfloat16, device=dev)
    u = torch.empty(B, T, H, V, dtype=torch.bfloat16, device=dev)
    # g_cumsum is stored head-major ([B,H,T] memory, returned as a [B,T,H] view): every token
    # belongs to a chunk, so the kernel writes all of it, and FwdH and the chunk output read
    # one chunk's gate row of one head as 256 contiguous bytes (no relayout in FwdH)
    gc = torch.empty(B, H, T, dtype=torch.float32, device=dev).transpose(1, 2)
    a = _abi.WyArgs()
    a.k, a.v, a.beta, a.g = k.data_ptr(), v.data_ptr(), beta.data_ptr(), _ptr(g)
    a.cu_seqlens, a.chunk_indices = _ptr(cu_dev), _ptr(ci_dev)
    a.w, a.u, a.g_cumsum = w.data_ptr(), u.data_ptr(), gc.data_ptr()
    a.B, a.T, a.H, a.Hg, a.K, a.V, a.N, a.NT = B, T, H, Hg, K, V, N, NT
    a.chunk_size = CHUNK_SIZE
    a.in_dtype = _abi.CGDR_BF16
    a.beta_dtype = _abi.CGDR_F32 if beta.dtype == torch.float32 else _abi.CGDR_BF16
    a.stride_k[:] = list(k.stride()[:3])
    a.stride_v[:] = list(v.stride()[:3])
    a.stride_beta[:] = list(beta.stride())
    if g is not None:
        a.stride_g[:] = list(g.stride())
    a.stride_w[:] = list(w.stride()[:3])
    a.stride_u[:] = list(u.stride()[:3])
    a.stride_g_cumsum[:] = list(gc.stride())
    _abi.wy_launch(a, torch.cuda.current_stream(dev).cuda_stream)
    return w, u, gc


def chunk_gated_delta_rule_fwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor | None,
    beta: torch.Tensor,
    scale: float | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    cu_seqlens: torch.LongTensor | None = None,
    chunk_size: int = CHUNK_SIZE,
):
    """``(o [B,T,H,V] bf16, final_state [N,H,K,V] fp32 or None)``; see the module docstring."""
    w, u, gc = wy_fwd(k, v, beta, g=g, cu_seqlens=cu_seqlens, chunk_size=chunk_size)
    h, v_new, final = chunk_gated_delta_rule_fwd_h(
        k, w, u, g=gc if g is not None else None, initial_state=initial_state,
        output_final_state=output_final_state, chunk_size=chunk_size, cu_seqlens=cu_seqlens)
    o = chunk_fwd_o(q, k, v_new, h, g=gc if g is not None else None, scale=scale,
                    cu_seqlens=cu_seqlens, chunk_size=chunk_size)
    return o, final
