"""Python operator interface of the chunk output on MI355X, the consumer of FwdH's h and v_new.

``chunk_fwd_o(q, k, v, h, g=None, scale=None, cu_seqlens=None, chunk_indices=None,
chunk_size=64)`` returns ``o [B,T,H,V]`` for token-major q, k ``[B,T,Hg,K]``, v (FwdH's
``v_new``) ``[B,T,H,V]``, h ``[B,NT,H,K,V]`` and g ``[B,T,H]``::

    o_i = scale * (e^{g_i} q_i . h_c + sum_{j <= i in chunk c} (q_i . k_j) e^{g_i - g_j} v_j)

This is the per-chunk output of the reference's full operator
(``ref/chunk_gated_delta_rule/tests/pytest/chunk_gated_delta_rule_golden.py:136-142``, paths
relative to ``ChunkGatedDeltaRuleFwdH_problem_290_template/``; on the device its stage 2
``attn_inter`` and stage 3 masked product).  The argument names follow the FLA ``chunk_fwd_o``
the reference's statement names as upstream (``docs/problem.txt:27``).  ``scale`` defaults to
``K ** -0.5`` (``chunk_gated_delta_rule_golden.py:99``).  It calls ``cgdr_chunk_o_launch``
(``include/cgdr_chunk_o.h``); there is no CPU path.
"""

from __future__ import annotations

import torch

from . import _abi
from .fwd_h import CHUNK_SIZE, _host_to_device, _prep_input, _ptr, _varlen_meta


def _args(q, k, v, h, g, cu_dev, ci_dev, o, scale, N, NT) -> _abi.ChunkOArgs:
    B, T, Hg, K = q.shape
    H, V = v.shape[2], v.shape[3]
    a = _abi.ChunkOArgs()
    a.q, a.k, a.v_new, a.h = q.data_ptr(), k.data_ptr(), v.data_ptr(), h.data_ptr()
    a.g = _ptr(g)
    a.cu_seqlens, a.chunk_indices = _ptr(cu_dev), _ptr(ci_dev)
    a.o = o.data_ptr()
    a.B, a.T, a.H, a.Hg, a.K, a.V, a.N, a.NT = B, T, H, Hg, K, V, N, NT
    a.chunk_size = CHUNK_SIZE
    a.scale = float(scale)
    a.in_dtype = _abi.CGDR_BF16
    a.stride_q[:] = list(q.stride()[:3])
    a.stride_k[:] = list(k.stride()[:3])
    a.stride_v[:] = list(v.stride()[:3])
    a.stride_h[:] = list(h.stride()[:3])
    if g is not None:
        a.stride_g[:] = list(g.stride())
    a.stride_o[:] = list(o.stride()[:3])
    return a


def chunk_fwd_o(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    h: torch.Tensor,
    g: torch.Tensor | None = None,
    scale: float | None = None,
    cu_seqlens: torch.LongTensor | None = None,
    chunk_indices: torch.Tensor | None = None,
    chunk_size: int = CHUNK_SIZE,
) -> torch.Tensor:
    """``o`` for token-major inputs; see the module docstring.  bf16 inputs only."""
    if chunk_size != CHUNK_SIZE:
        raise ValueError(f"chunk_size must be {CHUNK_SIZE}, but got {chunk_size}")
    for t, name in ((q, "q"), (k, "k"), (v, "v"), (h, "h")):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16 (got {t.dtype})")
        if t.device.type != "cuda":
            raise ValueError(f"{name} must be a HIP device tensor (got {t.device})")
    if q.dim() != 4 or k.shape != q.shape or v.dim() != 4 or h.dim() != 5:
        raise ValueError("q, k must be [B,T,Hg,K], v [B,T,H,V] and h [B,NT,H,K,V]")
    B, T, Hg, K = q.shape
    H, V = v.shape[2], v.shape[3]
    if tuple(v.shape[:2]) != (B, T) or H % Hg != 0:
        raise ValueError(f"v must be [B,T,H,V] with H a multiple of Hg={Hg}, got {list(v.shape)}")
    dev = q.device
    if cu_seqlens is None:
        if chunk_indices is not None:
            raise ValueError("chunk_indices requires cu_seqlens")
        N, NT, cu_dev, ci_dev = B, (T + CHUNK_SIZE - 1) // CHUNK_SIZE, None, None
    else:
        if B != 1:
            raise ValueError(f"cu_seqlens requires B == 1, got B={B}")
        N, NT, cu_dev, _ = _varlen_meta(cu_seqlens, T, chunk_indices, None, dev, want_offsets=False)
        ci_dev = _host_to_device(_abi.prepare_chunk_indices(
            [int(x) for x in cu_seqlens.detach().to("cpu", torch.int64).tolist()], CHUNK_SIZE),
            dev).reshape(-1, 2) if NT > 0 else None
    if tuple(h.shape) != (B, NT, H, K, V):
        raise ValueError(f"h must have shape [B,NT,H,K,V]={[B, NT, H, K, V]}, got {list(h.shape)}")
    if g is not None:
        if tuple(g.shape) != (B, T, H):
            raise ValueError(f"g must have shape [B,T,H]={[B, T, H]}, got {list(g.shape)}")
        if g.dtype != torch.float32:
            g = g.float()
    q, k, v = _prep_input(q, "q", 16), _prep_input(k, "k", 16), _prep_input(v, "v", 16)
    blocks_ok = (h.stride(-1) == 1 and h.stride(-2) == V and h.stride(-3) == K * V
                 and h.data_ptr() % 16 == 0 and all(s % 8 == 0 for s in h.stride()[:3]))
    if not blocks_ok:
        h = h.contiguous()
    o = torch.empty(B, T, H, V, dtype=torch.bfloat16, device=dev)
    a = _args(q, k, v, h, g, cu_dev, ci_dev, o, K ** -0.5 if scale is None else scale, N, NT)
    _abi.chunk_o_launch(a, torch.cuda.current_stream(dev).cuda_stream)
    return o


def plan(q: torch.Tensor, v: torch.Tensor) -> dict:
    """V-tile and grid the library picks for fixed-length inputs of these shapes."""
    B, T, Hg, K = q.shape
    H, V = v.shape[2], v.shape[3]
    NT = (T + CHUNK_SIZE - 1) // CHUNK_SIZE
    a = _abi.ChunkOArgs()
    a.q = a.k = a.v_new = a.h = a.o = 256
    a.B, a.T, a.H, a.Hg, a.K, a.V, a.N, a.NT = B, T, H, Hg, K, V, B, NT
    a.chunk_size, a.scale, a.in_dtype = CHUNK_SIZE, 1.0, _abi.CGDR_BF16
    a.stride_q[:] = a.stride_k[:] = [T * Hg * K, Hg * K, K]
    a.stride_v[:] = a.stride_o[:] = [T * H * V, H * V, V]
    a.stride_h[:] = [NT * H * K * V, H * K * V, K * V]
    vt, wg = _abi.chunk_o_plan(a)
    return {"v_tile": vt, "workgroups": wg}
