"""Python operator interface of ChunkGatedDeltaRuleFwdH on MI355X.

Mirrors the reference's Python entry points (paths relative to the reference's
``ChunkGatedDeltaRuleFwdH_problem_290_template/``):

* ``chunk_gated_delta_rule_fwd_h`` -- the Triton wrapper of ``docs/problem.txt:436-500``
  (token-major k ``[B,T,Hg,K]``, w ``[B,T,H,K]``, u ``[B,T,H,V]``, g ``[B,T,H]``) returning
  ``h [B,NT,H,K,V]`` (k dtype), ``v_new`` (like u) and ``final_state [N,H,K,V]`` (fp32), with
  the ``output_final_state`` switch of the FLA signature.
* ``run`` -- the contest reference ``run(k, w, u, g, initial_state, cu_seqlens,
  chunk_indices, chunk_size)`` of ``docs/problem.txt:81-167`` in its head-major layout
  (w ``[B,HV,T,K]``, u ``[B,HV,T,V]``, g ``[B,HV,T]``) returning ``S [B,HV,NT,K,V]``,
  ``v [B,HV,T,V]`` and ``final_state [N,HV,K,V]`` in u's dtype.

Both call the same C ABI (``include/cgdr_fwd_h.h``); layouts are passed as strides, so
neither copies its inputs.  PyTorch provides device memory and the current HIP stream.
Varlen metadata is validated on the host like ``prepare_chunk_indices`` in the reference
(which also syncs to build its Python list).
"""

from __future__ import annotations

import ctypes

import torch

from . import _abi

CHUNK_SIZE = _abi.CHUNK_SIZE

_DTYPES = {torch.bfloat16: _abi.CGDR_BF16, torch.float32: _abi.CGDR_F32}
# "default": the Triton kernel's rounding model (docs/problem.txt:330-432) for bf16 inputs,
# exact fp32 for fp32 inputs; "contest": the contest reference run()'s fp16-saturating,
# bf16-state numerics (docs/problem.txt:81-167), bf16 inputs only.
_NUMERICS = {"default": _abi.CGDR_NUMERICS_DEFAULT, "contest": _abi.CGDR_NUMERICS_CONTEST}
_STATE_LAYOUTS = {"kv": _abi.CGDR_STATE_KV, "vk": _abi.CGDR_STATE_VK}


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _aligned(t: torch.Tensor, row_bytes_align: int) -> bool:
    es = t.element_size()
    return (t.data_ptr() % row_bytes_align == 0
            and all((s * es) % row_bytes_align == 0 for s in t.stride()[:-1]))


def _prep_input(t: torch.Tensor, name: str, align: int) -> torch.Tensor:
    """Innermost dim contiguous and rows aligned for the DMA path; copy only if needed."""
    if t.stride(-1) != 1 or not _aligned(t, align):
        t = t.contiguous()
        if not _aligned(t, align):
            t = t.clone()
    return t


def _host_to_device(vals, device) -> torch.Tensor:
    """int64 values from the host to the device through pinned memory, without blocking the host:
    a copy from pageable memory would wait for the stream's earlier work, leaving the GPU idle
    while the host prepares the next call.  (torch keeps the pinned block until the copy is done.)"""
    host = torch.as_tensor(vals, dtype=torch.int64)
    if device.type != "cuda":
        return host.to(device)
    return host.pin_memory().to(device, non_blocking=True)


def _varlen_meta(cu_seqlens: torch.Tensor, T: int, chunk_indices, chunk_offsets, device,
                 want_offsets: bool = True):
    """Host validation of cu_seqlens (``code/tests/golden/generate_golden.py:326-339``,
    ``code/op_host/chunk_gated_delta_rule_fwd_h_infershape.cpp:240-275``) and the device
    chunk offsets.  Returns (N, NT, cu_device_int64, chunk_offsets_device_int64 or None).
    A cu_seqlens on the host is read without a device round trip; one on the device is copied
    to the host once (NT, the leading dimension of h, depends on it)."""
    if cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2:
        raise ValueError("cu_seqlens must be one-dimensional with at least two entries")
    cu_host = [int(x) for x in cu_seqlens.detach().to("cpu", torch.int64).tolist()]
    if cu_host[0] != 0:
        raise ValueError("cu_seqlens must start at zero")
    if cu_host[-1] != T:
        raise ValueError(f"cu_seqlens[-1] must equal T={T}, got {cu_host[-1]}")
    if any(b < a for a, b in zip(cu_host, cu_host[1:])):
        raise ValueError("cu_seqlens must be non-decreasing")
    offs = _abi.prepare_chunk_offsets(cu_host, CHUNK_SIZE)
    N, NT = len(cu_host) - 1, offs[-1]
    if chunk_indices is not None:
        ci = chunk_indices.detach().to("cpu", torch.int64)
        expect = _abi.prepare_chunk_indices(cu_host, CHUNK_SIZE)
        if ci.dim() != 2 or ci.shape[1] != 2 or [tuple(r) for r in ci.tolist()] != expect:
            raise ValueError("chunk_indices does not match cu_seqlens")
    if chunk_offsets is not None:
        co = [int(x) for x in chunk_offsets.detach().to("cpu", torch.int64).tolist()]
        if co[: N + 1] != offs:
            raise ValueError("chunk_offsets does not match cu_seqlens")
    if cu_seqlens.device == device and cu_seqlens.dtype == torch.int64 and cu_seqlens.is_contiguous():
        cu_dev = cu_seqlens
    else:
        cu_dev = _host_to_device(cu_host, device)
    offs_dev = _host_to_device(offs, device) if want_offsets else None
    return N, NT, cu_dev, offs_dev


def _launch(k, w, u, g, h0, cu_dev, offs_dev, h, v_new, final, B, T, H, Hg, K, V, N, NT,
            strides: dict, numerics: str = "default", tuning: dict | None = None,
            state_layout: str = "kv") -> None:
    a = _abi.FwdHArgs()
    a.state_layout = _STATE_LAYOUTS[state_layout]
    if tuning:
        t = _abi.make_tuning(**tuning)
        a.tuning = ctypes.pointer(t)
    a.k, a.w, a.u = k.data_ptr(), w.data_ptr(), u.data_ptr()
    a.g = _ptr(g)
    a.initial_state = _ptr(h0)
    a.cu_seqlens = _ptr(cu_dev)
    a.chunk_offsets = _ptr(offs_dev)
    a.h, a.v_new, a.final_state = h.data_ptr(), _ptr(v_new), _ptr(final)
    a.B, a.T, a.H, a.Hg, a.K, a.V, a.N, a.NT = B, T, H, Hg, K, V, N, NT
    a.chunk_size = CHUNK_SIZE
    a.in_dtype = _DTYPES[k.dtype]
    a.h0_dtype = _DTYPES[h0.dtype] if h0 is not None else _abi.CGDR_F32
    a.final_dtype = _DTYPES[final.dtype] if final is not None else _abi.CGDR_F32
    if numerics not in _NUMERICS:
        raise ValueError(f"numerics must be one of {sorted(_NUMERICS)}, got {numerics!r}")
    a.numerics = _NUMERICS[numerics]
    for name in ("stride_k", "stride_w", "stride_u", "stride_g", "stride_h", "stride_v",
                 "stride_h0", "stride_final"):
        vals = strides.get(name)
        if vals is not None:
            getattr(a, name)[:] = list(vals)
    if T == 0:
        return
    nws = _abi.workspace_size(a)
    ws = torch.empty(nws, dtype=torch.uint8, device=k.device) if nws > 0 else None
    _abi.launch(a, torch.cuda.current_stream(k.device).cuda_stream,
                0 if ws is None else ws.data_ptr(), nws)


def _check_common(k, w, u, g, initial_state, chunk_size):
    if chunk_size != CHUNK_SIZE:
        raise ValueError(f"chunk_size must be {CHUNK_SIZE}, but got {chunk_size}")
    if k.dim() != 4 or w.dim() != 4 or u.dim() != 4:
        raise ValueError("k, w and u must have rank 4")
    if g is not None and g.dim() != 3:
        raise ValueError("g must have rank 3")
    if initial_state is not None and initial_state.dim() != 4:
        raise ValueError("initial_state must have rank 4")
    if k.dtype not in _DTYPES or w.dtype != k.dtype or u.dtype != k.dtype:
        raise TypeError(f"k, w, u must share dtype bfloat16 or float32 (got {k.dtype}, {w.dtype}, {u.dtype})")
    for t, name in ((k, "k"), (w, "w"), (u, "u")):
        if t.device.type != "cuda":
            raise ValueError(f"{name} must be a HIP device tensor (got {t.device})")
    if not (k.device == w.device == u.device):
        raise ValueError("k, w and u must be on the same device")


def chunk_gated_delta_rule_fwd_h(
    k: torch.Tensor,
    w: torch.Tensor,
    u: torch.Tensor,
    g: torch.Tensor | None = None,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    chunk_size: int = CHUNK_SIZE,
    save_new_value: bool = True,
    cu_seqlens: torch.LongTensor | None = None,
    chunk_indices: torch.Tensor | None = None,
    chunk_offsets: torch.Tensor | None = None,
    final_state_dtype: torch.dtype = torch.float32,
    numerics: str = "default",
    tuning: dict | None = None,
    state_layout: str = "kv",
):
    """``(h, v_new, final_state)`` for token-major inputs; see the module docstring.
    ``state_layout="vk"`` takes ``initial_state`` and returns ``final_state`` as ``[N,H,V,K]``
    blocks (the full operator's ``[B,Nv,Dv,Dk]`` state,
    ``ref/chunk_gated_delta_rule/tests/pytest/chunk_gated_delta_rule_benchmark.py:184``); h stays
    ``[B,NT,H,K,V]``.
    ``numerics="contest"`` selects the contest reference's rounding model (bf16 inputs).
    ``tuning`` overrides fields of the launch plan (``cgdr_fwd_h_tuning``: v_tile, helpers,
    load_waves, stages, ...); outputs do not depend on it.

    ``g`` and ``initial_state`` may be any floating dtype; g is used in fp32 and
    initial_state in fp32 or bf16 (other dtypes are upcast to fp32).
    """
    _check_common(k, w, u, g, initial_state, chunk_size)
    if state_layout not in _STATE_LAYOUTS:
        raise ValueError(f"state_layout must be one of {sorted(_STATE_LAYOUTS)}, got {state_layout!r}")
    B, T, Hg, K = k.shape
    H, V = u.shape[-2], u.shape[-1]
    if tuple(w.shape) != (B, T, H, K):
        raise ValueError(f"w must have shape [B,T,H,K]={[B, T, H, K]}, got {list(w.shape)}")
    if tuple(u.shape[:2]) != (B, T):
        raise ValueError(f"u must have shape [B,T,H,V], got {list(u.shape)}")
    if H % Hg != 0:
        raise ValueError(f"H must be divisible by Hg: H={H}, Hg={Hg}")
    if g is not None:
        if tuple(g.shape) != (B, T, H):
            raise ValueError(f"g must have shape [B,T,H]={[B, T, H]}, got {list(g.shape)}")
        # any strides: the library reads g in place when its token stride is 1 (e.g. a
        # head-major buffer) and copies it head-major into the workspace otherwise
        g = g.float() if g.dtype != torch.float32 else g
    dev = k.device
    if cu_seqlens is None:
        if chunk_indices is not None or chunk_offsets is not None:
            raise ValueError("chunk_indices/chunk_offsets require cu_seqlens")
        N, NT, cu_dev, offs_dev = B, (T + CHUNK_SIZE - 1) // CHUNK_SIZE, None, None
    else:
        if B != 1:
            raise ValueError(f"cu_seqlens requires B == 1, got B={B}")
        N, NT, cu_dev, offs_dev = _varlen_meta(cu_seqlens, T, chunk_indices, chunk_offsets, dev)
    h0 = None
    if initial_state is not None:
        want = (N, H, K, V) if state_layout == "kv" else (N, H, V, K)
        if tuple(initial_state.shape) != want:
            raise ValueError(f"initial_state must have shape {list(want)} ({state_layout}), got {list(initial_state.shape)}")
        h0 = initial_state if initial_state.dtype in _DTYPES else initial_state.float()
        h0 = h0.contiguous()
    # 16-byte rows for the direct-to-LDS (bf16) and vector (fp32) loads; with K or V not a
    # multiple of 16 the library copies k, w and u into padded rows itself
    align = 16 if K % 16 == 0 and V % 16 == 0 else k.element_size()
    k, w, u = _prep_input(k, "k", align), _prep_input(w, "w", align), _prep_input(u, "u", align)

    h = k.new_empty(B, NT, H, K, V)
    v_new = torch.empty(B, T, H, V, dtype=u.dtype, device=dev) if save_new_value else None
    fshape = (N, H, K, V) if state_layout == "kv" else (N, H, V, K)
    final = (torch.empty(*fshape, dtype=final_state_dtype, device=dev)
             if output_final_state else None)
    if final is not None and final.dtype not in _DTYPES:
        raise TypeError("final_state_dtype must be float32 or bfloat16")
    strides = dict(
        stride_k=k.stride()[:3], stride_w=w.stride()[:3], stride_u=u.stride()[:3],
        stride_g=g.stride() if g is not None else None,
        stride_h=h.stride()[:3], stride_v=v_new.stride()[:3] if v_new is not None else None,
        stride_h0=h0.stride()[:2] if h0 is not None else None,
        stride_final=final.stride()[:2] if final is not None else None,
    )
    _launch(k, w, u, g, h0, cu_dev, offs_dev, h, v_new, final, B, T, H, Hg, K, V, N, NT, strides, numerics,
            tuning, state_layout)
    return h, v_new, final


def run(k, w, u, g, initial_state, cu_seqlens, chunk_indices, chunk_size=CHUNK_SIZE, numerics="default"):
    """Contest reference signature (``docs/problem.txt:81``), head-major layouts.

    k ``[B,T,HK,K]``, w ``[B,HV,T,K]``, u ``[B,HV,T,V]``, g ``[B,HV,T]``, initial_state
    ``[N,HV,K,V]`` (or None) -> ``(S [B,HV,NT,K,V], v [B,HV,T,V], final_state [N,HV,K,V])``.
    By default the state recurrence keeps fp32 state (the Triton rounding model);
    ``numerics="contest"`` reproduces run()'s own casts (bf16 state, saturating fp16).  ``S``
    is k's dtype and ``final_state`` u's dtype as in the reference's output declaration.
    """
    _check_common(k, w, u, g, initial_state, chunk_size)
    B, T, Hg, K = k.shape
    H, V = u.shape[1], u.shape[3]
    if tuple(w.shape) != (B, H, T, K) or tuple(u.shape) != (B, H, T, V):
        raise ValueError("w must be [B,HV,T,K] and u [B,HV,T,V]")
    if g is not None and tuple(g.shape) != (B, H, T):
        raise ValueError("g must be [B,HV,T]")
    if H % Hg != 0:
        raise ValueError(f"HV must be divisible by HK: HV={H}, HK={Hg}")
    if g is not None and (g.dtype != torch.float32 or g.stride(-1) != 1):
        g = g.float().contiguous()
    dev = k.device
    if cu_seqlens is None:
        N, NT, cu_dev, offs_dev = B, (T + CHUNK_SIZE - 1) // CHUNK_SIZE, None, None
    else:
        if B != 1:
            raise ValueError("cu_seqlens requires B == 1")
        N, NT, cu_dev, offs_dev = _varlen_meta(cu_seqlens, T, chunk_indices, None, dev)
    h0 = None
    if initial_state is not None:
        h0 = initial_state.reshape(N, H, K, V)
        h0 = (h0 if h0.dtype in _DTYPES else h0.float()).contiguous()
    # 16-byte rows for the direct-to-LDS (bf16) and vector (fp32) loads; with K or V not a
    # multiple of 16 the library copies k, w and u into padded rows itself
    align = 16 if K % 16 == 0 and V % 16 == 0 else k.element_size()
    k, w, u = _prep_input(k, "k", align), _prep_input(w, "w", align), _prep_input(u, "u", align)
    S = torch.empty(B, H, NT, K, V, dtype=k.dtype, device=dev)
    v = torch.empty(B, H, T, V, dtype=u.dtype, device=dev)
    final = torch.empty(N, H, K, V, dtype=u.dtype, device=dev)
    # head-major tensors expressed as (b, t, head) strides
    strides = dict(
        stride_k=k.stride()[:3],
        stride_w=(w.stride(0), w.stride(2), w.stride(1)),
        stride_u=(u.stride(0), u.stride(2), u.stride(1)),
        stride_g=(g.stride(0), g.stride(2), g.stride(1)) if g is not None else None,
        stride_h=(S.stride(0), S.stride(2), S.stride(1)),
        stride_v=(v.stride(0), v.stride(2), v.stride(1)),
        stride_h0=h0.stride()[:2] if h0 is not None else None,
        stride_final=final.stride()[:2],
    )
    _launch(k, w, u, g, h0, cu_dev, offs_dev, S, v, final, B, T, H, Hg, K, V, N, NT, strides, numerics)
    return S, v, final


def plan(k: torch.Tensor, u: torch.Tensor, H: int | None = None, N: int | None = None,
         cu_seqlens_len: int | None = None, numerics: str = "default", NT: int | None = None,
         tuning: dict | None = None) -> dict:
    """Launch plan the library picks for token-major inputs of these shapes (host only).
    ``NT`` is the real chunk count of a packed batch (default ceil(T/64), a lower bound)."""
    B, T, Hg, K = k.shape
    H = u.shape[-2] if H is None else H
    V = u.shape[-1]
    a = _abi.FwdHArgs()
    fake = 1 << 20
    a.k = a.w = a.u = a.h = fake
    a.B, a.T, a.H, a.Hg, a.K, a.V = B, T, H, Hg, K, V
    a.N = B if N is None else N
    a.NT = (T + CHUNK_SIZE - 1) // CHUNK_SIZE if NT is None else NT
    if tuning:
        t = _abi.make_tuning(**tuning)
        a.tuning = ctypes.pointer(t)
    if cu_seqlens_len is not None:
        a.cu_seqlens = fake
        a.N = cu_seqlens_len - 1
    a.chunk_size = CHUNK_SIZE
    a.in_dtype = _DTYPES[k.dtype]
    a.stride_k[:] = [T * Hg * K, Hg * K, K]
    a.stride_w[:] = [T * H * K, H * K, K]
    a.stride_u[:] = [T * H * V, H * V, V]
    NT = a.NT
    a.stride_h[:] = [NT * H * K * V, H * K * V, K * V]
    a.numerics = _NUMERICS[numerics]
    p = _abi.get_plan(a)
    return {f: getattr(p, f) for f, _ in _abi.FwdHPlan._fields_}
