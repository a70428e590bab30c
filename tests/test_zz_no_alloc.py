"""cgdr_fwd_h_launch_no_alloc (the entry point that allocates nothing: its workspace is a static
per-GPU device array) against cgdr_fwd_h_launch with a caller-allocated workspace, bit for bit.

Four calls in a row, each smaller than the one before, so each starts from what the last left
in the shared scratch: token-major g (the head-major relayout of g lives in the scratch), helper
workgroups (their progress counters), contest numerics (the per-head flags), and a head dim
that is not a multiple of 16 (the padded copies), in bf16 and in fp32.  The
oversize rejection is checked on the host, before anything touches a GPU."""

import ctypes

import numpy as np
import pytest
import torch

from cgdr_amd import _abi
from gpu_util import abi_call, dev_inputs
from oracle import cgdr_oracle as O


def _inp(seed, T, H, K=128, V=128, cu=None, dtype="bf16"):
    print(f"[no_alloc] seed={seed} T={T} H={H} K={K} V={V} varlen={cu is not None} {dtype}", flush=True)
    return O.make_inputs(seed, 1, T, H, K, V, dtype=dtype, gate="logsigmoid", gate_shift=4.0, with_h0=True,
                         cu_seqlens=cu, profile="wy")


def _same(a, b):
    for x, y in zip(a, b):
        if x is None:
            assert y is None
            continue
        assert torch.equal(x.view(torch.int16) if x.dtype == torch.bfloat16 else x.view(torch.int32),
                           y.view(torch.int16) if y.dtype == torch.bfloat16 else y.view(torch.int32))


@pytest.mark.gpu
def test_no_alloc_matches_workspace_launch(dev):
    # call 1: 8 heads x 4 V-tiles of 32 columns with helpers (progress counters), token-major g
    # (its relayout: 256 KiB of the scratch); call 2: a smaller packed batch in contest numerics
    # call 3: K = V = 100, which runs on padded copies held in the scratch too; call 4: the same
    # in fp32 (fp32 kernel, all four waves computing with the state rows split four ways)
    cases = [(_inp(1, 8192, 8), dict(helpers=1, v_tile=32), 0, torch.bfloat16),
             (_inp(2, 1000, 4, cu=np.array([0, 300, 301, 1000], np.int64)), None, 1, torch.bfloat16),
             (_inp(3, 300, 2, K=100, V=100), None, 0, torch.bfloat16),
             (_inp(4, 200, 2, K=100, V=100, dtype="f32"), None, 0, torch.float32)]
    for inp, tuning, numerics, dt in cases:
        d = dev_inputs(inp, dt, dev)
        assert d["g"].stride(1) != 1   # token-major g: the workspace holds its relayout
        ref = abi_call(d, tuning=tuning, numerics=numerics)
        got = abi_call(d, tuning=tuning, numerics=numerics, no_alloc=True)
        _same(ref, got)
        again = abi_call(d, tuning=tuning, numerics=numerics, no_alloc=True)
        _same(ref, again)


def _graph_args(d, h, v, f, tuning, numerics):
    """Launch arguments of one FwdH call into preallocated outputs (so that a captured graph
    allocates nothing), fixed-length batch."""
    k, w, u, g, h0 = d["k"], d["w"], d["u"], d["g"], d["initial_state"]
    B, T, Hg, K = k.shape
    H, V = u.shape[2], u.shape[3]
    a = _abi.FwdHArgs()
    a.k, a.w, a.u, a.g = k.data_ptr(), w.data_ptr(), u.data_ptr(), g.data_ptr()
    a.initial_state = h0.data_ptr()
    a.h, a.v_new, a.final_state = h.data_ptr(), v.data_ptr(), f.data_ptr()
    a.B, a.T, a.H, a.Hg, a.K, a.V, a.N, a.NT = B, T, H, Hg, K, V, B, h.shape[1]
    a.chunk_size = 64
    a.in_dtype = _abi.CGDR_BF16
    a.h0_dtype = _abi.CGDR_F32 if h0.dtype == torch.float32 else _abi.CGDR_BF16
    a.final_dtype = _abi.CGDR_F32 if f.dtype == torch.float32 else _abi.CGDR_BF16
    a.stride_k[:] = list(k.stride()[:3])
    a.stride_w[:] = list(w.stride()[:3])
    a.stride_u[:] = list(u.stride()[:3])
    a.stride_g[:] = list(g.stride())
    a.stride_h[:] = list(h.stride()[:3])
    a.stride_v[:] = list(v.stride()[:3])
    a.stride_h0[:] = list(h0.stride()[:2])
    a.stride_final[:] = list(f.stride()[:2])
    a.numerics = numerics
    t = None
    if tuning:
        t = _abi.make_tuning(**tuning)
        a.tuning = ctypes.pointer(t)
    return a, t


@pytest.mark.gpu
@pytest.mark.parametrize("numerics", [0, 1])
def test_no_alloc_in_captured_graph(dev, numerics):
    """The entry point that allocates nothing, captured in a HIP graph and replayed three times
    (outputs refilled with NaN and an eager call on other buffers between replays): every replay
    equals the eager call bit for bit.  A replay reuses the launch's epoch, so the helpers read
    the previous replay's progress counters and stop early, and contest flags raised by an
    earlier replay send those heads through the full pass again; neither changes a result."""
    inp = _inp(5, 2048, 8)
    d = dev_inputs(inp, torch.bfloat16, dev)
    B, T, H, K, V = 1, 2048, 8, 128, 128
    fdt = torch.float32 if numerics == 0 else torch.bfloat16
    h = torch.empty(B, T // 64, H, K, V, dtype=torch.bfloat16, device=dev)
    v = torch.empty(B, T, H, V, dtype=torch.bfloat16, device=dev)
    f = torch.empty(B, H, K, V, dtype=fdt, device=dev)
    if numerics == 1:
        d["initial_state"] = d["initial_state"].to(torch.bfloat16)
    tuning = dict(helpers=1, v_tile=32)
    a, _keep = _graph_args(d, h, v, f, tuning, numerics)

    def refill():
        for x in (h, v, f):
            x.fill_(float("nan"))

    refill()
    _abi.launch_no_alloc(a, torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    ref = (h.clone(), v.clone(), f.clone())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _abi.launch_no_alloc(a, torch.cuda.current_stream(dev).cuda_stream)
    torch.cuda.synchronize()
    other = abi_call(d, tuning=tuning, numerics=numerics, final_dtype=fdt)
    for rep in range(3):
        print(f"[no_alloc graph] numerics={numerics} replay {rep}", flush=True)
        refill()
        graph.replay()
        torch.cuda.synchronize()
        _same(ref, (h, v, f))
        _same(ref, other)
        other = abi_call(d, tuning=tuning, numerics=numerics, final_dtype=fdt)


def test_no_alloc_rejects_oversize_scratch():
    """A token-major g of B*H*T*4 bytes beyond the 16 MiB scratch is refused with a message,
    before any device call (no GPU needed)."""
    a = _abi.FwdHArgs()
    fake = 1 << 24
    a.k = a.w = a.u = a.h = a.g = fake
    B, T, H, K, V = 1, 1 << 17, 64, 64, 64          # g relayout: 32 MiB
    a.B, a.T, a.H, a.Hg, a.K, a.V, a.N, a.NT = B, T, H, H, K, V, B, T // 64
    a.chunk_size = 64
    a.in_dtype = _abi.CGDR_BF16
    a.stride_k[:] = [T * H * K, H * K, K]
    a.stride_w[:] = [T * H * K, H * K, K]
    a.stride_u[:] = [T * H * V, H * V, V]
    a.stride_g[:] = [T * H, H, 1]
    a.stride_h[:] = [(T // 64) * H * K * V, H * K * V, K * V]
    n = ctypes.c_size_t(0)
    assert _abi.load().cgdr_fwd_h_workspace_size(ctypes.byref(a), ctypes.byref(n)) == _abi.CGDR_OK
    assert n.value > _abi.NO_ALLOC_SCRATCH_BYTES
    st = _abi.load().cgdr_fwd_h_launch_no_alloc(ctypes.byref(a), None)
    assert st == _abi.CGDR_ERR_UNSUPPORTED
    assert "scratch" in _abi.last_error()
