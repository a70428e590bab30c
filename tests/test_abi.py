"""C ABI checks that need no GPU: the library loads, exports what include/cgdr_fwd_h.h
declares, the ctypes mirror matches the C struct layout, and host-side validation returns
the documented status codes (mirroring the reference's infershape rejection cases,
code/tests/ut/op_host/test_chunk_gated_delta_rule_fwd_h_infershape.cpp:137-223)."""

import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from cgdr_amd import _abi
from oracle import cgdr_oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "cgdr_fwd_h.h")


@pytest.fixture(scope="module")
def lib():
    return _abi.load()


def test_exports_every_declared_symbol(lib):
    inc = os.path.dirname(HEADER)
    text = "".join(open(os.path.join(inc, f)).read() for f in sorted(os.listdir(inc)) if f.endswith(".h"))
    # function declarations: a return type at the start of a line, then the name and "("
    declared = set(re.findall(r"^(?:cgdr_status|const char\s*\*|int)\s+(cgdr_[a-z0-9_]+)\s*\(", text, re.M))
    assert declared == set(_abi.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.cgdr_abi_version() == _abi.ABI_VERSION


def test_struct_layout_matches_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(r'''
#include <stdio.h>
#include <stddef.h>
#include "cgdr_fwd_h.h"
#include "cgdr_chunk_o.h"
#include "cgdr_wy.h"
#define F(s, f) printf(#s "." #f " %zu\n", offsetof(s, f))
int main(void) {
  printf("args %zu\nplan %zu\nochunk %zu\nwy %zu\n", sizeof(cgdr_fwd_h_args), sizeof(cgdr_fwd_h_plan),
         sizeof(cgdr_chunk_o_args), sizeof(cgdr_wy_args));
  F(cgdr_wy_args, g_cumsum); F(cgdr_wy_args, chunk_size); F(cgdr_wy_args, beta_dtype);
  F(cgdr_wy_args, stride_k); F(cgdr_wy_args, stride_g_cumsum);
  F(cgdr_chunk_o_args, o); F(cgdr_chunk_o_args, chunk_size); F(cgdr_chunk_o_args, scale);
  F(cgdr_chunk_o_args, in_dtype); F(cgdr_chunk_o_args, stride_q); F(cgdr_chunk_o_args, stride_o);
  F(cgdr_fwd_h_args, final_state); F(cgdr_fwd_h_args, B); F(cgdr_fwd_h_args, chunk_size);
  F(cgdr_fwd_h_args, in_dtype); F(cgdr_fwd_h_args, numerics); F(cgdr_fwd_h_args, stride_k);
  F(cgdr_fwd_h_args, stride_h0); F(cgdr_fwd_h_args, stride_final); F(cgdr_fwd_h_args, tuning);
  F(cgdr_fwd_h_args, state_layout); F(cgdr_fwd_h_args, reserved);
  F(cgdr_fwd_h_plan, lds_bytes); F(cgdr_fwd_h_plan, workgroups); F(cgdr_fwd_h_plan, helpers);
  F(cgdr_fwd_h_plan, xcd_count); F(cgdr_fwd_h_plan, row_split);
  F(cgdr_fwd_h_tuning, helpers); F(cgdr_fwd_h_tuning, cu_count); F(cgdr_fwd_h_tuning, row_split);
  printf("tuning %zu\n", sizeof(cgdr_fwd_h_tuning));
  return 0;
}''')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)],
                   check=True)
    out = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                              check=True).stdout.split("\n") if line)
    assert int(out["args"]) == ctypes.sizeof(_abi.FwdHArgs)
    assert int(out["plan"]) == ctypes.sizeof(_abi.FwdHPlan)
    assert int(out["ochunk"]) == ctypes.sizeof(_abi.ChunkOArgs)
    assert int(out["wy"]) == ctypes.sizeof(_abi.WyArgs)
    assert int(out["tuning"]) == ctypes.sizeof(_abi.FwdHTuning)
    classes = {"cgdr_fwd_h_args": _abi.FwdHArgs, "cgdr_fwd_h_plan": _abi.FwdHPlan, "cgdr_chunk_o_args": _abi.ChunkOArgs,
               "cgdr_wy_args": _abi.WyArgs, "cgdr_fwd_h_tuning": _abi.FwdHTuning}
    for key, val in out.items():
        if "." in key:
            s, f = key.split(".")
            cls = classes[s]
            assert getattr(cls, f).offset == int(val), key


def _args(B=1, T=256, H=4, Hg=2, K=128, V=128, dtype=_abi.CGDR_BF16, varlen=None, tuning=None):
    a = _abi.FwdHArgs()
    if tuning is not None:
        a._keep = _abi.make_tuning(**tuning)
        a.tuning = ctypes.pointer(a._keep)
    fake = 1 << 24     # aligned, never dereferenced: validation is host-only
    a.k = a.w = a.u = a.h = fake
    a.B, a.T, a.H, a.Hg, a.K, a.V = B, T, H, Hg, K, V
    a.chunk_size = 64
    a.in_dtype = dtype
    if varlen is None:
        a.N, a.NT = B, (T + 63) // 64
    else:
        a.cu_seqlens = fake
        a.N = len(varlen) - 1
        a.NT = int(O.prepare_chunk_offsets(np.asarray(varlen))[-1])
    a.stride_k[:] = [T * Hg * K, Hg * K, K]
    a.stride_w[:] = [T * H * K, H * K, K]
    a.stride_u[:] = [T * H * V, H * V, V]
    a.stride_h[:] = [a.NT * H * K * V, H * K * V, K * V]
    return a


def _status(a):
    n = ctypes.c_size_t(123)
    return _abi.load().cgdr_fwd_h_workspace_size(ctypes.byref(a), ctypes.byref(n)), n.value


def test_valid_args_need_no_workspace(lib):
    # no g and no helper workgroups (12 tasks: not a multiple of the 8 XCDs)
    assert _status(_args(H=3, Hg=1)) == (_abi.CGDR_OK, 0)
    assert _status(_args(varlen=[0, 61, 64], T=64))[0] == _abi.CGDR_OK
    assert _status(_args(dtype=_abi.CGDR_F32, K=64, V=64)) == (_abi.CGDR_OK, 0)


def _with_g(a, token_major=True):
    a.g = 1 << 24
    B, T, H = a.B, a.T, a.H
    a.stride_g[:] = [T * H, H, 1] if token_major else [H * T, 1, T]
    return a


def test_token_major_g_needs_head_major_workspace(lib):
    # a token-major g is copied head-major into the workspace (B*H*T floats); a head-major g
    # (token stride 1) is read in place
    # (3 heads: 12 tasks, no helper workgroups; the copy is rounded up to 256 bytes)
    assert _status(_with_g(_args(B=1, T=256, H=3, Hg=1))) == (_abi.CGDR_OK, 3 * 256 * 4)
    assert _status(_with_g(_args(B=1, T=200, H=3, Hg=1))) == (_abi.CGDR_OK, 2560)
    assert _status(_with_g(_args(B=1, T=200, H=3, Hg=1), token_major=False)) == (_abi.CGDR_OK, 0)
    # varlen, 2 sequences x 3 heads: one chunk per sequence, too short for helper workgroups
    assert _status(_with_g(_args(varlen=[0, 61, 64], T=64, H=3, Hg=1)))[1] == 3 * 64 * 4
    # 2 sequences of 96 and 100 chunks x 3 heads x 4 V-tiles = 24 tasks: helpers, 24 progress lines
    assert _status(_mi355x(_with_g(_args(varlen=[0, 6144, 12544], T=12544, H=3, Hg=1))))[1] == \
        3 * 12544 * 4 + 24 * 128


def test_contest_numerics_need_one_flag_per_head(lib):
    # contest numerics: one int32 flag per (sequence, head) for the full pass, after the
    # progress lines of any helper workgroups
    a = _args(H=3, Hg=1)   # 12 tasks: no helper workgroups
    a.numerics = _abi.CGDR_NUMERICS_CONTEST
    assert _status(a) == (_abi.CGDR_OK, 3 * 4)
    a = _args(varlen=[0, 61, 64], T=64, H=3, Hg=1)
    a.numerics = _abi.CGDR_NUMERICS_CONTEST
    assert _status(a)[1] == 2 * 3 * 4
    a = _args(varlen=[0, 6144, 12544], T=12544, H=3, Hg=1)
    a.numerics = _abi.CGDR_NUMERICS_CONTEST
    assert _status(a)[1] == 24 * 128 + 2 * 3 * 4


def test_launch_rejects_missing_or_short_workspace(lib):
    # host-side check before anything is enqueued, so it runs without a GPU
    a = _with_g(_args())
    need = _status(a)[1]
    assert lib.cgdr_fwd_h_launch(ctypes.byref(a), None, 0, None) == _abi.CGDR_ERR_INVALID
    assert "workspace" in _abi.last_error()
    assert lib.cgdr_fwd_h_launch(ctypes.byref(a), ctypes.c_void_p(1 << 24), need - 4, None) == _abi.CGDR_ERR_INVALID
    assert lib.cgdr_fwd_h_launch(ctypes.byref(a), ctypes.c_void_p((1 << 24) + 4), need, None) == _abi.CGDR_ERR_INVALID
    assert "aligned" in _abi.last_error()


@pytest.mark.parametrize("mutate,expect", [
    (lambda a: setattr(a, "k", None), _abi.CGDR_ERR_NULLPTR),
    (lambda a: setattr(a, "w", None), _abi.CGDR_ERR_NULLPTR),
    (lambda a: setattr(a, "u", None), _abi.CGDR_ERR_NULLPTR),
    (lambda a: setattr(a, "h", None), _abi.CGDR_ERR_NULLPTR),
    (lambda a: setattr(a, "chunk_size", 32), _abi.CGDR_ERR_UNSUPPORTED),
    (lambda a: setattr(a, "Hg", 3), _abi.CGDR_ERR_INVALID),          # H % Hg != 0
    (lambda a: setattr(a, "T", 0), _abi.CGDR_ERR_INVALID),
    (lambda a: setattr(a, "NT", 5), _abi.CGDR_ERR_INVALID),
    (lambda a: setattr(a, "N", 2), _abi.CGDR_ERR_INVALID),
    (lambda a: setattr(a, "K", 300), _abi.CGDR_ERR_INVALID),         # K > 256
    (lambda a: setattr(a, "K", 16), _abi.CGDR_ERR_UNSUPPORTED),    # below 32, as the reference
    (lambda a: setattr(a, "K", 20), _abi.CGDR_ERR_UNSUPPORTED),
    (lambda a: setattr(a, "in_dtype", 7), _abi.CGDR_ERR_INVALID),
    (lambda a: setattr(a, "state_layout", 2), _abi.CGDR_ERR_INVALID),
    (lambda a: setattr(a, "reserved", 1), _abi.CGDR_ERR_INVALID),
    (lambda a: setattr(a, "k", (1 << 24) + 8), _abi.CGDR_ERR_UNSUPPORTED),   # DMA needs 16B rows
    (lambda a: setattr(a, "chunk_offsets", 1 << 24), _abi.CGDR_ERR_INVALID),  # without cu_seqlens
])
def test_rejections(lib, mutate, expect):
    a = _args()
    mutate(a)
    st, _ = _status(a)
    assert st == expect, (_abi.status_string(st), _abi.last_error())
    assert _abi.last_error()


def test_varlen_rejections(lib):
    a = _args(varlen=[0, 61, 64], T=64)
    a.B = 2
    assert _status(a)[0] == _abi.CGDR_ERR_INVALID        # varlen needs B == 1
    a = _args(varlen=[0, 61, 64], T=64)
    a.NT = 3                                              # impossible for T=64, N=2
    assert _status(a)[0] == _abi.CGDR_ERR_INVALID
    assert "impossible" in _abi.last_error()


def test_null_pointers_to_entry_points(lib):
    n = ctypes.c_size_t(0)
    assert lib.cgdr_fwd_h_workspace_size(None, ctypes.byref(n)) == _abi.CGDR_ERR_NULLPTR
    assert lib.cgdr_fwd_h_workspace_size(ctypes.byref(_args()), None) == _abi.CGDR_ERR_NULLPTR
    assert lib.cgdr_fwd_h_get_plan(ctypes.byref(_args()), None) == _abi.CGDR_ERR_NULLPTR


def test_status_strings(lib):
    assert _abi.status_string(_abi.CGDR_OK) == "CGDR_OK"
    assert _abi.status_string(_abi.CGDR_ERR_LAUNCH) == "CGDR_ERR_LAUNCH"


@pytest.mark.parametrize("cu", [[0, 61, 64], [0, 1], [0, 63, 127, 192, 1000], [0, 64, 128]])
def test_host_chunk_metadata_matches_oracle(lib, cu):
    assert _abi.prepare_chunk_offsets(cu) == O.prepare_chunk_offsets(np.asarray(cu)).tolist()
    assert _abi.prepare_chunk_indices(cu) == [tuple(r) for r in O.prepare_chunk_indices(np.asarray(cu)).tolist()]


def test_host_chunk_metadata_rejects_bad_cu(lib):
    with pytest.raises(_abi.CgdrError):
        _abi.prepare_chunk_offsets([1, 5])
    with pytest.raises(_abi.CgdrError):
        _abi.prepare_chunk_offsets([0, 5, 3])


def _mi355x(a, **kw):
    """Plan as for MI355X (256 CUs, 8 XCDs), whatever device this host has."""
    t = _abi.make_tuning(cu_count=256, xcd_count=8, **kw)
    a.tuning = ctypes.pointer(t)
    a._keep = t
    return a


def test_plan_headline_fills_the_chip(lib):
    # 32 heads x 4 V-tiles of 32 columns, each task with an L2-prefetch helper workgroup on
    # its XCD: 256 workgroups, one per CU
    p = _abi.get_plan(_mi355x(_args(B=1, T=32768, H=32, Hg=32, K=128, V=128)))
    assert p.cu_count == 256 and p.xcd_count == 8 and p.helpers == 1
    assert p.kernel == 0 and p.v_tile == 32 and p.workgroups == 256
    assert p.lds_bytes <= 160 * 1024
    # helpers need the doubled grid to fit the chip and tasks in multiples of 8 (per XCD);
    # without them, 32-column tiles when 16-column ones would take more than one round of
    # the chip at one task workgroup per CU
    p = _abi.get_plan(_mi355x(_args(B=2, T=4096, H=32, Hg=32, K=128, V=128)))
    assert p.v_tile == 32 and p.workgroups == 2 * 32 * 4
    p = _abi.get_plan(_mi355x(_args(B=1, T=8192, H=16, Hg=16, K=128, V=128)))   # 128 tasks of 16 columns
    assert p.v_tile == 32 and p.workgroups == 2 * 16 * 4                         # helper mode
    p = _abi.get_plan(_mi355x(_args(B=1, T=8192, H=6, Hg=6, K=128, V=128)))
    assert p.workgroups == 6 * 8
    # sequences under 96 chunks: no helpers, 16-column tiles while they fit one round
    p = _abi.get_plan(_mi355x(_args(B=1, T=4096, H=16, Hg=16, K=128, V=128)))
    assert p.v_tile == 16 and p.workgroups == 16 * 8


@pytest.mark.parametrize("B,T,H,K,V,vt,rs", [
    (2, 2048, 16, 128, 128, 16, 4),    # 256 tasks of 16 columns: one round, all waves on rows
    (4, 4096, 32, 128, 128, 64, 1),    # 1,024 / 512 / 256 tasks: one round of 64 columns wins
    (4, 2048, 64, 128, 128, 64, 1),
    (3, 2048, 16, 128, 128, 32, 2),    # 384 tasks of 16 columns = 2 rounds; 192 of 32 = 1
    (2, 2048, 16, 256, 256, 32, 1),    # K = 256: no row split, 32 columns fill one round
    (1, 256, 2, 64, 64, 16, 4),        # the CPU-runnable case: 8 tasks, all four waves on rows
    (2, 2048, 16, 32, 32, 16, 2),      # K = 32: two 16-row tiles, split two ways at most
])
def test_plan_fp32_tile_width_and_row_split(lib, B, T, H, K, V, vt, rs):
    """fp32 plans: the tile width with the least (rounds of the device) x (relative time of one
    round: 1 / 1.62 / 2.25 at 16 / 32 / 64 columns with the row split, 1 / 1.13 / 1.22 at
    K = 256), and the row split that puts all four waves on state rows where K <= 128."""
    p = _abi.get_plan(_mi355x(_args(B=B, T=T, H=H, Hg=H, K=K, V=V, dtype=_abi.CGDR_F32)))
    assert (p.kernel, p.v_tile, p.row_split) == (1, vt, rs)
    assert p.workgroups == B * H * (V // vt) and p.lds_bytes <= 160 * 1024


def test_plan_bf16_row_split_default(lib):
    """bf16, default numerics: the state rows are split two ways at 16-column tiles without
    helpers (short sequences), not in helper mode (the headline) nor at 32-column tiles."""
    p = _abi.get_plan(_mi355x(_args(B=2, T=2048, H=16, Hg=16, K=128, V=128)))
    assert (p.v_tile, p.helpers, p.row_split) == (16, 0, 2)
    p = _abi.get_plan(_mi355x(_args(B=1, T=32768, H=32, Hg=32, K=128, V=128)))
    assert (p.v_tile, p.helpers, p.row_split) == (32, 1, 1)
    p = _abi.get_plan(_mi355x(_args(B=4, T=8192, H=8, Hg=8, K=128, V=256)))
    assert (p.v_tile, p.helpers, p.row_split) == (32, 0, 1)
    p = _abi.get_plan(_mi355x(_args(B=2, T=2048, H=16, Hg=16, K=32, V=32)))
    assert p.row_split == 1        # the bf16 split needs K of 64 or 128


def test_plan_follows_the_device_topology(lib):
    """The plan is made for the device's CU and XCD counts: on a smaller device (a partition
    of 64 CUs in 2 XCDs) the headline's 128 tasks + 128 helpers no longer fit, so it runs
    without helpers; helpers come back when the tasks fit half the CUs and split evenly over
    the XCDs, and stay off when they do not split evenly."""
    a = _args(B=1, T=32768, H=32, Hg=32, K=128, V=128)
    a.tuning = ctypes.pointer(t := _abi.make_tuning(cu_count=64, xcd_count=2))
    p = _abi.get_plan(a)
    assert (p.cu_count, p.xcd_count, p.helpers) == (64, 2, 0)
    assert (p.v_tile, p.workgroups) == (32, 128)
    p = _abi.get_plan(_args(B=1, T=32768, H=8, Hg=8, K=128, V=128, tuning=dict(cu_count=64, xcd_count=2)))
    assert (p.helpers, p.v_tile, p.workgroups) == (1, 32, 2 * 8 * 4)
    p = _abi.get_plan(_args(B=1, T=32768, H=5, Hg=5, K=128, V=128, tuning=dict(cu_count=64, xcd_count=8)))
    assert p.helpers == 0          # 20 tasks of 32 columns do not split over 8 XCDs
    p = _abi.get_plan(_args(B=1, T=32768, H=8, Hg=8, K=128, V=128, tuning=dict(cu_count=64, xcd_count=8)))
    assert p.helpers == 1 and p.workgroups == 64
    del t


@pytest.mark.parametrize("K,V,kd_plan", [(48, 48, dict(v_tile=16)), (96, 96, dict(v_tile=32, helpers=1)),
                                          (160, 160, dict(v_tile=16, helpers=0)), (224, 224, dict(v_tile=16)),
                                          (96, 128, dict(v_tile=32))])
def test_plan_accepts_padded_head_dims(lib, K, V, kd_plan):
    """Key dims that are multiples of 16 between the kernels' 32, 64, 128 and 256 are accepted
    (the reference takes any K = V in [32, 256]) and planned as the next instantiated key dim:
    K = 160 and 224 run the K = 256 layout (one compute wave, 16 columns, no helpers)."""
    a = _mi355x(_args(B=1, T=32768, H=32, Hg=32, K=K, V=V))
    st, _ = _status(a)
    assert st == _abi.CGDR_OK, _abi.last_error()
    p = _abi.get_plan(a)
    for key, want in kd_plan.items():
        assert getattr(p, key) == want, (K, V, key, getattr(p, key))
    a.in_dtype = _abi.CGDR_F32
    assert _status(a)[0] == _abi.CGDR_OK, _abi.last_error()   # fp32 up to K = 256


@pytest.mark.parametrize("B,T,H,K", [(5, 2000, 32, 32), (4, 4000, 32, 64)])
def test_plan_wide_tiles_without_helpers(lib, B, T, H, K):
    """The shapes of test_gpu_parity.test_default_plan_wide_tiles_without_helpers plan 32-column
    tiles with one load wave and no helpers on MI355X."""
    p = _abi.get_plan(_mi355x(_args(B=B, T=T, H=H, Hg=H, K=K, V=K)))
    assert (p.v_tile, p.helpers, p.load_waves) == (32, 0, 1)


@pytest.mark.parametrize("K,V,dtype", [(100, 100, _abi.CGDR_BF16), (33, 33, _abi.CGDR_BF16),
                                       (128, 100, _abi.CGDR_F32), (200, 200, _abi.CGDR_BF16)])
def test_workspace_holds_padded_copies(lib, K, V, dtype):
    """K or V not a multiple of 16 (the reference accepts any K = V in [32, 256]): the call runs
    on copies padded to multiples of 16, which the workspace holds (k, w, u, h0, h, v_new and
    the final state, each rounded up to 256 bytes) ahead of the padded call's own workspace."""
    B, T, H, Hg = 1, 256, 4, 2
    a = _mi355x(_args(B=B, T=T, H=H, Hg=Hg, K=K, V=V, dtype=dtype))
    a.initial_state = a.final_state = a.v_new = 1 << 24
    a.h0_dtype = a.final_dtype = _abi.CGDR_F32
    a.stride_h0[:] = [H * K * V, K * V]
    a.stride_final[:] = [H * K * V, K * V]
    a.stride_v[:] = [T * H * V, H * V, V]
    st, n = _status(a)
    assert st == _abi.CGDR_OK, _abi.last_error()
    Kp, Vp, NT = (K + 15) // 16 * 16, (V + 15) // 16 * 16, T // 64
    es = 2 if dtype == _abi.CGDR_BF16 else 4
    r256 = lambda x: (x + 255) // 256 * 256
    copies = (r256(B * T * Hg * Kp * es) + r256(B * T * H * Kp * es) + r256(B * T * H * Vp * es)
              + r256(H * Kp * Vp * 4) + r256(B * NT * H * Kp * Vp * es) + r256(B * T * H * Vp * es)
              + r256(H * Kp * Vp * 4))
    assert n == copies      # the padded call itself needs no workspace here (no g, no helpers)
    assert _abi.get_plan(a).v_tile >= 16


def test_tuning_overrides_and_rejections(lib):
    """Explicit plan overrides take effect, and out-of-range values are rejected."""
    p = _abi.get_plan(_args(B=1, T=32768, H=32, Hg=32, K=128, V=128,
                            tuning=dict(cu_count=256, xcd_count=8, helpers=0, v_tile=16)))
    assert (p.helpers, p.v_tile, p.workgroups) == (0, 16, 256)
    p = _abi.get_plan(_args(B=1, T=32768, H=32, Hg=32, K=128, V=128,
                            tuning=dict(cu_count=256, xcd_count=8, load_waves=1, stages=2)))
    assert (p.load_waves, p.stages) == (1, 2)
    for bad in (dict(v_tile=48), dict(helpers=2), dict(load_waves=3), dict(stages=5), dict(row_split=3),
                dict(cu_count=-1)):
        a = _args(tuning=bad)
        assert _status(a)[0] == _abi.CGDR_ERR_INVALID, bad


def test_helper_mode_workspace_holds_progress_counters(lib):
    # one 128-byte progress line per task, after the (256-byte rounded) head-major g copy
    # (helpers from 96 chunks per sequence on)
    a = _mi355x(_args(B=1, T=6100, H=32, Hg=32, K=128, V=128))
    assert _status(a) == (_abi.CGDR_OK, 128 * 128)
    a = _mi355x(_with_g(_args(B=1, T=6100, H=32, Hg=32, K=128, V=128)))
    assert _status(a) == (_abi.CGDR_OK, ((32 * 6100 * 4 + 255) // 256) * 256 + 128 * 128)
    assert _status(_mi355x(_args(B=1, T=6000, H=32, Hg=32, K=128, V=128))) == (_abi.CGDR_OK, 0)   # 94 chunks


def test_wrapper_refuses_cpu_tensors():
    import torch

    import cgdr_amd
    k = torch.zeros(1, 64, 1, 64, dtype=torch.bfloat16)
    w = torch.zeros(1, 64, 1, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="HIP device"):
        cgdr_amd.chunk_gated_delta_rule_fwd_h(k, w, w)


def test_plan_accepts_random_configurations(lib):
    """Every configuration of the random GPU parity cases (tests/test_gpu_random.py) is planned:
    its head dims, batch layout, dtype, numerics and tuning fields are all accepted, as for
    MI355X."""
    import test_gpu_random as R
    for i in range(R.CASES):
        c = R.draw(i)
        dt = _abi.CGDR_F32 if c["dtype"] == "f32" else _abi.CGDR_BF16
        a = _args(B=c["B"], T=c["T"], H=c["H"], Hg=c["Hg"], K=c["K"], V=c["V"], dtype=dt,
                  varlen=None if c["cu"] is None else c["cu"].tolist())
        a.g = 1 << 24
        a.stride_g[:] = [c["T"] * c["H"], c["H"], 1]
        a.numerics = 1 if c["contest"] else 0
        _mi355x(a, **c["tuning"])
        p = _abi.get_plan(a)
        assert p.workgroups > 0, (i, c)
