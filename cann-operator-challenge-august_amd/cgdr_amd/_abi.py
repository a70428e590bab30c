"""ctypes binding of the C ABI declared in ``include/cgdr_fwd_h.h``, ``include/cgdr_chunk_o.h``
and ``include/cgdr_wy.h``.

The shared library ``libcgdr_fwd_h.so`` is built in-tree by ``cgdr_amd.build`` into
``<package root>/lib``.  Loading it does not touch the GPU; only ``cgdr_fwd_h_launch``
does.  There is no fallback: if the library is missing, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os

CHUNK_SIZE = 64
ABI_VERSION = 4

CGDR_OK = 0
CGDR_ERR_NULLPTR = 1
CGDR_ERR_INVALID = 2
CGDR_ERR_UNSUPPORTED = 3
CGDR_ERR_LAUNCH = 4

CGDR_BF16 = 0
CGDR_F32 = 1

CGDR_NUMERICS_DEFAULT = 0
CGDR_NUMERICS_CONTEST = 1

CGDR_STATE_KV = 0
CGDR_STATE_VK = 1

EXPORTED_SYMBOLS = (
    "cgdr_fwd_h_workspace_size",
    "cgdr_fwd_h_launch",
    "cgdr_fwd_h_launch_no_alloc",
    "cgdr_fwd_h_get_plan",
    "cgdr_prepare_chunk_offsets",
    "cgdr_prepare_chunk_indices",
    "cgdr_status_string",
    "cgdr_last_error",
    "cgdr_abi_version",
    "cgdr_chunk_o_launch",
    "cgdr_chunk_o_get_plan",
    "cgdr_wy_launch",
)

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(_PKG_ROOT, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libcgdr_fwd_h.so")

_c_i64_p = ctypes.POINTER(ctypes.c_int64)


class FwdHTuning(ctypes.Structure):
    """Mirror of ``cgdr_fwd_h_tuning`` (launch-plan overrides; results never depend on them)."""

    _fields_ = [
        ("v_tile", ctypes.c_int32),
        ("helpers", ctypes.c_int32),
        ("load_waves", ctypes.c_int32),
        ("stages", ctypes.c_int32),
        ("prefetch", ctypes.c_int32),
        ("helper_lead", ctypes.c_int32),
        ("helper_waves", ctypes.c_int32),
        ("cu_count", ctypes.c_int32),
        ("xcd_count", ctypes.c_int32),
        ("row_split", ctypes.c_int32),
    ]


def make_tuning(**kw) -> FwdHTuning:
    """A ``cgdr_fwd_h_tuning`` with the library's choice everywhere except the given fields."""
    t = FwdHTuning(helpers=-1, prefetch=-1, helper_lead=-1)
    for k, v in kw.items():
        if k not in dict(FwdHTuning._fields_):
            raise ValueError(f"unknown tuning field {k!r}")
        setattr(t, k, int(v))
    return t


class FwdHArgs(ctypes.Structure):
    """Mirror of ``cgdr_fwd_h_args``."""

    _fields_ = [
        ("k", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("u", ctypes.c_void_p),
        ("g", ctypes.c_void_p),
        ("initial_state", ctypes.c_void_p),
        ("cu_seqlens", ctypes.c_void_p),
        ("chunk_offsets", ctypes.c_void_p),
        ("h", ctypes.c_void_p),
        ("v_new", ctypes.c_void_p),
        ("final_state", ctypes.c_void_p),
        ("B", ctypes.c_int64),
        ("T", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("Hg", ctypes.c_int64),
        ("K", ctypes.c_int64),
        ("V", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("NT", ctypes.c_int64),
        ("chunk_size", ctypes.c_int64),
        ("in_dtype", ctypes.c_int32),
        ("h0_dtype", ctypes.c_int32),
        ("final_dtype", ctypes.c_int32),
        ("numerics", ctypes.c_int32),
        ("stride_k", ctypes.c_int64 * 3),
        ("stride_w", ctypes.c_int64 * 3),
        ("stride_u", ctypes.c_int64 * 3),
        ("stride_g", ctypes.c_int64 * 3),
        ("stride_h", ctypes.c_int64 * 3),
        ("stride_v", ctypes.c_int64 * 3),
        ("stride_h0", ctypes.c_int64 * 2),
        ("stride_final", ctypes.c_int64 * 2),
        ("tuning", ctypes.POINTER(FwdHTuning)),
        ("state_layout", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class FwdHPlan(ctypes.Structure):
    """Mirror of ``cgdr_fwd_h_plan``."""

    _fields_ = [
        ("kernel", ctypes.c_int32),
        ("v_tile", ctypes.c_int32),
        ("compute_waves", ctypes.c_int32),
        ("total_waves", ctypes.c_int32),
        ("stages", ctypes.c_int32),
        ("lds_bytes", ctypes.c_int32),
        ("workgroups", ctypes.c_int64),
        ("helpers", ctypes.c_int32),
        ("load_waves", ctypes.c_int32),
        ("cu_count", ctypes.c_int32),
        ("xcd_count", ctypes.c_int32),
        ("row_split", ctypes.c_int32),
    ]


class ChunkOArgs(ctypes.Structure):
    """Mirror of ``cgdr_chunk_o_args``."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v_new", ctypes.c_void_p),
        ("h", ctypes.c_void_p),
        ("g", ctypes.c_void_p),
        ("cu_seqlens", ctypes.c_void_p),
        ("chunk_indices", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("B", ctypes.c_int64),
        ("T", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("Hg", ctypes.c_int64),
        ("K", ctypes.c_int64),
        ("V", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("NT", ctypes.c_int64),
        ("chunk_size", ctypes.c_int64),
        ("scale", ctypes.c_float),
        ("in_dtype", ctypes.c_int32),
        ("stride_q", ctypes.c_int64 * 3),
        ("stride_k", ctypes.c_int64 * 3),
        ("stride_v", ctypes.c_int64 * 3),
        ("stride_h", ctypes.c_int64 * 3),
        ("stride_g", ctypes.c_int64 * 3),
        ("stride_o", ctypes.c_int64 * 3),
    ]


class WyArgs(ctypes.Structure):
    """Mirror of ``cgdr_wy_args``."""

    _fields_ = [
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("beta", ctypes.c_void_p),
        ("g", ctypes.c_void_p),
        ("cu_seqlens", ctypes.c_void_p),
        ("chunk_indices", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("u", ctypes.c_void_p),
        ("g_cumsum", ctypes.c_void_p),
        ("B", ctypes.c_int64),
        ("T", ctypes.c_int64),
        ("H", ctypes.c_int64),
        ("Hg", ctypes.c_int64),
        ("K", ctypes.c_int64),
        ("V", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("NT", ctypes.c_int64),
        ("chunk_size", ctypes.c_int64),
        ("in_dtype", ctypes.c_int32),
        ("beta_dtype", ctypes.c_int32),
        ("stride_k", ctypes.c_int64 * 3),
        ("stride_v", ctypes.c_int64 * 3),
        ("stride_beta", ctypes.c_int64 * 3),
        ("stride_g", ctypes.c_int64 * 3),
        ("stride_w", ctypes.c_int64 * 3),
        ("stride_u", ctypes.c_int64 * 3),
        ("stride_g_cumsum", ctypes.c_int64 * 3),
    ]


class CgdrError(RuntimeError):
    """A non-zero ``cgdr_status`` from the library, with its message."""

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"{status_string(status)}: {message}")


_lib = None


def load(path: str | None = None):
    """Load (once) and return the shared library; raise if it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise RuntimeError(
            f"{p} not found: the HIP library is not built (run __graft_entry__.build() "
            "or python -m cgdr_amd.build); there is no CPU fallback")
    lib = ctypes.CDLL(p)
    lib.cgdr_fwd_h_workspace_size.argtypes = [ctypes.POINTER(FwdHArgs), ctypes.POINTER(ctypes.c_size_t)]
    lib.cgdr_fwd_h_workspace_size.restype = ctypes.c_int
    lib.cgdr_fwd_h_launch.argtypes = [ctypes.POINTER(FwdHArgs), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    lib.cgdr_fwd_h_launch.restype = ctypes.c_int
    lib.cgdr_fwd_h_launch_no_alloc.argtypes = [ctypes.POINTER(FwdHArgs), ctypes.c_void_p]
    lib.cgdr_fwd_h_launch_no_alloc.restype = ctypes.c_int
    lib.cgdr_fwd_h_get_plan.argtypes = [ctypes.POINTER(FwdHArgs), ctypes.POINTER(FwdHPlan)]
    lib.cgdr_fwd_h_get_plan.restype = ctypes.c_int
    lib.cgdr_prepare_chunk_offsets.argtypes = [_c_i64_p, ctypes.c_int64, ctypes.c_int64, _c_i64_p]
    lib.cgdr_prepare_chunk_offsets.restype = ctypes.c_int
    lib.cgdr_prepare_chunk_indices.argtypes = [_c_i64_p, ctypes.c_int64, ctypes.c_int64, _c_i64_p,
                                               ctypes.c_int64, _c_i64_p]
    lib.cgdr_prepare_chunk_indices.restype = ctypes.c_int
    lib.cgdr_status_string.argtypes = [ctypes.c_int]
    lib.cgdr_status_string.restype = ctypes.c_char_p
    lib.cgdr_last_error.argtypes = []
    lib.cgdr_last_error.restype = ctypes.c_char_p
    lib.cgdr_chunk_o_launch.argtypes = [ctypes.POINTER(ChunkOArgs), ctypes.c_void_p]
    lib.cgdr_chunk_o_launch.restype = ctypes.c_int
    lib.cgdr_chunk_o_get_plan.argtypes = [ctypes.POINTER(ChunkOArgs), ctypes.POINTER(ctypes.c_int32),
                                          ctypes.POINTER(ctypes.c_int64)]
    lib.cgdr_chunk_o_get_plan.restype = ctypes.c_int
    lib.cgdr_wy_launch.argtypes = [ctypes.POINTER(WyArgs), ctypes.c_void_p]
    lib.cgdr_wy_launch.restype = ctypes.c_int
    lib.cgdr_abi_version.argtypes = []
    lib.cgdr_abi_version.restype = ctypes.c_int
    if lib.cgdr_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{p}: ABI version {lib.cgdr_abi_version()} != {ABI_VERSION}")
    if path is None:
        _lib = lib
    return lib


def status_string(status: int) -> str:
    return load().cgdr_status_string(status).decode()


def last_error() -> str:
    return load().cgdr_last_error().decode()


def check(status: int) -> None:
    if status != CGDR_OK:
        raise CgdrError(status, last_error())


def workspace_size(args: FwdHArgs) -> int:
    n = ctypes.c_size_t(0)
    check(load().cgdr_fwd_h_workspace_size(ctypes.byref(args), ctypes.byref(n)))
    return n.value


def get_plan(args: FwdHArgs) -> FwdHPlan:
    plan = FwdHPlan()
    check(load().cgdr_fwd_h_get_plan(ctypes.byref(args), ctypes.byref(plan)))
    return plan


def launch(args: FwdHArgs, stream: int, workspace: int = 0, workspace_bytes: int = 0) -> None:
    """Enqueue on `stream`; `workspace` is a device pointer of workspace_size(args) bytes
    that stays untouched by the caller until the launch has completed on that stream."""
    check(load().cgdr_fwd_h_launch(ctypes.byref(args), ctypes.c_void_p(workspace or None),
                                   ctypes.c_size_t(workspace_bytes), ctypes.c_void_p(stream)))


NO_ALLOC_SCRATCH_BYTES = 16 << 20   # CGDR_NO_ALLOC_SCRATCH_BYTES


def launch_no_alloc(args: FwdHArgs, stream: int) -> None:
    """Enqueue on `stream` with the library's static per-GPU scratch instead of a workspace
    (no device allocation); launches that overlap on one GPU race on that scratch."""
    check(load().cgdr_fwd_h_launch_no_alloc(ctypes.byref(args), ctypes.c_void_p(stream)))


def chunk_o_launch(args: ChunkOArgs, stream: int) -> None:
    check(load().cgdr_chunk_o_launch(ctypes.byref(args), ctypes.c_void_p(stream)))


def wy_launch(args: WyArgs, stream: int) -> None:
    check(load().cgdr_wy_launch(ctypes.byref(args), ctypes.c_void_p(stream)))


def chunk_o_plan(args: ChunkOArgs) -> tuple[int, int]:
    """(v_tile, workgroups) of the launch for ``args``."""
    vt, wg = ctypes.c_int32(0), ctypes.c_int64(0)
    check(load().cgdr_chunk_o_get_plan(ctypes.byref(args), ctypes.byref(vt), ctypes.byref(wg)))
    return vt.value, wg.value


def prepare_chunk_offsets(cu_seqlens: list[int], chunk_size: int = CHUNK_SIZE) -> list[int]:
    n = len(cu_seqlens) - 1
    cu = (ctypes.c_int64 * (n + 1))(*cu_seqlens)
    out = (ctypes.c_int64 * (n + 1))()
    check(load().cgdr_prepare_chunk_offsets(cu, n, chunk_size, out))
    return list(out)


def prepare_chunk_indices(cu_seqlens: list[int], chunk_size: int = CHUNK_SIZE) -> list[tuple[int, int]]:
    n = len(cu_seqlens) - 1
    cu = (ctypes.c_int64 * (n + 1))(*cu_seqlens)
    nt = ctypes.c_int64(0)
    check(load().cgdr_prepare_chunk_indices(cu, n, chunk_size, None, 0, ctypes.byref(nt)))
    rows = (ctypes.c_int64 * max(1, 2 * nt.value))()
    check(load().cgdr_prepare_chunk_indices(cu, n, chunk_size, rows, nt.value, ctypes.byref(nt)))
    return [(rows[2 * i], rows[2 * i + 1]) for i in range(nt.value)]
