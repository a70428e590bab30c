"""CPU oracle for the ChunkGatedDeltaRuleFwdH chunk recurrence (numpy).

TEST INFRASTRUCTURE ONLY.  This module is the reference for the tests: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path (the HIP library behind ``include/cgdr_fwd_h.h``)
never calls into it and never falls back to it.

What it restates (paths relative to the reference's
``ChunkGatedDeltaRuleFwdH_problem_290_template/``):

* ``fwd_h(..., rounding=None)`` -- the exact recurrence ("O3"): the fp32 chunk
  loop of ``ref/chunk_gated_delta_rule/tests/pytest/chunk_gated_delta_rule_golden.py:136-149``
  written against the FwdH inputs (w = k_cumdecay, u = value there).  Decay is
  applied to ``v_new`` instead of ``k`` (``docs/problem.txt:400-405``), which is
  the same product.  Output timing follows ``docs/problem.txt:81-167``:
  ``h[c]`` is the state *entering* chunk c, ``v_new`` is the un-gated
  ``U - W @ S`` and ``final`` the state after the last chunk.
* ``fwd_h(..., rounding="bf16")`` -- the same loop with the rounding points of
  the Triton kernel ``chunk_gated_delta_rule_fwd_kernel_h_blockdim64``
  (``docs/problem.txt:330-432``, "O1"): ``bf16(S)`` feeds ``W @ S`` and the h
  snapshot (``:356-360``, ``:392-394``), ``v_new`` is stored in the input dtype
  (``:396-398``), the gated value is rounded to bf16 before ``K^T @ .``
  (``:401-405``) and the state stays fp32.  The kernel text cannot run here; every one of
  these rounding points is pinned by closed forms on one-hot operands, where each
  contraction has a single nonzero product and so is exact in any summation order
  (``tests/o1_probe.py``, ``tests/test_oracle.py``): moving any one of them (the
  ``mistake`` variants below) breaks the closed form.
* ``fwd_h_o2`` -- the contest reference ``run()`` / the golden generator's
  ``run_reference`` ("O2", ``code/tests/golden/generate_golden.py:350-440``,
  ``docs/problem.txt:81-167``): bf16 state, bf16 GEMM outputs, saturating fp16 casts
  (``cast_to_float16``, ``generate_golden.py:285-290``) and ``nan_to_num`` after each GEMM.
  Pinned by the reference's own golden cases (``tests/golden/cases``).
* ``fwd_h_bf16_state`` -- the reference's bf16 benchmark ``stage2_opt``
  (``ref/chunk_gated_delta_rule/tests/pytest/chunk_gated_delta_rule_benchmark.py:96-142``, key
  gating from ``stage1_opt`` ``:74,83``): the state is rounded to bf16 after every chunk,
  the gate scales k instead of v_new, every GEMM output is rounded to bf16.  It is the
  "benchmark" side of the reference's three-way accuracy gate
  (``ref/chunk_gated_delta_rule/tests/assets/impl/compare.py:32-35,93-196``).  Pinned by
  vectors the reference's own ``stage1_opt``/``stage2_opt`` wrote
  (``tests/golden/bf16_state``, ``tests/golden/make_bf16_state_golden.py``).
* ``prepare_chunk_offsets`` / ``prepare_chunk_indices`` -- ``docs/problem.txt:251-270``
  and ``code/tests/golden/generate_golden.py:260-282``.
* ``safe_exp`` -- ``docs/problem.txt:272-274``.
* ``wy_prepare`` -- the producer of (w, u, g) from (k, v, beta, per-token
  log-decay): ``chunk_gated_delta_rule_golden.py:102-124``.
* ``chunk_o(..., rounding=None)`` -- the chunk output, the consumer of ``h`` and
  ``v_new``: ``o_i = scale (e^{g_i} q_i h_c + sum_{j<=i in chunk} (q_i.k_j) e^{g_i-g_j} v_new_j)``,
  the loop body of ``chunk_gated_delta_rule_golden.py:136-142`` (query pre-scaled at
  ``:99-100``, decay mask ``:116``) and, on the device side, ``attn_inter`` of
  ``ref/chunk_gated_delta_rule/op_kernel/arch22/chunk_gated_delta_rule_stage2.h:170`` plus
  the masked ``q k^T`` product of ``.../chunk_gated_delta_rule_stage3.h:131-180``.
  ``rounding="bf16"`` is the rounding model of the HIP kernel: the masked, decayed and
  scaled ``q k^T`` is rounded to bf16 (it is an MFMA operand, as in stage3 ``:157-160``), both
  products accumulate in fp32 and ``o`` is rounded once.
* ``gated_delta_rule_tokenwise`` -- the token-by-token Gated DeltaNet recurrence
  ``S_t = e^{a_t} (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T`` and, given
  queries, its output ``o_t = scale S_t^T q_t``.  It is not in the reference; it is
  the textbook definition that the chunked form must reproduce, and the tests use it
  to pin ``fwd_h`` and ``chunk_o`` independently of any chunked restatement.

Layouts are token-major (FLA / Triton wrapper ``docs/problem.txt:434-472``):
k ``[B,T,Hg,K]``, w ``[B,T,H,K]``, u ``[B,T,H,V]``, g ``[B,T,H]``,
h0 ``[N,H,K,V]`` -> h ``[B,NT,H,K,V]``, v_new ``[B,T,H,V]``, final ``[N,H,K,V]``.
``to_token_major`` / ``from_token_major`` convert the head-major layout of the
contest reference ``run()`` (``docs/problem.txt:81-97``).
"""

from __future__ import annotations

import numpy as np

CHUNK_SIZE = 64


# ----------------------------------------------------------------------------- rounding

def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), returned as float32.

    NaN stays NaN; +-Inf and overflow follow IEEE round-to-nearest-even, which is
    what ``torch.Tensor.to(torch.bfloat16)`` and ``v_cvt_pk_bf16_f32`` do.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    # uint32 arithmetic wraps only for NaN payloads (>= 0xFFFF8000), which are restored below.
    out = u >> 16
    out &= 1
    out += 0x7FFF
    out += u
    out &= np.uint32(0xFFFF0000)
    out = out.view(np.float32)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.nan
    return out.reshape(x.shape)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """bfloat16 storage bits (uint16) of float32 values, ties to even."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits: np.ndarray) -> np.ndarray:
    """float32 values of bfloat16 storage bits."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------- varlen metadata

def prepare_lens(cu_seqlens: np.ndarray) -> np.ndarray:
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    return cu[1:] - cu[:-1]


def prepare_chunk_offsets(cu_seqlens: np.ndarray, chunk_size: int = CHUNK_SIZE) -> np.ndarray:
    """``[0, C_0, C_0+C_1, ...]`` with ``C_n = ceil(L_n / chunk_size)``.

    Follows ``docs/problem.txt:263-270`` (and ``:181-185``).
    """
    lens = prepare_lens(cu_seqlens)
    counts = (lens + chunk_size - 1) // chunk_size
    return np.concatenate([np.zeros(1, np.int64), np.cumsum(counts, dtype=np.int64)])


def prepare_chunk_indices(cu_seqlens: np.ndarray, chunk_size: int = CHUNK_SIZE) -> np.ndarray:
    """Rows ``(sequence, chunk-within-sequence)``, shape ``[NT, 2]`` int64.

    Follows ``docs/problem.txt:251-261`` and ``code/tests/golden/generate_golden.py:260-270``.
    """
    rows = []
    for n, length in enumerate(prepare_lens(cu_seqlens)):
        rows.extend((n, c) for c in range(int((length + chunk_size - 1) // chunk_size)))
    if not rows:
        return np.zeros((0, 2), np.int64)
    return np.asarray(rows, dtype=np.int64)


def safe_exp(x: np.ndarray) -> np.ndarray:
    """``exp(x)`` for ``x <= 0`` and ``0`` for ``x > 0`` (``docs/problem.txt:272-274``)."""
    x = np.asarray(x)
    return np.exp(np.where(x <= 0, x, -np.inf))


# ----------------------------------------------------------------------------- layouts

def to_token_major(w: np.ndarray, u: np.ndarray, g: np.ndarray | None):
    """Head-major ``w [B,H,T,K]``, ``u [B,H,T,V]``, ``g [B,H,T]`` (``docs/problem.txt:216-219``)
    to token-major.  ``k`` is ``[B,T,Hg,K]`` in both conventions."""
    w_t = np.swapaxes(w, 1, 2)
    u_t = np.swapaxes(u, 1, 2)
    g_t = None if g is None else np.swapaxes(g, 1, 2)
    return w_t, u_t, g_t


def from_token_major(h: np.ndarray, v_new: np.ndarray | None):
    """Token-major ``h [B,NT,H,K,V]`` / ``v_new [B,T,H,V]`` to the head-major outputs
    ``[B,H,NT,K,V]`` / ``[B,H,T,V]`` of ``docs/problem.txt:94-96``."""
    return np.swapaxes(h, 1, 2), None if v_new is None else np.swapaxes(v_new, 1, 2)


# ----------------------------------------------------------------------------- the recurrence

def sequence_bounds(B: int, T: int, cu_seqlens: np.ndarray | None, chunk_size: int = CHUNK_SIZE):
    """Per sequence ``(batch_row, bos, eos, first_chunk)``; mirrors the bos/eos/boh
    derivation of ``docs/problem.txt:336-350`` (varlen and fixed-length branches)."""
    out = []
    if cu_seqlens is None:
        nt = (T + chunk_size - 1) // chunk_size
        for b in range(B):
            out.append((b, 0, T, 0, nt))  # each batch row owns chunks [b, 0:NT)
        return out, nt
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    offs = prepare_chunk_offsets(cu, chunk_size)
    for n in range(cu.size - 1):
        out.append((0, int(cu[n]), int(cu[n + 1]), int(offs[n]), None))
    return out, int(offs[-1])


def fwd_h(
    k: np.ndarray,
    w: np.ndarray,
    u: np.ndarray,
    g: np.ndarray | None = None,
    initial_state: np.ndarray | None = None,
    output_final_state: bool = True,
    chunk_size: int = CHUNK_SIZE,
    cu_seqlens: np.ndarray | None = None,
    rounding: str | None = None,
    compute_dtype=np.float32,
    save_new_value: bool = True,
    mistake: str | None = None,
):
    """Chunked gated delta-rule state recurrence, token-major layouts.

    ``rounding=None`` is the exact recurrence in ``compute_dtype``;
    ``rounding="bf16"`` applies the bf16 rounding points of the Triton kernel
    (the rounding model of the bf16 HIP kernel).  Inputs are taken as given
    (bf16 inputs should be passed as their float32 values).

    Returns ``(h, v_new, final)`` as arrays of ``compute_dtype``; ``h`` and
    ``v_new`` are already rounded to bf16 values when ``rounding="bf16"``.

    ``mistake`` moves one rounding point of the bf16 model, for the tests that show the
    closed-form pins catch such a change (never used to produce a reference):
    ``"mm1_fp32_state"`` feeds the unrounded state to ``W @ S``; ``"gate_rounded_v_new"``
    gates the bf16-rounded v_new (``bf16(bf16(Vn) gamma)``); ``"mm2_fp32_operand"`` leaves
    the gated value unrounded in ``K^T @ .``; ``"bf16_state"`` rounds the carried state to
    bf16 after every chunk.
    """
    if chunk_size != CHUNK_SIZE:
        raise ValueError(f"chunk_size must be {CHUNK_SIZE}, got {chunk_size}")
    if rounding not in (None, "bf16"):
        raise ValueError(f"unknown rounding {rounding!r}")
    rnd = bf16_round if rounding == "bf16" else (lambda a: a)
    mistakes = (None, "mm1_fp32_state", "gate_rounded_v_new", "mm2_fp32_operand", "bf16_state")
    if mistake not in mistakes or (mistake is not None and rounding != "bf16"):
        raise ValueError(f"mistake must be one of {mistakes} (with rounding='bf16'), got {mistake!r}")
    cd = np.dtype(compute_dtype)

    k = np.asarray(k, dtype=cd)
    w = np.asarray(w, dtype=cd)
    u = np.asarray(u, dtype=cd)
    B, T, Hg, K = k.shape
    H, V = u.shape[2], u.shape[3]
    if w.shape != (B, T, H, K) or u.shape[:2] != (B, T):
        raise ValueError("w must be [B,T,H,K] and u [B,T,H,V]")
    if H % Hg != 0:
        raise ValueError("H must be a multiple of Hg")
    if cu_seqlens is not None and B != 1:
        raise ValueError("cu_seqlens requires B == 1")
    gq = None if g is None else np.asarray(g, dtype=cd)
    head_of_key = np.arange(H) // (H // Hg)  # docs/problem_understanding.md:52-71

    seqs, NT = sequence_bounds(B, T, cu_seqlens, chunk_size)
    N = len(seqs)
    h_out = np.zeros((B, NT, H, K, V), dtype=cd)
    v_out = np.zeros((B, T, H, V), dtype=cd) if save_new_value else None
    final = np.zeros((N, H, K, V), dtype=cd) if output_final_state else None
    h0 = None if initial_state is None else np.asarray(initial_state, dtype=cd)

    for n, (b, bos, eos, boh, _) in enumerate(seqs):
        S = np.zeros((H, K, V), dtype=cd) if h0 is None else h0[n].astype(cd, copy=True)
        for c, t0 in enumerate(range(bos, eos, chunk_size)):
            t1 = min(t0 + chunk_size, eos)
            Sr = rnd(S) if rounding else S
            h_out[b, boh + c] = Sr
            if mistake == "mm1_fp32_state":
                Sr = S
            Kc = np.transpose(k[b, t0:t1][:, head_of_key, :], (1, 0, 2))   # [H, L, K]
            Wc = np.transpose(w[b, t0:t1], (1, 0, 2))                       # [H, L, K]
            Uc = np.transpose(u[b, t0:t1], (1, 0, 2))                       # [H, L, V]
            Vn = Uc - np.matmul(Wc, Sr)                                     # [H, L, V]
            if save_new_value:
                v_out[b, t0:t1] = np.transpose(rnd(Vn) if rounding else Vn, (1, 0, 2))
            Vg = rnd(Vn) if mistake == "gate_rounded_v_new" else Vn
            if gq is not None:
                gc = np.transpose(gq[b, t0:t1], (1, 0))                     # [H, L]
                g_last = gc[:, -1]
                gamma = safe_exp(g_last[:, None] - gc).astype(cd)
                Vd = Vg * gamma[:, :, None]
                S = S * np.exp(g_last).astype(cd)[:, None, None]
            else:
                Vd = Vg
            if rounding and mistake != "mm2_fp32_operand":
                Vd = rnd(Vd)
            S = S + np.matmul(np.transpose(Kc, (0, 2, 1)), Vd)
            if mistake == "bf16_state":
                S = rnd(S)
        if output_final_state:
            final[n] = S
    return h_out, v_out, final


# ----------------------------------------------------------------------------- bf16-state benchmark

def fwd_h_bf16_state(
    k: np.ndarray,
    w: np.ndarray,
    u: np.ndarray,
    g: np.ndarray | None = None,
    initial_state: np.ndarray | None = None,
    cu_seqlens: np.ndarray | None = None,
    chunk_size: int = CHUNK_SIZE,
):
    """The reference's bf16 benchmark of the state recurrence, ``stage2_opt``
    (``ref/chunk_gated_delta_rule/tests/pytest/chunk_gated_delta_rule_benchmark.py:96-142``) with
    the key gating of its ``stage1_opt`` (``:74``, ``:83``), written against the FwdH inputs
    (``k_cumdecay = -w``, ``v_inner = u``, ``g_cum = g``) in the token-major layouts of
    ``fwd_h``.  Per chunk, with S the state entering it (the initial state as given, bf16
    values from the first chunk on):

      v_new = bf16(u + bf16(-(w @ S)))                      (:130-131, bf16 + bf16 in bf16)
      kg    = bf16(k * exp(g_last - g))                     (stage1 :74, :83; no clamp)
      S     = bf16(bf16(S * exp(g_last)) + bf16(kg^T @ v_new))   (:133-136)

    Every product is rounded once to bf16 (the benchmark's float32 accumulations, here taken
    in float64, then rounded to float32 and to bf16).  ``h[c]`` (which the benchmark
    does not return) is taken as bf16 of the state entering chunk c, the FwdH output's
    definition.  Returns ``(h, v_new, final)`` as float32 arrays of bf16 values; the reference
    keeps the benchmark's transposed ``[V, K]`` state, this keeps ``[K, V]``."""
    if chunk_size != CHUNK_SIZE:
        raise ValueError(f"chunk_size must be {CHUNK_SIZE}, got {chunk_size}")
    f32 = np.float32
    k = np.asarray(k, f32)
    w = np.asarray(w, f32)
    u = np.asarray(u, f32)
    B, T, Hg, K = k.shape
    H, V = u.shape[2], u.shape[3]
    head_of_key = np.arange(H) // (H // Hg)
    gq = None if g is None else np.asarray(g, f32)
    seqs, NT = sequence_bounds(B, T, cu_seqlens, chunk_size)
    h_out = np.zeros((B, NT, H, K, V), f32)
    v_out = np.zeros((B, T, H, V), f32)
    final = np.zeros((len(seqs), H, K, V), f32)
    h0 = None if initial_state is None else np.asarray(initial_state, f32)
    for n, (b, bos, eos, boh, _) in enumerate(seqs):
        S = np.zeros((H, K, V), f32) if h0 is None else h0[n].copy()
        for c, t0 in enumerate(range(bos, eos, chunk_size)):
            t1 = min(t0 + chunk_size, eos)
            h_out[b, boh + c] = bf16_round(S)
            Kc = np.transpose(k[b, t0:t1][:, head_of_key, :], (1, 0, 2))   # [H, L, K]
            Wc = np.transpose(w[b, t0:t1], (1, 0, 2))
            Uc = np.transpose(u[b, t0:t1], (1, 0, 2))
            vp = bf16_round(np.matmul(-Wc.astype(np.float64), S).astype(f32))
            vn = bf16_round((Uc + vp).astype(f32))
            v_out[b, t0:t1] = np.transpose(vn, (1, 0, 2))
            if gq is not None:
                gc = np.transpose(gq[b, t0:t1], (1, 0))                     # [H, L]
                g_last = gc[:, -1]
                kg = bf16_round((Kc * np.exp((g_last[:, None] - gc).astype(f32))[:, :, None]).astype(f32))
                decay = np.exp(g_last).astype(f32)[:, None, None]
            else:
                kg = Kc
                decay = f32(1.0)
            upd = bf16_round(np.matmul(np.transpose(kg, (0, 2, 1)).astype(np.float64), vn).astype(f32))
            S = bf16_round((bf16_round((S * decay).astype(f32)) + upd).astype(f32))
        final[n] = S
    return h_out, v_out, final


# ----------------------------------------------------------------------------- O2 (contest run())

def f16_sat(x: np.ndarray) -> np.ndarray:
    """``cast_to_float16`` (``code/tests/golden/generate_golden.py:285-290``): round to fp16;
    finite inputs that overflow saturate to +-65504, inf and NaN pass through."""
    x = np.asarray(x, np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        h = x.astype(np.float16)
    special = ~np.isfinite(x)
    return np.where(special, h, np.clip(h, np.float16(-65504), np.float16(65504))).astype(np.float16)


def f16_nan_to_num(x: np.ndarray) -> np.ndarray:
    """``torch.nan_to_num(x.to(float16), nan=0, posinf=inf, neginf=-inf)``."""
    with np.errstate(over="ignore", invalid="ignore"):
        h = np.asarray(x, np.float32).astype(np.float16)
    return np.where(np.isnan(h), np.float16(0), h).astype(np.float16)


def fwd_h_o2(k, w, u, g, initial_state=None, cu_seqlens=None, chunk_size: int = CHUNK_SIZE):
    """O2: the golden generator's ``run_reference`` (``generate_golden.py:350-440``), in its
    head-major layouts: k ``[1,T,HK,K]``, w ``[1,HV,T,K]``, u ``[1,HV,T,V]``, g ``[1,HV,T]``,
    initial_state ``[N,HV,K,V]`` -> h ``[1,HV,NT,K,V]``, v ``[1,HV,T,V]``, final ``[N,HV,K,V]``,
    all bf16 values (float32 arrays).  A bf16 GEMM is a float32 product rounded once to bf16
    (``ws = w_sel @ state``, ``update = k^T @ v_decay_bf16``, ``:397``, ``:423``)."""
    k = np.asarray(k, np.float32)
    w = np.asarray(w, np.float32)
    u = np.asarray(u, np.float32)
    g = np.asarray(g, np.float32)
    _, T, HK, K = k.shape
    HV, V = u.shape[1], u.shape[3]
    cu = np.array([0, T]) if cu_seqlens is None else np.asarray(cu_seqlens, np.int64)
    offs = prepare_chunk_offsets(cu, chunk_size)
    N, NT = len(cu) - 1, int(offs[-1])
    ratio = HV // HK
    h_out = np.zeros((1, HV, NT, K, V), np.float32)
    v_out = np.zeros((1, HV, T, V), np.float32)
    final = np.zeros((N, HV, K, V), np.float32)
    f32 = lambda x: np.asarray(x, np.float32)
    for n in range(N):
        bos, eos = int(cu[n]), int(cu[n + 1])
        for hh in range(HV):
            S = np.zeros((K, V), np.float32) if initial_state is None else bf16_round(initial_state[n, hh])
            for c, t0 in enumerate(range(bos, eos, chunk_size)):
                t1 = min(t0 + chunk_size, eos)
                h_out[0, hh, int(offs[n]) + c] = S
                ks = k[0, t0:t1, hh // ratio]
                ws = bf16_round(w[0, hh, t0:t1] @ S)
                v16 = f16_sat(f32(f16_sat(u[0, hh, t0:t1])) - f32(f16_nan_to_num(ws)))
                gs = g[0, hh, t0:t1]
                gate = f16_sat(np.exp(gs[-1] - gs))
                vd = bf16_round(f32(f16_sat(f32(v16) * f32(gate)[:, None])))
                with np.errstate(over="ignore"):
                    sg = np.exp(f32(f16_sat(gs[-1:]))).astype(np.float16)
                hd16 = f16_sat(f32(f16_sat(S)) * f32(sg))
                upd16 = f16_nan_to_num(bf16_round(ks.T @ vd))
                S = bf16_round(f32(bf16_round(f32(hd16))) + f32(bf16_round(f32(upd16))))
                v_out[0, hh, t0:t1] = bf16_round(f32(v16))
            final[n, hh] = S
    return h_out, v_out, final


# ----------------------------------------------------------------------------- producer / textbook recurrence

def wy_prepare(k: np.ndarray, v: np.ndarray, beta: np.ndarray, a: np.ndarray,
               chunk_size: int = CHUNK_SIZE, cu_seqlens: np.ndarray | None = None,
               rounding: str | None = None):
    """(w, u, g) from keys, values, beta and per-token log-decay ``a`` (token-major).

    Restates ``chunk_gated_delta_rule_golden.py:102-124`` in float64: per chunk
    ``g = cumsum(a)`` (chunk-local), ``A = tril(beta_i k_i.k_j e^{g_i-g_j}, -1)``,
    ``T = (I + A)^{-1}``, ``w = T (beta * e^g * k)``, ``u = T (beta * v)``.
    The reference's forward-substitution loop (``:117-121``) is replaced by a
    triangular solve, which is the same matrix.
    k ``[B,T,Hg,K]`` (head h uses key head h // (H/Hg)), v ``[B,T,H,V]``, beta/a ``[B,T,H]``.

    ``rounding="bf16"`` is the rounding model of the HIP kernel: ``g`` is the float32
    sequential cumsum, ``T`` stays exact, its columns are scaled by ``beta_j e^{g_j}`` (w) or
    ``beta_j`` (u) and rounded to bf16 (the MFMA operand; the reference's bf16 variant rounds
    ``T``, ``beta v`` and ``beta e^g k`` separately, ``chunk_gated_delta_rule_benchmark.py:79-88``),
    the products accumulate exactly and w, u are rounded to bf16.
    """
    if rounding not in (None, "bf16"):
        raise ValueError(f"unknown rounding {rounding!r}")
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    beta = np.asarray(beta, np.float64)
    B, T, Hg, K = k.shape
    H = v.shape[2]
    w = np.zeros((B, T, H, K))
    u = np.zeros(v.shape)
    g = np.zeros((B, T, H))
    seqs, _ = sequence_bounds(B, T, cu_seqlens, chunk_size)
    for (b, bos, eos, _, _) in seqs:
        for t0 in range(bos, eos, chunk_size):
            t1 = min(t0 + chunk_size, eos)
            for hh in range(H):
                kc, vc, bc = k[b, t0:t1, hh * Hg // H], v[b, t0:t1, hh], beta[b, t0:t1, hh]
                if rounding:
                    gc = np.cumsum(np.asarray(a[b, t0:t1, hh], np.float32), dtype=np.float32).astype(np.float64)
                else:
                    gc = np.cumsum(np.asarray(a[b, t0:t1, hh], np.float64))
                L = t1 - t0
                decay = np.exp(gc[:, None] - gc[None, :])
                A = np.tril((bc[:, None] * (kc @ kc.T)) * decay, -1)
                Tm = np.linalg.solve(np.eye(L) + A, np.eye(L))
                if rounding:
                    w[b, t0:t1, hh] = bf16_round(bf16_round(Tm * (bc * np.exp(gc))[None, :]) @ kc)
                    u[b, t0:t1, hh] = bf16_round(bf16_round(Tm * bc[None, :]) @ vc)
                else:
                    w[b, t0:t1, hh] = Tm @ (bc[:, None] * np.exp(gc)[:, None] * kc)
                    u[b, t0:t1, hh] = Tm @ (bc[:, None] * vc)
                g[b, t0:t1, hh] = gc
    return w, u, g


def gated_delta_rule_tokenwise(k: np.ndarray, v: np.ndarray, beta: np.ndarray, a: np.ndarray,
                               initial_state: np.ndarray | None = None,
                               chunk_size: int = CHUNK_SIZE,
                               cu_seqlens: np.ndarray | None = None,
                               q: np.ndarray | None = None, scale: float | None = None):
    """Token-by-token Gated DeltaNet state recurrence in float64.

    ``S_t = e^{a_t} (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T`` with
    ``S`` of shape ``[K, V]``.  Returns the states entering every chunk,
    ``[B, NT, H, K, V]``, and the final states ``[N, H, K, V]``; with queries ``q``
    (``[B,T,H,K]``) also the outputs ``o_t = scale S_t^T q_t`` (``[B,T,H,V]``,
    scale defaulting to ``K**-0.5``).
    """
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, T, H, K = k.shape
    V = v.shape[-1]
    seqs, NT = sequence_bounds(B, T, cu_seqlens, chunk_size)
    states = np.zeros((B, NT, H, K, V))
    final = np.zeros((len(seqs), H, K, V))
    out = None if q is None else np.zeros((B, T, H, V))
    sc = K ** -0.5 if scale is None else scale
    for n, (b, bos, eos, boh, _) in enumerate(seqs):
        for hh in range(H):
            S = np.zeros((K, V)) if initial_state is None else np.array(initial_state[n, hh], np.float64)
            for t in range(bos, eos):
                if (t - bos) % chunk_size == 0:
                    states[b, boh + (t - bos) // chunk_size, hh] = S
                kt, vt = k[b, t, hh], v[b, t, hh]
                S = np.exp(a[b, t, hh]) * S
                S = S + beta[b, t, hh] * np.outer(kt, vt - S.T @ kt)
                if out is not None:
                    out[b, t, hh] = sc * (S.T @ np.asarray(q[b, t, hh], np.float64))
            final[n, hh] = S
    if out is not None:
        return states, final, out
    return states, final


# ----------------------------------------------------------------------------- chunk output

def chunk_o(
    q: np.ndarray,
    k: np.ndarray,
    v_new: np.ndarray,
    h: np.ndarray,
    g: np.ndarray | None = None,
    scale: float | None = None,
    chunk_size: int = CHUNK_SIZE,
    cu_seqlens: np.ndarray | None = None,
    rounding: str | None = None,
    compute_dtype=np.float32,
):
    """Chunk output from the FwdH outputs, token-major layouts.

    q, k ``[B,T,Hg,K]``, v_new ``[B,T,H,V]``, h ``[B,NT,H,K,V]`` (state entering each
    chunk), g ``[B,T,H]`` (chunk-local cumulative log-decay, the FwdH gate) ->
    o ``[B,T,H,V]``::

        o_i = scale * ( e^{g_i} q_i . h_c  +  sum_{j <= i, j in chunk c} (q_i . k_j) e^{g_i - g_j} v_new_j )

    (``chunk_gated_delta_rule_golden.py:136-142``: ``attn_inter + attn @ v_new`` with the
    query scaled by ``scale`` (``:99-100``) and the decay mask ``exp((g_i - g_j).tril())``
    kept on and below the diagonal (``:116``, ``:131-138``)).  ``scale`` defaults to
    ``K**-0.5`` (``:99``).  ``rounding="bf16"``: the masked product
    ``bf16(scale (q_i.k_j) e^{g_i-g_j})`` feeds the second product, both accumulate in
    ``compute_dtype`` and ``o`` is rounded to bf16.
    """
    if chunk_size != CHUNK_SIZE:
        raise ValueError(f"chunk_size must be {CHUNK_SIZE}, got {chunk_size}")
    if rounding not in (None, "bf16"):
        raise ValueError(f"unknown rounding {rounding!r}")
    cd = np.dtype(compute_dtype)
    q = np.asarray(q, cd)
    k = np.asarray(k, cd)
    v_new = np.asarray(v_new, cd)
    h = np.asarray(h, cd)
    B, T, Hg, K = q.shape
    H, V = v_new.shape[2], v_new.shape[3]
    if k.shape != q.shape or v_new.shape[:2] != (B, T) or H % Hg != 0:
        raise ValueError("q and k must be [B,T,Hg,K], v_new [B,T,H,V] with H a multiple of Hg")
    if cu_seqlens is not None and B != 1:
        raise ValueError("cu_seqlens requires B == 1")
    sc = cd.type(K ** -0.5 if scale is None else scale)
    gq = None if g is None else np.asarray(g, cd)
    head_of_key = np.arange(H) // (H // Hg)
    seqs, NT = sequence_bounds(B, T, cu_seqlens, chunk_size)
    if h.shape != (B, NT, H, K, V):
        raise ValueError(f"h must be {(B, NT, H, K, V)}")
    o = np.zeros((B, T, H, V), dtype=cd)
    for (b, bos, eos, boh, _) in seqs:
        for c, t0 in enumerate(range(bos, eos, chunk_size)):
            t1 = min(t0 + chunk_size, eos)
            L = t1 - t0
            Qc = np.transpose(q[b, t0:t1][:, head_of_key, :], (1, 0, 2))   # [H, L, K]
            Kc = np.transpose(k[b, t0:t1][:, head_of_key, :], (1, 0, 2))   # [H, L, K]
            Vc = np.transpose(v_new[b, t0:t1], (1, 0, 2))                   # [H, L, V]
            A = np.matmul(Qc, np.transpose(Kc, (0, 2, 1)))                  # [H, L, L]
            inter = np.matmul(Qc, h[b, boh + c])                            # [H, L, V]
            tri = np.tril(np.ones((L, L), dtype=bool))
            if gq is not None:
                gc = np.transpose(gq[b, t0:t1], (1, 0))                     # [H, L]
                diff = np.where(tri, gc[:, :, None] - gc[:, None, :], 0)
                A = A * np.exp(diff).astype(cd)
                inter = inter * np.exp(gc).astype(cd)[:, :, None]
            A = np.where(tri, A * sc, 0).astype(cd)
            if rounding:
                A = bf16_round(A)
            oc = inter * sc + np.matmul(A, Vc)
            if rounding:
                oc = bf16_round(oc)
            o[b, t0:t1] = np.transpose(oc, (1, 0, 2))
    return o


# ----------------------------------------------------------------------------- synthetic inputs

def make_gate(rng: np.random.Generator, B: int, T: int, H: int, kind: str = "logsigmoid",
              cu_seqlens: np.ndarray | None = None, chunk_size: int = CHUNK_SIZE, shift: float = 0.0):
    """Chunk-local cumulative log-decay ``g [B,T,H]`` (non-increasing, <= 0 in every chunk).

    kind="logsigmoid": cumsum of ``logsigmoid(randn + shift)`` restarted at every chunk
    (the benchmark configurations' distributions; shift=-2 is the strongly decaying variant).
    kind="linear": ``g = -rate * (1..L)`` with ``rate = 0.01 + 0.0025 (h % 5)``, the mild gate of
    ``code/tests/golden/generate_golden.py:443-459``.
    """
    if kind == "logsigmoid":
        z = rng.standard_normal((B, T, H)).astype(np.float32) + np.float32(shift)
        inc = -np.logaddexp(np.float32(0.0), -z).astype(np.float32)
    elif kind == "linear":
        rate = (0.01 + 0.0025 * (np.arange(H) % 5)).astype(np.float32)
        inc = np.broadcast_to(-rate, (B, T, H)).astype(np.float32)
    else:
        raise ValueError(kind)
    g = np.zeros((B, T, H), np.float32)
    seqs, _ = sequence_bounds(B, T, cu_seqlens, chunk_size)
    for (b, bos, eos, _, _) in seqs:
        for t0 in range(bos, eos, chunk_size):
            t1 = min(t0 + chunk_size, eos)
            g[b, t0:t1] = np.cumsum(inc[b, t0:t1], axis=0, dtype=np.float32)
    return g


def make_inputs(seed: int, B: int, T: int, H: int, K: int, V: int, Hg: int | None = None,
                dtype: str = "bf16", gate: str | None = "logsigmoid", gate_shift: float = 0.0,
                with_h0: bool = True, cu_seqlens: np.ndarray | None = None, h0_scale: float = 0.1,
                profile: str = "baseline"):
    """Seeded synthetic FwdH inputs.

    profile="baseline": k = L2-normalised randn over K; w = randn * K^-1/2; u = randn;
        h0 = randn * h0_scale (the benchmark configurations' distributions).  With a mild gate this w makes
        the per-chunk state transition exp(g_last) I - K^T diag(gamma) W expansive
        (spectral radius > 1), so long sequences amplify rounding differences; with the
        benchmark configurations' logsigmoid gate exp(g_last) ~ 1e-22 and every chunk starts afresh.
    profile="golden": k, u ~ U(-1,1), w ~ U(-1,1)/K, h0 ~ randn * 0.25
        (``code/tests/golden/generate_golden.py:472-490``); small w keeps the transition
        contracting.
    profile="wy": w, u produced by ``wy_prepare`` from L2-normalised keys, randn values,
        beta = sigmoid(randn) and the gate's per-token log-decay: the inputs a Gated
        DeltaNet layer really feeds this operator, whose transitions are contractions.
        g is then the chunk-local cumsum of that decay (gate "logsigmoid" with gate_shift).
    For dtype="bf16" k/w/u are rounded to bf16 values (float32 arrays holding bf16 values);
    g and h0 are float32.
    """
    rng = np.random.default_rng(seed)
    Hg = H if Hg is None else Hg
    N = B if cu_seqlens is None else len(cu_seqlens) - 1
    if profile == "baseline":
        k = rng.standard_normal((B, T, Hg, K)).astype(np.float32)
        k /= np.maximum(np.linalg.norm(k, axis=-1, keepdims=True), 1e-6)
        w = (rng.standard_normal((B, T, H, K)) * K ** -0.5).astype(np.float32)
        u = rng.standard_normal((B, T, H, V)).astype(np.float32)
        h0 = (rng.standard_normal((N, H, K, V)) * h0_scale).astype(np.float32) if with_h0 else None
        g = None if gate is None else make_gate(rng, B, T, H, gate, cu_seqlens, shift=gate_shift)
    elif profile == "golden":
        k = (rng.random((B, T, Hg, K)) * 2 - 1).astype(np.float32)
        w = ((rng.random((B, T, H, K)) * 2 - 1) / K).astype(np.float32)
        u = (rng.random((B, T, H, V)) * 2 - 1).astype(np.float32)
        h0 = (rng.standard_normal((N, H, K, V)) * 0.25).astype(np.float32) if with_h0 else None
        g = None if gate is None else make_gate(rng, B, T, H, gate, cu_seqlens, shift=gate_shift)
    elif profile == "wy":
        k = rng.standard_normal((B, T, Hg, K))
        k /= np.maximum(np.linalg.norm(k, axis=-1, keepdims=True), 1e-6)
        v = rng.standard_normal((B, T, H, V))
        beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H))))
        z = rng.standard_normal((B, T, H)) + gate_shift
        a = -np.logaddexp(0.0, -z) if gate is not None else np.zeros((B, T, H))
        kfull = np.repeat(k, H // Hg, axis=2)
        w, u, gc = wy_prepare(kfull, v, beta, a, cu_seqlens=cu_seqlens)
        k, w, u = k.astype(np.float32), w.astype(np.float32), u.astype(np.float32)
        g = None if gate is None else gc.astype(np.float32)
        h0 = (rng.standard_normal((N, H, K, V)) * h0_scale).astype(np.float32) if with_h0 else None
    else:
        raise ValueError(profile)
    if dtype == "bf16":
        k, w, u = bf16_round(k), bf16_round(w), bf16_round(u)
    elif dtype != "f32":
        raise ValueError(dtype)
    return dict(k=k, w=w, u=u, g=g, initial_state=h0, cu_seqlens=cu_seqlens)


def varlen_cu_seqlens(seed: int, n: int, lo: int, hi: int, chunk_size: int = CHUNK_SIZE) -> np.ndarray:
    """``n`` seeded lengths uniform in ``[lo, hi]``, each moved off multiples of the chunk size."""
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=n)
    lens = np.where(lens % chunk_size == 0, lens + np.where(lens + 1 <= hi, 1, -1), lens)
    return np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
