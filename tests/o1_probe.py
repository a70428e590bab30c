"""One-hot probe inputs that pin the rounding points of the bf16 (Triton, "O1") model.

The Triton kernel (``docs/problem.txt:353-422`` of the reference) rounds in four places:
  * ``b_h.to(bf16)`` is both the stored snapshot ``h[c]`` and the ``W @ .`` operand (``:356-360``,
    ``:392-394``): MM1 sees ``bf16(S)``;
  * ``v_new`` is stored from the fp32 ``u - W bf16(S)`` before any gating (``:396-398``);
  * the gated value ``(u - W bf16(S)) * gamma`` is rounded to bf16 once, as the ``K^T @ .``
    operand (``:400-405``);
  * the carried state stays fp32 (``b_h1_bv1`` is an fp32 block, ``:330-331``, decayed and
    accumulated in fp32).

With every row of W and of K one-hot, each contraction has exactly one nonzero product, so
it is exact in any summation order and the outputs follow from those four rules alone:

  chunk c, token m:  W[m] = e_{i(c,m)},  K[m] = e_{16+m} for m < 16 (else 0),
                     g[m] = d[c,m] for m < 16, g = 0 elsewhere, so g_last = 0, a = 1 and
                     gamma_m = exp(-d[c,m])
  v_new[m]   = bf16(u[m] - bf16(S)[i(c,m)])
  Vd[m]      = bf16((u[m] - bf16(S)[i(c,m)]) * gamma_m)                  (m < 16)
  S[16 + m] += Vd[m]   (fp32),   every other row of S is carried unchanged

Rows 0..15 of the initial state hold fp32 values that bf16 cannot represent; tokens m >= 16
read them (i = m % 16) in every chunk, and they reach the final state unchanged.  Tokens
m < 16 read row m in chunk 0 and row 16 + m (the running sums of the Vd values) later.

``closed_form`` evaluates these rules element by element; ``gamma_margin_ok`` checks that no
Vd lands within 2^-20 (relative) of a bf16 rounding boundary, so a 1-ulp difference between
the device's fp32 exp and numpy's cannot change a result, and the GPU comparison is exact.
"""

from __future__ import annotations

import numpy as np

from oracle import cgdr_oracle as O

PROBE_ROWS = 16   # rows 0..15: fp32 values bf16 cannot hold; rows 16..31: running Vd sums


def _w_row(c: int, m: int) -> int:
    return (16 + m) if (m < 16 and c >= 1) else (m % 16)


def probe_inputs(K: int, V: int, n_chunks: int, H: int = 1, seed: int = 0) -> dict:
    """Token-major inputs (B=1, T=64*n_chunks, Hg=H) as float32 arrays of bf16 values
    (k, w, u), fp32 g (g_last = 0 in every chunk) and an fp32 initial state."""
    assert K >= 32, "the probe needs rows 0..31 of the state"
    rng = np.random.default_rng(seed)
    T = 64 * n_chunks
    k = np.zeros((1, T, H, K), np.float32)
    w = np.zeros((1, T, H, K), np.float32)
    g = np.zeros((1, T, H), np.float32)
    for c in range(n_chunks):
        for m in range(64):
            t = 64 * c + m
            w[0, t, :, _w_row(c, m)] = 1.0
            if m < 16:
                k[0, t, :, 16 + m] = 1.0
                g[0, t, :] = rng.uniform(0.05, 2.0, H).astype(np.float32)
    # u: bf16 values from 2^-12 to 2, either sign, so that u - bf16(S) keeps bits below bf16's
    mag = np.exp2(rng.uniform(-12, 1, (1, T, H, V)))
    u = O.bf16_round((mag * rng.choice([-1.0, 1.0], mag.shape)).astype(np.float32))
    h0 = np.zeros((1, H, K, V), np.float32)
    base = O.bf16_round(rng.uniform(0.5, 2.0, (H, PROBE_ROWS, V)).astype(np.float32))
    frac = rng.choice(np.array([2.0 ** -9, 3 * 2.0 ** -10, -(2.0 ** -9), 5 * 2.0 ** -11]), base.shape)
    h0[0, :, :PROBE_ROWS] = (base * (1.0 + frac)).astype(np.float32)
    assert not np.array_equal(O.bf16_round(h0), h0)
    # Move every u whose gated value would sit within MARGIN of a bf16 rounding boundary to
    # the next bf16 value away from zero (chunk by chunk: later Vn depend on earlier Vd).
    for hh in range(H):
        S = h0[0, hh].copy()
        for c in range(n_chunks):
            Sb = O.bf16_round(S)
            vd = np.zeros((16, V), np.float32)
            for m in range(16):
                t = 64 * c + m
                i = _w_row(c, m)
                gamma = _gamma(g[0, t, hh])
                for _ in range(64):
                    vn = (u[0, t, hh] - Sb[i]).astype(np.float32)
                    bad = ~_stable(vn, gamma)
                    if not bad.any():
                        break
                    up = u[0, t, hh].view(np.uint32) + np.uint32(1 << 16)
                    u[0, t, hh] = np.where(bad, up.view(np.float32), u[0, t, hh])
                vd[m] = O.bf16_round((vn * gamma).astype(np.float32))
            S[16:32] = (S[16:32] + vd).astype(np.float32)
    return dict(k=k, w=w, u=u, g=g, initial_state=h0, cu_seqlens=None)


MARGIN = 2.0 ** -20


def _gamma(gt) -> np.float32:
    return np.exp(np.asarray([np.float32(0.0) - np.float32(gt)], np.float32))[0]


def _stable(vn: np.ndarray, gamma, rel: float = MARGIN) -> np.ndarray:
    """Per element: bf16(fl32(vn * gamma')) is the same for gamma' = gamma (1 +- rel)."""
    outs = [O.bf16_round((vn.astype(np.float64) * float(gamma) * f).astype(np.float32))
            for f in (1 - rel, 1.0, 1 + rel)]
    return (outs[0] == outs[1]) & (outs[1] == outs[2])


def closed_form(inp: dict):
    """(h, v_new, final) of the bf16 model from the four rounding rules above."""
    k, w, u, g, h0 = inp["k"], inp["w"], inp["u"], inp["g"], inp["initial_state"]
    _, T, H, K = w.shape
    V = u.shape[-1]
    n_chunks = T // 64
    h = np.zeros((1, n_chunks, H, K, V), np.float32)
    v_new = np.zeros((1, T, H, V), np.float32)
    final = np.zeros((1, H, K, V), np.float32)
    for hh in range(H):
        S = h0[0, hh].astype(np.float32).copy()
        for c in range(n_chunks):
            Sb = O.bf16_round(S)
            h[0, c, hh] = Sb
            vd = np.zeros((16, V), np.float32)
            for m in range(64):
                t = 64 * c + m
                i = int(np.argmax(w[0, t, hh]))
                vn = (u[0, t, hh] - Sb[i]).astype(np.float32)
                v_new[0, t, hh] = O.bf16_round(vn)
                if m < 16:
                    vd[m] = O.bf16_round((vn * _gamma(g[0, t, hh])).astype(np.float32))
            S[16:32] = (S[16:32] + vd).astype(np.float32)
        final[0, hh] = S
    return h, v_new, final


def gamma_margin_ok(inp: dict) -> bool:
    """True when every gated value Vn * gamma of the probe keeps its bf16 rounding under a
    relative change of gamma by +-MARGIN (so the result does not depend on which correctly
    rounded or 1-ulp-off fp32 exp computed gamma)."""
    w, u, g, h0 = inp["w"], inp["u"], inp["g"], inp["initial_state"]
    _, T, H, K = w.shape
    for hh in range(H):
        S = h0[0, hh].astype(np.float32).copy()
        for c in range(T // 64):
            Sb = O.bf16_round(S)
            vd = np.zeros((16, u.shape[-1]), np.float32)
            for m in range(16):
                t = 64 * c + m
                vn = (u[0, t, hh] - Sb[_w_row(c, m)]).astype(np.float32)
                gamma = _gamma(g[0, t, hh])
                if not _stable(vn, gamma).all():
                    return False
                vd[m] = O.bf16_round((vn * gamma).astype(np.float32))
            S[16:32] = (S[16:32] + vd).astype(np.float32)
    return True
