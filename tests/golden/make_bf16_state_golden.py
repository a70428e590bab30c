"""Write input/output vectors of the reference's bf16 benchmark recurrence as test fixtures.

Runs only in the build container, where the reference is mounted read-only: it imports
``ref/chunk_gated_delta_rule/tests/pytest/chunk_gated_delta_rule_benchmark.py`` (torch only)
and calls its ``stage1_opt`` and ``stage2_opt`` (``:13-93``, ``:96-142``) on seeded inputs
drawn as the reference's input adapter draws them (``tests/assets/impl/inputs.py``:
L2-normalised q and k, g in [-1, 0], beta in (0, 1)), with a bf16 initial state.  No
check of this repository pins that recurrence otherwise.

Each case is stored in the FwdH form the oracle's ``fwd_h_bf16_state`` takes, token-major:
k ``[1,T,Hk,K]`` (the raw keys), w = -k_cumdecay ``[1,T,H,K]``, u = v_inner ``[1,T,H,V]``,
g = g_cum ``[1,T,H]``, h0 ``[N,H,K,V]`` (the benchmark's ``[H,V,K]`` state transposed),
cu_seqlens, and the benchmark's outputs v_new ``[1,T,H,V]``, final ``[N,H,K,V]`` and the
gated keys kg ``[1,T,H,K]``; bf16 values as float32, in ``.npz`` files (no pickles).

    python tests/golden/make_bf16_state_golden.py [--out tests/golden/bf16_state]
"""

from __future__ import annotations

import argparse
import importlib.util
import pathlib

import numpy as np
import torch
import torch.nn.functional as F

REFERENCE_BENCHMARK = pathlib.Path(
    "/root/reference/ChunkGatedDeltaRuleFwdH_problem_290_template/ref/chunk_gated_delta_rule/tests/pytest/"
    "chunk_gated_delta_rule_benchmark.py")

C = 64
# name: (sequence lengths, key heads, value heads, head dim, seed)
CASES = {
    "gqa_partial": ([200], 2, 4, 64, 0),
    "d128_two_chunks": ([128], 1, 2, 128, 1),
    "varlen_two_seqs": ([70, 130], 2, 2, 64, 2),
    "long_d32": ([640], 1, 1, 32, 3),
}


def _case(mod, lens, nk, nv, d, seed):
    gen = torch.Generator().manual_seed(seed)
    T = sum(lens)
    q = F.normalize(torch.randn(T, nk, d, generator=gen), dim=-1).to(torch.bfloat16)
    k = F.normalize(torch.randn(T, nk, d, generator=gen), dim=-1).to(torch.bfloat16)
    v = torch.randn(T, nv, d, generator=gen).to(torch.bfloat16)
    g = -torch.rand(T, nv, generator=gen)
    beta = torch.sigmoid(torch.randn(T, nv, generator=gen))
    state0 = (0.1 * torch.randn(len(lens), nv, d, d, generator=gen)).to(torch.bfloat16)   # [N, H, V, K]
    out = {n: [] for n in ("w", "u", "g", "v_new", "kg")}
    finals = []
    start = 0
    for i, L in enumerate(lens):
        sl = slice(start, start + L)
        g_cum, k_cumdecay, v_inner, q_prime, kg, _ = mod.stage1_opt(q[sl], k[sl], v[sl], g[sl], beta[sl],
                                                                   d ** -0.5, C)
        final, _, v_new = mod.stage2_opt(q_prime, v_inner, g_cum, k_cumdecay, state0[i].clone(), kg, C)
        tm = lambda x: x[:, :L].transpose(0, 1).float()          # [H, Sp, D] -> [L, H, D]
        out["w"].append(-tm(k_cumdecay))
        out["u"].append(tm(v_inner))
        out["g"].append(g_cum[:, :L].transpose(0, 1).float())
        out["v_new"].append(tm(v_new))
        out["kg"].append(tm(kg))
        finals.append(final.transpose(-1, -2).float())            # [H, V, K] -> [H, K, V]
        start += L
    arrs = {n: torch.cat(x, 0)[None].numpy() for n, x in out.items()}
    arrs["k"] = k.float()[None].numpy()
    arrs["h0"] = state0.transpose(-1, -2).float().numpy()
    arrs["final"] = torch.stack(finals, 0).numpy()
    arrs["cu_seqlens"] = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    return arrs


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", type=pathlib.Path, default=pathlib.Path(__file__).parent / "bf16_state")
    args = ap.parse_args()
    spec = importlib.util.spec_from_file_location("reference_benchmark", REFERENCE_BENCHMARK)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    args.out.mkdir(parents=True, exist_ok=True)
    torch.set_num_threads(1)
    for name, (lens, nk, nv, d, seed) in CASES.items():
        arrs = _case(mod, lens, nk, nv, d, seed)
        np.savez_compressed(args.out / f"{name}.npz", **{n: np.ascontiguousarray(a) for n, a in arrs.items()})
        print(name, {n: a.shape for n, a in arrs.items()})


if __name__ == "__main__":
    main()
