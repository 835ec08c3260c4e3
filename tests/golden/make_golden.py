#!/usr/bin/env python3
"""Writes the golden fixtures of tests/golden/ from the CPU oracle (oracle/) and the seeded synthetic
layers (phoenix-lai_amd/synth.py).

The reference holds no golden vectors for the MoE path (its kernel tests keep no stored outputs), so
these fixtures freeze the oracle's outputs once it has passed its pins (tests/test_oracle_*.py):
later changes to the oracle, the synthetic generator or the GPU path are compared against them.
Weights are not stored (megabytes); their SHA-256 over the GGUF bytes is, and the tests regenerate
them from the seeds and check the digest first.

  c1_tiny.npz     configs[0] at full size: T=16, d=512, E=8, top-2, ffn 1024, Q4_0, N(1, 0.1) norms,
                  a random `shared` input; outputs for both weight rules, logits, expert lists.
  kquant_tiny.npz Q4_K gate|up, Q6_K down with the down K-dimension padded 288 -> 512, T=4.
  c3_hist.npz     the realised expert histogram of configs[2] (T=2048, E=128, top-8, Zipf(1.1) bias).

Run: python tests/golden/make_golden.py  (about a minute on 8 cores).
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

KQ_CFG = dict(idx=10, T=4, d=512, E=4, k=2, nf=288, gu=12, dn=14)


def package():
    import __graft_entry__ as ge
    if not ge._built():
        ge.build()
    return ge.load_package()


def layer_digest(L: dict) -> str:
    h = hashlib.sha256()
    for k in sorted(L):
        v = L[k]
        if isinstance(v, np.ndarray):
            h.update(k.encode())
            h.update(np.ascontiguousarray(v).tobytes())
    return h.hexdigest()


def c1_inputs(S):
    L = S.make_layer("c1_tiny", norms="noisy")
    x = S.make_input("c1_tiny")
    shared = S.normal(1001, "golden.shared", x.shape)
    return L, x, shared


def kq_inputs(S):
    L = S.make_layer(KQ_CFG)
    x = S.make_input(KQ_CFG)
    return L, x


def c3_router_inputs(S):
    L = S.make_layer("c3_prefill", experts=False)
    x = S.make_input("c3_prefill")
    return L, x


def c3_hist(orc, L, x):
    ids = np.stack([orc.router(L, x[t])[1] for t in range(x.shape[0])])
    return ids, np.bincount(ids.reshape(-1), minlength=L["n_expert"]).astype(np.int32)


def main():
    from oracle import oracle as orc
    pkg = package()
    S = pkg.synth

    L, x, shared = c1_inputs(S)
    rec = dict(layer_sha256=np.array(layer_digest(L)), x=x, shared=shared)
    for rule in (0, 1):
        L["weight_rule"] = rule
        out, ids, w = orc.moe_block(L, x, shared)
        rec[f"out_r{rule}"], rec[f"ids_r{rule}"], rec[f"w_r{rule}"] = out, ids, w
    L["weight_rule"] = 0
    rec["logits"] = np.stack([orc.router(L, x[t])[0] for t in range(x.shape[0])])
    rec["offsets"], rec["perm"] = orc.bucket(rec["ids_r0"], L["n_expert"])
    np.savez_compressed(HERE / "c1_tiny.npz", **rec)

    L, x = kq_inputs(S)
    out, ids, w = orc.moe_block(L, x)
    np.savez_compressed(HERE / "kquant_tiny.npz", layer_sha256=np.array(layer_digest(L)), x=x, out=out, ids=ids, w=w)

    L, x = c3_router_inputs(S)
    ids, hist = c3_hist(orc, L, x)
    np.savez_compressed(HERE / "c3_hist.npz", router_sha256=np.array(layer_digest(L)),
                        ids_sha256=np.array(hashlib.sha256(ids.tobytes()).hexdigest()), hist=hist)
    print("hist (sorted):", np.sort(hist)[::-1][:16], "... distinct", int((hist > 0).sum()))


if __name__ == "__main__":
    main()
