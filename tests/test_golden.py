"""The committed golden fixtures (tests/golden/, written by tests/golden/make_golden.py): the seeded
generator still produces the same layers, and the oracle still reproduces the stored outputs bit for
bit.  The GPU path is compared with the same fixtures in tests/test_gpu_parity.py.  CPU only."""
import hashlib
import sys
from pathlib import Path

import numpy as np

GOLD = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLD))

import make_golden as MG  # noqa: E402


def _load(name):
    return np.load(GOLD / name)  # allow_pickle is False by default


def test_c1_fixture(orc, pkg):
    f = _load("c1_tiny.npz")
    L, x, shared = MG.c1_inputs(pkg.synth)
    assert MG.layer_digest(L) == str(f["layer_sha256"])
    assert np.array_equal(x, f["x"]) and np.array_equal(shared, f["shared"])
    for rule in (0, 1):
        L["weight_rule"] = rule
        out, ids, w = orc.moe_block(L, x, shared)
        assert np.array_equal(ids, f[f"ids_r{rule}"])
        assert np.array_equal(w.view(np.uint32), f[f"w_r{rule}"].view(np.uint32))
        assert np.array_equal(out.view(np.uint32), f[f"out_r{rule}"].view(np.uint32))
    off, perm = orc.bucket(f["ids_r0"], L["n_expert"])
    assert np.array_equal(off, f["offsets"]) and np.array_equal(perm, f["perm"])


def test_c1_fixture_invariants():
    f = _load("c1_tiny.npz")
    ids, logits = f["ids_r0"], f["logits"]
    T, k = ids.shape
    assert (T, k) == (16, 2)
    for t in range(T):
        order = np.lexsort((np.arange(logits.shape[1]), -logits[t].astype(np.float64)))
        assert list(ids[t]) == list(order[:k])
    assert np.array_equal(f["ids_r1"], ids)  # the weight rule never changes the selection
    assert f["offsets"][-1] == T * k


def test_kquant_fixture(orc, pkg):
    f = _load("kquant_tiny.npz")
    L, x = MG.kq_inputs(pkg.synth)
    assert L["down_cols"] == 512 and L["n_ff"] == 288
    assert MG.layer_digest(L) == str(f["layer_sha256"])
    out, ids, w = orc.moe_block(L, x)
    assert np.array_equal(ids, f["ids"])
    assert np.array_equal(out.view(np.uint32), f["out"].view(np.uint32))


def test_c3_zipf_histogram(orc, pkg):
    f = _load("c3_hist.npz")
    L, x = MG.c3_router_inputs(pkg.synth)
    assert MG.layer_digest(L) == str(f["router_sha256"])
    ids, hist = MG.c3_hist(orc, L, x)
    assert hashlib.sha256(ids.tobytes()).hexdigest() == str(f["ids_sha256"])
    assert np.array_equal(hist, f["hist"])
    # the realised popularity is Zipf-like: the top experts are capped near T, the tail is long
    s = np.sort(hist)[::-1]
    assert hist.sum() == 2048 * 8 and s[0] <= 2048 and s[0] > 10 * s[64] and (hist > 0).sum() >= 100
