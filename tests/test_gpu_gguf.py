"""Real-model ingestion on the GPU: layers written as a GGUF file (tests/gguf_writer.py), opened with the
library's reader, uploaded from the mapped tensors (phx_gguf_layer_desc -> phx_moe_layer_upload) and
run, against the CPU oracle on the same layers: ids and lists bit-exact, gate/up/down products bit
for bit, outputs bit for bit through the exact router and within tolerance otherwise."""
import sys

import pytest

import gguf_writer as GW
from test_gpu_parity import check_layer

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


CASES = {
    # C2 shapes: Q4_0 experts and the layer's Q4_0 dense FFN as the shared FFN
    "c2_q4_0": ("c2_decode", 2, [(1, False), (8, False), (40, False), (4, True)]),
    # K-quants with whole-block down rows (n_ff = 512)
    "kquant": (dict(idx=24, T=8, d=1024, E=16, k=4, nf=512, gu=12, dn=14), 1, [(12, False), (3, True)]),
    # a Q5_K_M-like layer: Q5_K gate|up, Q3_K down (GGUF types 13 and 11), the dense FFN in Q5_K
    "q5k_q3k": (dict(idx=25, T=8, d=512, E=8, k=2, nf=512, gu=13, dn=11, nff=512, sh=13), 1, [(6, False), (40, True)]),
}


@pytest.mark.parametrize("case", list(CASES))
def test_gguf_layers_on_gpu(ctx, pkg, orc, tmp_path, case):
    cfg, n, runs = CASES[case]
    say(f"gguf {case}: writing {n} layers ...")
    layers = [pkg.synth.make_layer(cfg, layer=i, norms="noisy") for i in range(n)]
    path = GW.moe_model(layers).write(tmp_path / "model.gguf")
    with pkg.gguf.GgufFile.Open(str(path)) as g:
        assert g.moe_config()["n_layer"] == n
        for i, L in enumerate(layers):
            pkg.gguf.upload_layer(ctx, g, i, without_shared=not L.get("n_ff_shared"))
    for i, L in enumerate(layers):
        for T, exact in runs:
            x = pkg.synth.make_input(cfg, T=T, seed=77 + i)
            check_layer(ctx, orc, L, x, tag=f"gguf {case} layer {i} T={T} exact={exact}", exact=exact, layer=i)
