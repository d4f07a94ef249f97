"""The SigLIP-B encoder layer through the library (softhier_mlir_amd.encoder) against the oracle: the
reference's LCG layer (siglip_ref.py seeds, S=256) with both call sequences, BASELINE config 5 at B=32
(1 layer) and a 12-layer stack."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import to_dev, to_np
from oracle import refs
from softhier_mlir_amd import data, encoder

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("sequence", ["reference", "fused"])
def test_reference_lcg_layer(lib, gpu, sequence):
    S, D, F, H = 256, 768, 3072, 12
    p = refs.siglip_params_lcg(D, F)
    x = refs.siglip_input_lcg(S, D)
    enc = encoder.Encoder(D, F, H)
    out = enc.forward(to_dev(x), [encoder.LayerParams.from_host(p)], B=1, S=S, sequence=sequence)
    want = refs.encoder_layer(x, p, H)
    bad, err, _ = refs.close(to_np(out), want)
    assert bad == 0, err


@pytest.mark.parametrize("sequence", ["fused", "reference"])
def test_baseline_config5_b32(lib, gpu, sequence):
    B, S, D, F, H = 32, 256, 768, 3072, 12
    p = data.encoder_params(D, F, seed=100)
    x = data.normal((B * S, D), 7)
    enc = encoder.Encoder(D, F, H)
    out = enc.forward(to_dev(x), [encoder.LayerParams.from_host(p)], B=B, S=S, sequence=sequence)
    want = refs.encoder_layer(x, p, H, B=B)
    bad, err, _ = refs.close(to_np(out), want)
    assert bad == 0, err


def test_twelve_layer_stack(lib, gpu):
    B, S, D, F, H = 2, 256, 768, 3072, 12
    ps = [data.encoder_params(D, F, seed=200 + 20 * i) for i in range(12)]
    x = data.normal((B * S, D), 8)
    enc = encoder.Encoder(D, F, H)
    out = enc.forward(to_dev(x), [encoder.LayerParams.from_host(p) for p in ps], B=B, S=S, sequence="fused")
    want = refs.encoder_stack(x, ps, H, B=B)
    bad, err, _ = refs.close(to_np(out), want)
    assert bad == 0, err


def test_fused_stack_reference_lcg_layers(lib, gpu):
    """The fused sequence over four layers with the reference's LCG parameter table, whose seeds move by 100 per
    layer (siglip.py:110-124): non-trivial gamma / beta and biases reach every folded GEMM, and layers 1-3 take
    their LayerNorm statistics from the row partials the previous layer's FFN-down wrote. Two sequences (the
    reference's LCG input and a second one derived from it), every element against the oracle's stack."""
    S, D, F, H, B = 256, 768, 3072, 12, 2
    x0 = refs.siglip_input_lcg(S, D)
    x = np.concatenate([x0, (-x0.astype(np.float32)[::-1]).astype(np.float16)], 0)
    ps = [refs.siglip_params_lcg(D, F, layer=L) for L in range(4)]
    enc = encoder.Encoder(D, F, H)
    out = enc.forward(to_dev(x), [encoder.LayerParams.from_host(p) for p in ps], B=B, S=S, sequence="fused")
    got = to_np(out)
    want = refs.encoder_stack(x, ps, H, B=B)
    bad, err, _ = refs.close(got, want)
    assert bad == 0, err
    assert np.isfinite(got).all()


def test_stack_prefetch_changes_no_bits(lib, gpu):
    """The stack with its weight prefetch (each layer's attention reads the layer's later weights and the next layer's
    QKV weight into the caches) stores exactly the bits of the stack without it: the prefetch only reads."""
    import torch
    B, S, D, F, H = 2, 256, 768, 3072, 12
    ps = [encoder.LayerParams.from_host(data.encoder_params(D, F, seed=300 + i)) for i in range(4)]
    x = to_dev(data.normal((B * S, D), 9))
    outs = []
    for pre in (True, False):
        enc = encoder.Encoder(D, F, H)
        enc.prefetch = pre
        outs.append(enc.forward(x, ps, B=B, S=S, sequence="fused").clone())
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    bad, err, _ = refs.close(to_np(outs[0]), refs.encoder_stack(data.normal((B * S, D), 9),
                                                                [{k: v.cpu().numpy() for k, v in p.t.items()} for p in ps], H, B=B))
    assert bad == 0, err


def test_baseline_config5_twelve_layer_stack_b32(lib, gpu):
    """BASELINE config 5 as configured: the 12-layer stack at B = 32, S = 256 (layer l seeded 100 + l, input
    seed 7: the workload bench.py measures), every element of the last layer's output against the oracle's
    12-layer stack (siglip.py:133-168 per layer, the layer loop of siglip.py:168)."""
    B, S, D, F, H = 32, 256, 768, 3072, 12
    ps = [data.encoder_params(D, F, seed=100 + i) for i in range(12)]
    x = data.normal((B * S, D), 7)
    enc = encoder.Encoder(D, F, H)
    out = enc.forward(to_dev(x), [encoder.LayerParams.from_host(p) for p in ps], B=B, S=S, sequence="fused")
    got = to_np(out)
    want = refs.encoder_stack(x, ps, H, B=B)
    bad, err, _ = refs.close(got, want)
    assert bad == 0, err
    assert np.isfinite(got).all()


def test_captured_layer_graph_replays_match_eager(lib, gpu):
    """The fused layer recorded into a HIP graph: every replay (with eager library work and synchronisations
    between replays, and a new input copied into the captured buffer) stores exactly what the eager call
    sequence stores for the same input."""
    import torch
    B, S, D, F, H = 4, 256, 768, 3072, 12
    p = encoder.LayerParams.from_host(data.encoder_params(D, F, seed=100))
    enc = encoder.Encoder(D, F, H)
    x = to_dev(data.normal((B * S, D), 7))
    out = torch.empty_like(x)
    g = enc.capture(x, out, p, B, S)
    eager = torch.empty_like(x)
    for seed in (7, 8, 9):
        x.copy_(to_dev(data.normal((B * S, D), seed)))
        g.replay()
        torch.cuda.synchronize()
        got = out.clone()
        enc.layer_fused(x, eager, p, B, S)          # eager work between replays (same buffers for the scratch)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), eager.view(torch.int16))
    want = refs.encoder_layer(data.normal((B * S, D), 9), {k: v.cpu().numpy() for k, v in p.t.items()}, H, B=B)
    bad, err, _ = refs.close(to_np(out), want)
    assert bad == 0, err


def test_captured_layer_survives_a_call_with_another_row_count(lib, gpu):
    """A captured layer keeps the scratch buffers it addresses: after an eager call with another batch size (which
    replaces the encoder's scratch set), replaying the graph still stores what the eager layer stores."""
    import torch
    B, S, D, F, H = 2, 256, 768, 3072, 12
    p = encoder.LayerParams.from_host(data.encoder_params(D, F, seed=100))
    enc = encoder.Encoder(D, F, H)
    x = to_dev(data.normal((B * S, D), 7))
    out = torch.empty_like(x)
    g = enc.capture(x, out, p, B, S)
    x3 = to_dev(data.normal((3 * S, D), 8))
    enc.layer_fused(x3, torch.empty_like(x3), p, 3, S)       # another row count: a new scratch set
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    junk = torch.full((64 << 20,), 7, dtype=torch.float16, device="cuda")   # reuse whatever the cache freed
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    eager = torch.empty_like(x)
    enc.layer_fused(x, eager, p, B, S)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), eager.view(torch.int16))
    del junk
