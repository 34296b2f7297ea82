"""GPU parity of the two-layer decode step (the seven quantized linears per
layer on librq, the glue in f32) against the C oracle's decoder layer
(oracle/rq_oracle.c rqo_decoder_layer, which restates the glue ops of
raster/dl/nn.clj and raster/dl/attention.clj over qlinear-q8).

Bar: normwise max|y - ref| / max|ref| < 1e-3 on the layer outputs and on the
new K / V cache rows (f32 activations; the reference's own decoder-layer test
uses 2e-2, test/raster/dl/decoder_layer_gpu_test.clj:82)."""
import numpy as np
import pytest

from raster_amd import workloads as wl

pytestmark = pytest.mark.gpu

TOL = 1e-3


@pytest.fixture(scope="module")
def torch():
    import torch as t

    if not t.cuda.is_available():
        pytest.skip("no GPU")
    return t


@pytest.fixture(scope="module")
def ctx(torch):
    import raster_amd

    c = raster_amd.Context(0)
    yield c
    c.close()


def run_decoder(torch, ctx, cfg, layers, x, graph=False, replays=1, fused=True):
    from raster_amd.decoder import DecoderLayer

    dl = [DecoderLayer(ctx, L["weights"], L["gain1"], L["gain2"], cfg["d"], cfg["n_q"], cfg["n_kv"],
                       cfg["head_dim"], cfg["ffn"], cfg["eps"], cfg["theta"], fused=fused) for L in layers]
    kcs = [torch.from_numpy(L["kcache"]).cuda() for L in layers]
    vcs = [torch.from_numpy(L["vcache"]).cuda() for L in layers]
    pos = cfg["cached"]
    xin = torch.from_numpy(x).cuda()

    def step():
        h = xin
        for layer, kc, vc in zip(dl, kcs, vcs):
            h = layer.step(h, kc, vc, pos)
        return h

    outs = []
    if graph:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            step()  # warm-up: rope tables, torch workspaces
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            y = step()
        for _ in range(replays):
            g.replay()
            torch.cuda.synchronize()
            outs.append(y.cpu().numpy().copy())
            _ = torch.ones(16, device="cuda").sum().item()  # eager work between replays
    else:
        outs.append(step().cpu().numpy())
    torch.cuda.synchronize()
    res = (outs, [k.cpu().numpy() for k in kcs], [v.cpu().numpy() for v in vcs])
    for layer in dl:
        layer.destroy()
    return res


def oracle_decoder(orc, cfg, layers, x):
    h = x
    kcs, vcs = [], []
    for L in layers:
        h, kc, vc = orc.decoder_layer(h, L["weights"], L["gain1"], L["gain2"], L["kcache"], L["vcache"], cfg["d"],
                                      cfg["n_q"], cfg["n_kv"], cfg["head_dim"], cfg["ffn"], cfg["cached"] + 1,
                                      cfg["eps"], cfg["theta"])
        kcs.append(kc.reshape(L["kcache"].shape))
        vcs.append(vc.reshape(L["vcache"].shape))
    return h, kcs, vcs


def check(outs, kcs, vcs, ref, cfg):
    want, kref, vref = ref
    for y in outs:
        assert np.all(np.isfinite(y))
        assert orc_err(y, want) < TOL
    pos = cfg["cached"]
    for kc, vc, kr, vr in zip(kcs, vcs, kref, vref):
        assert np.array_equal(kc[:pos], kr[:pos]) and np.array_equal(vc[:pos], vr[:pos])
        assert orc_err(kc[pos], kr[pos]) < TOL and orc_err(vc[pos], vr[pos]) < TOL


def orc_err(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(np.max(np.abs(a - b)) / max(1e-9, np.max(np.abs(b))))


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "unfused"])
def test_two_layer_decode_step(torch, ctx, orc, fused):
    cfg = wl.DECODER
    layers, x = wl.decoder_weights(cfg, seed=0)
    print(f"[gpu] decoder d={cfg['d']} layers={cfg['layers']} cached={cfg['cached']} fused={fused}", flush=True)
    outs, kcs, vcs = run_decoder(torch, ctx, cfg, layers, x, fused=fused)
    check(outs, kcs, vcs, oracle_decoder(orc, cfg, layers, x), cfg)


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "unfused"])
def test_decode_step_graph_replays(torch, ctx, orc, fused):
    # a captured step replayed several times (eager work in between) gives the
    # eager result every time; a small grouped-query config
    cfg = dict(wl.DECODER, d=512, n_q=8, n_kv=2, head_dim=64, ffn=1024, cached=9)
    layers, x = wl.decoder_weights(cfg, seed=3)
    print(f"[gpu] decoder graph d={cfg['d']} n_q={cfg['n_q']} n_kv={cfg['n_kv']} fused={fused}", flush=True)
    outs, kcs, vcs = run_decoder(torch, ctx, cfg, layers, x, graph=True, replays=3, fused=fused)
    ref = oracle_decoder(orc, cfg, layers, x)
    check(outs, kcs, vcs, ref, cfg)
    assert all(np.array_equal(outs[0], o) for o in outs[1:])
