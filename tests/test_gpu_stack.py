"""Config 4, decode half: a stack of 42 resident 288-expert layers (H=5120, I=1536, 3 bpw; 107.5 GB of trellis in HBM
on one MI355X) registered in one context; the first and the last layer decode one token bit-exactly against the
oracle's EXACT layer (ft_core.h:1338-1407)."""
import numpy as np
import pytest


@pytest.mark.gpu
def test_42_layer_stack_first_and_last_bitexact(gpu, oracle):
    import torch
    import _native
    import synth
    from oracle import Mat
    H, I, E, NL = 5120, 1536, 288, 42
    free, total = torch.cuda.mem_get_info()
    if free < 120e9:
        pytest.skip(f"needs ~110 GB of free device memory, {free / 1e9:.0f} GB free")
    ctx = _native.Context(0)   # a context of its own, released with the 107 GB at the end
    layers = []
    for r in range(NL):
        L = synth.SynthLayer(400 + r, E, H, I, (3, 3, 3))
        L.register(ctx, 400 + r)
        layers.append(L)
    print(f"stack: {NL} layers, {NL * E * layers[0].quant_bytes_per_expert / 1e9:.1f} GB resident", flush=True)
    rng = np.random.default_rng(4000)
    for r in (0, NL - 1):
        L = layers[r]
        x16 = rng.standard_normal((1, H)).astype(np.float16)
        (sel, w16), _ = synth.route_uniform(1, E, 8, rng)
        xd = torch.from_numpy(x16.view(np.int16)).view(torch.float16).cuda()
        out = torch.empty((1, H), dtype=torch.float32, device="cuda")
        ctx.moe_forward(400 + r, xd, torch.from_numpy(sel).cuda(),
                        torch.from_numpy(w16.view(np.int16)).view(torch.float16).cuda(), out)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        ids = [int(e) for e in sel[0]]
        ex = []
        for e in ids:
            mats = []
            for p in range(3):
                tr, suh, svh = L.matrix(e, p)
                k, n = (H, I) if p < 2 else (I, H)
                mats.append(Mat(tr, suh, svh, k, n, 3))
            ex.append(tuple(mats))
        sub = np.arange(8, dtype=np.int64)[None, :]
        want = oracle.moe_forward(ex, x16.astype(np.float32), sub, w16.astype(np.float32), mode=1)
        nbad = int(np.count_nonzero(got != want))
        print(f"stack layer {r}: experts {ids}, mismatched {nbad}/{want.size}", flush=True)
        assert nbad == 0
    ctx.close()
    del ctx, layers, L
    torch.cuda.empty_cache()
