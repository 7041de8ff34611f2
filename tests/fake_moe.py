"""Duck-typed stand-ins for exllamav3's BlockSparseMLP as the reference's expert_cache / cpu_tier read it
(num_experts, routing_first, routing_fn, multi_{gate,up,down}.ptrs_trellis and .linears[e].inner.{trellis,suh,svh})."""
import types

import torch


def _inner(trellis, suh, svh):
    return types.SimpleNamespace(inner=types.SimpleNamespace(trellis=trellis, suh=suh, svh=svh))


def module(key, E, H, I, mats, device, routing_fn=None):
    """mats[p][e] = (trellis uint8 tensor, suh fp16 tensor, svh fp16 tensor) for p in gate/up/down."""
    m = types.SimpleNamespace(key=key, num_experts=E, num_local_experts=E, routing_first=0, hidden_size=H,
                              intermediate_size=I, device=torch.device(device))
    for name, p in (("multi_gate", 0), ("multi_up", 1), ("multi_down", 2)):
        lins = [_inner(*mats[p][e]) for e in range(E)]
        ptrs = torch.tensor([l.inner.trellis.data_ptr() for l in lins], dtype=torch.int64, device=device)
        setattr(m, name, types.SimpleNamespace(linears=lins, ptrs_trellis=ptrs))
    m.routing_fn = routing_fn or (lambda bsz, cfg, z, params: (None, None))
    return m


def from_synth(L, key="model.layers.0.mlp"):
    """Module over a synth.SynthLayer's device arenas (views, no copies)."""
    import numpy as np
    mats = [[None] * L.E for _ in range(3)]
    for e in range(L.E):
        for p in range(3):
            k, n, _ = L.dims[p]
            b = e * L.trec + L.toffs[p]
            tr = L.arena[b: b + L.tbytes[p]]
            sb = e * L.srec
            suh = L.sarena[sb + L.soffs[2 * p]: sb + L.soffs[2 * p] + 2 * k].view(torch.float16)
            svh = L.sarena[sb + L.soffs[2 * p + 1]: sb + L.soffs[2 * p + 1] + 2 * n].view(torch.float16)
            mats[p][e] = (tr, suh, svh)
    return module(key, L.E, L.H, L.I, mats, L.arena.device)
