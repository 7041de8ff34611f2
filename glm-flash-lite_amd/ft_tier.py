"""The CPU-tier extension surface of the reference, backed by the gfx950 library.

The reference builds kernels/cpu_avx2/ft_tier_ext.cpp + ft_tier_cu.cu into torch extensions and reaches them as
`cpu_tier._H` (tier_* calls) and `cpu_tier._CU` (ft_split / ft_combine) (glm53/cpu_tier.py:67-84). The same names,
argument lists and error behaviour (TORCH_CHECK -> RuntimeError) come from this build's own PyTorch-ROCm extension
(csrc/torch_ext.cpp, loaded through torch_ext.load()), re-exported here, so callers written against the reference's
extensions run unchanged:

  tier_init / tier_add_layer / tier_start / tier_stop / tier_forward / tier_stats / tier_set_act_limit / tier_set_e6 /
      tier_job_hist (ft_tier_ext.cpp:137-211, 629-666, 806-914)
  ft_split / ft_combine (ft_tier_cu.cu:238-294)
  tier_lut_build_grouped_rows (ft_tier_ext.cpp:1047-1097)

With every expert resident in HBM there is no host worker: tier_forward runs the experts on the GPU (EXACT
arithmetic, bit-identical to the reference's EXACT mode), and trellis pointers passed to tier_add_layer may be device
addresses of resident tiles or host addresses (the reference's pinned home copies, copied to the device once).
threads / cpus / swz are accepted and recorded, nothing more.
"""
import torch_ext

_EXT = torch_ext.load()

tier_init = _EXT.tier_init
tier_add_layer = _EXT.tier_add_layer
tier_start = _EXT.tier_start
tier_stop = _EXT.tier_stop
tier_forward = _EXT.tier_forward
tier_stats = _EXT.tier_stats
tier_set_act_limit = _EXT.tier_set_act_limit
tier_set_e6 = _EXT.tier_set_e6
tier_job_hist = _EXT.tier_job_hist
tier_lut_build_grouped_rows = _EXT.tier_lut_build_grouped_rows
ft_split = _EXT.ft_split
ft_combine = _EXT.ft_combine
tier_shutdown = _EXT.tier_shutdown   # release the singleton (the reference process never does; tests do)
tier_state = _EXT.tier_state         # (initialised, running, act_limit, layers registered)

__all__ = ["tier_init", "tier_add_layer", "tier_start", "tier_stop", "tier_forward", "tier_stats",
           "tier_set_act_limit", "tier_set_e6", "tier_job_hist", "ft_split", "ft_combine",
           "tier_lut_build_grouped_rows", "tier_shutdown", "tier_state", "install", "add_pool_layers"]


def install(cpu_tier):
    """Make a reference cpu_tier module use this library: `_H` (the tier_* extension) and `_CU` (split/combine)."""
    cpu_tier._H = _EXT
    cpu_tier._CU = _EXT
    return cpu_tier


def add_pool_layers(pool, bits=(3, 3, 3)):
    """Register every layer of a full-residency expert_cache.Pool, as cpu_tier.start does with tier_add_layer
    (glm53/cpu_tier.py:529-538): home pointers plus the suh/svh of each expert's three linears. bits: one
    (gate, up, down) triple for every layer, or a list with one triple per layer."""
    import torch
    per_layer = isinstance(bits[0], (tuple, list))
    for li, m in enumerate(pool.mods):
        sc = lambda lins, attr: torch.stack([getattr(l.inner, attr).reshape(-1) for l in lins]).half().contiguous()
        g, u, d = m.multi_gate.linears, m.multi_up.linears, m.multi_down.linears
        tier_add_layer(li, pool.home[li], sc(g, "suh"), sc(g, "svh"), sc(u, "suh"), sc(u, "svh"), sc(d, "suh"),
                       sc(d, "svh"), bits=bits[li] if per_layer else bits)
