"""Swap the CPU tier's split/combine handle for the gfx950 kernels (glm53/k_ftsplit.py:37-54 of the reference).

The reference's install() replaces the module-level `cpu_tier._CU` with a namespace whose ft_split routes small
calls to its faster k110 kernel. Here one kernel serves every size the split accepts (<= 1024 picks), bit-identical
to the reference's float cost model evaluated uncontracted, so install() routes every call to it:

    import cpu_tier, k_ftsplit
    k_ftsplit.install(cpu_tier)          # after cpu_tier.start(), as serve.py does with GLM53_K_FTSPLIT=1
"""
import types

import ft_tier

STATS = {"fast": 0, "stock": 0}


def install(cpu_tier=None):
    """Point `cpu_tier._CU` at ft_split / ft_combine of this library; returns the previous handle."""
    if cpu_tier is None:
        import cpu_tier   # the reference's module, when it is on the path
    stock = getattr(cpu_tier, "_CU", None)

    def ft_split(sel, *a):
        STATS["fast"] += 1
        return ft_tier.ft_split(sel, *a)

    cpu_tier._CU = types.SimpleNamespace(ft_split=ft_split, ft_combine=ft_tier.ft_combine)
    print(" -- k_ftsplit (gfx950): CPU-tier ft_split / ft_combine -> gfl kernels", flush=True)
    return stock
