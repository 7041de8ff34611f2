"""The routing hook of a MoE layer on the device: `routing_fn(bsz, cfg, z, params)` -> (sel, w), with the router's
scoring and top-k fused with ft_split in one launch (gfl_route_split), and the matching combine hook.

The reference wraps each MoE module's routing_fn and cpu_split_combine (glm53/cpu_tier.py:303-349): `routed` calls
the model's router, then ft_split on its picks, and returns the split's selection; `comb` runs ft_combine on the
layer output when a split is pending. Here the router projection (logits = z @ W_router^T, a plain library GEMM) runs
in torch, and the scoring, top-k and split run as one kernel; the selection it returns uses the reference's decode
sentinels (a pick served elsewhere becomes id -1 with weight 0, or keeps its id with weight 0 under keep_ids,
ft_tier_cu.cu:131-140), which the expert path skips. At full residency every pick stays on the device.

    hook = RoutingHook(W_router, E=288, topk=8, li=li, slotof=pool.slotof[li], pol=policy, ingress=ingress)
    module.routing_fn = hook.routing_fn
    module.cpu_split_combine = hook.wrap_combine(module.cpu_split_combine)
"""
import _native


class Ingress:
    """The split/combine pair's shared buffers (cpu_tier.S: ctrl, hx, picks, hout, dflag, stats, timeout), on the
    device: ctrl int64 [16], hx fp16 [max_bsz * H], picks int32 [max_bsz * topk * 3], hout fp32 [max_bsz * H]."""

    def __init__(self, H, max_bsz=4, topk=8, timeout_ns=2_000_000_000, device="cuda"):
        import torch
        self.ctrl = torch.zeros(16, dtype=torch.int64, device=device)
        self.hx = torch.zeros(max_bsz * H, dtype=torch.float16, device=device)
        self.picks = torch.zeros(max_bsz * topk * 3, dtype=torch.int32, device=device)
        self.hout = torch.zeros(max_bsz * H, dtype=torch.float32, device=device)
        self.dflag = torch.zeros(1, dtype=torch.int64, device=device)
        self.stats = torch.zeros(8, dtype=torch.int64, device=device)
        self.timeout_ns = int(timeout_ns)
        self.max_bsz = max_bsz
        self.seq = 0


class RoutingHook:
    """routing_fn + combine wrapper of one MoE layer (decode sizes: bsz <= ingress.max_bsz).

    W_router: fp32 [E, H] router weight on the device (logits = z @ W_router^T). slotof int32 [E] (the pool's
    residency row; >= 0 everywhere at full residency), score fp32 [E] (the CPU-preference scores, zeros by default),
    pol fp32 [20] (the split policy). first: the layer's first routed expert id."""

    def __init__(self, W_router, E, topk, li, slotof, pol, ingress, score=None, first=0, rres=None):
        import torch
        dev = W_router.device
        self.W = W_router.float().contiguous()
        self.E, self.topk, self.li, self.first = int(E), int(topk), int(li), int(first)
        self.slotof, self.pol, self.ing = slotof, pol, ingress
        self.score = score if score is not None else torch.zeros(self.E, dtype=torch.float32, device=dev)
        self.rres = rres if rres is not None else torch.empty(0, dtype=torch.int32, device=dev)
        n = ingress.max_bsz * self.topk
        self.sel = torch.empty(n, dtype=torch.int64, device=dev)       # the router's picks
        self.w = torch.empty(n, dtype=torch.float16, device=dev)
        self.sel_out = torch.empty(n, dtype=torch.int64, device=dev)   # the split's selection
        self.w_out = torch.empty(n, dtype=torch.float16, device=dev)
        self.pending = False

    def routing_fn(self, bsz, cfg, z, params):
        """(bsz, cfg, z, params) -> (sel int64 [bsz, topk], w fp16 [bsz, topk]): logits, then one launch for sigmoid
        top-k and the split. cfg / params are accepted as the model's routing_fn takes them."""
        import torch
        if bsz > self.ing.max_bsz:
            raise ValueError(f"routing hook: bsz {bsz} > {self.ing.max_bsz} (prefill goes through the grouped path)")
        zz = z.reshape(bsz, -1)
        if zz.dtype != torch.float16 or not zz.is_contiguous():
            zz = zz.half().contiguous()
        logits = (zz.float() @ self.W.t()).contiguous()
        n = bsz * self.topk
        self.ing.seq += 1
        sel, w = self.sel[:n].view(bsz, self.topk), self.w[:n].view(bsz, self.topk)
        so, wo = self.sel_out[:n], self.w_out[:n]
        _native.route_split(logits, self.topk, zz, self.E, self.first, self.slotof, self.score, self.pol,
                            self.ing.ctrl.data_ptr(), self.ing.hx.data_ptr(), self.ing.picks.data_ptr(), self.ing.seq,
                            self.li, int(bsz > 8), sel, w, so, wo, self.ing.dflag, self.ing.stats, self.rres)
        self.pending = True
        return so.view(bsz, self.topk), wo.view(bsz, self.topk)

    def combine(self, fhs):
        """ft_combine on the layer output when a split is pending (cpu_tier's comb); returns fhs (contiguous)."""
        if not self.pending:
            return fhs
        self.pending = False
        f = fhs if fhs.is_contiguous() else fhs.contiguous()
        _native.combine(f, self.ing.dflag, self.ing.ctrl.data_ptr(), self.ing.hout.data_ptr(), self.ing.stats,
                        self.ing.timeout_ns)
        return f

    def wrap_combine(self, orig):
        """The model's cpu_split_combine(fhs, cpu_partial, cpu_pending, shape), with the combine run first."""
        def comb(fhs, cpu_partial, cpu_pending, shape):
            return orig(self.combine(fhs), cpu_partial, cpu_pending, shape)
        return comb
