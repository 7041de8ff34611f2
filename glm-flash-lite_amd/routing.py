"""The routing hook of a MoE layer on the device: `routing_fn(bsz, cfg, z, params)` -> (sel, w) wrapping the model's
router the way cpu_tier.routed does (glm53/cpu_tier.py:303-335), and the matching combine hook (`comb`, :338-351).

The reference's `routed` calls the model's own routing_fn first. It returns that router's picks unchanged when the
tier is not the one to split them: a batch larger than maxbsz, a call flagged `autosplit_measure` or `tp_warmup`, or
more picks than its buffers hold (:315-317). Otherwise it runs ft_split on the picks and returns the split's
selection, in which a pick served elsewhere becomes id -1 with weight 0 (or keeps its id with weight 0 under
keep_ids, ft_tier_cu.cu:131-140); the expert path skips it. `comb` runs ft_combine on the layer output when a split
is pending.

RoutingHook does the same with this build's device kernels:

  * the router is the model's (`orig`, any routing_fn) or, given the router weight W_router instead, logits
    z @ W_router^T (a torch GEMM) scored by gfl_route (sigmoid, top-k, renormalised fp16 weights). In that second form
    a decode-sized call runs the router and the split as one launch (gfl_route_split);
  * a job the split publishes (picks of experts the slotof row marks as misses, or the empty handshake job of
    pol[7]) is served by the device worker (gfl_ingress_serve) when the hook is given a context holding the layer:
    computed on the stream right after the split and answered through ctrl[1], so the combine adds it without
    waiting. Without a context the job is left to a host worker on the same ingress buffers, as in the reference.

    hook = RoutingHook(E=288, topk=8, li=li, slotof=pool.slotof[li], pol=policy, ingress=ingress,
                       orig=module.routing_fn, ctx=ctx)
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
        self.max_picks = max_bsz * topk
        self.seq = 0


class RoutingHook:
    """routing_fn + combine wrapper of one MoE layer.

    Router: `orig` (the model's routing_fn(bsz, cfg, z, params) -> (sel int64 [bsz, topk], w fp16 [bsz, topk])) or
    W_router (fp32 [E, H] on the device; logits = z @ W_router^T). slotof int32 [E] (the pool's residency row; >= 0
    everywhere at full residency), score fp32 [E] (the CPU-preference scores, zeros by default), pol fp32 [20] (the
    split policy), first: the layer's first routed expert id. ctx: a _native.Context with layer li registered, to serve
    published jobs on the device (mode and act_limit as the tier's)."""

    def __init__(self, W_router=None, E=None, topk=8, li=0, slotof=None, pol=None, ingress=None, score=None, first=0,
                 rres=None, orig=None, ctx=None, mode=_native.MODE_AUTO, act_limit=0.0):
        import torch
        if (W_router is None) == (orig is None):
            raise ValueError("routing hook: give exactly one of W_router (the router weight) and orig (the model's "
                             "routing_fn)")
        if E is None or slotof is None or pol is None or ingress is None:
            raise ValueError("routing hook: E, slotof, pol and ingress are required")
        dev = slotof.device
        self.W = None if W_router is None else W_router.float().contiguous()
        self.orig = orig
        self.E, self.topk, self.li, self.first = int(E), int(topk), int(li), int(first)
        self.slotof, self.pol, self.ing = slotof, pol, ingress
        self.ctx, self.mode, self.act_limit = ctx, int(mode), float(act_limit)
        self.score = score if score is not None else torch.zeros(self.E, dtype=torch.float32, device=dev)
        self.rres = rres if rres is not None else torch.empty(0, dtype=torch.int32, device=dev)
        n = ingress.max_picks
        self.sel = torch.empty(n, dtype=torch.int64, device=dev)       # the router's picks (W_router form)
        self.w = torch.empty(n, dtype=torch.float16, device=dev)
        self.sel_out = torch.empty(n, dtype=torch.int64, device=dev)   # the split's selection
        self.w_out = torch.empty(n, dtype=torch.float16, device=dev)
        self.pending = False
        self.bypassed = 0

    def _bypass(self, bsz, params, npicks):
        """The cases in which cpu_tier.routed returns the router's picks unsplit (glm53/cpu_tier.py:315-317)."""
        p = params or {}
        return (bsz > self.ing.max_bsz or bool(p.get("autosplit_measure")) or bool(p.get("tp_warmup"))
                or npicks > self.ing.max_picks)

    def routing_fn(self, bsz, cfg, z, params):
        """(bsz, cfg, z, params) -> (sel int64 [bsz, topk], w fp16 [bsz, topk]): the router's picks, split when the
        call is decode-sized (see _bypass)."""
        import torch
        zz = z.reshape(bsz, -1)
        if zz.dtype != torch.float16 or not zz.is_contiguous():
            zz = zz.half().contiguous()
        self.pending = False
        if self.orig is not None:
            sel, w = self.orig(bsz, cfg, z, params)
            if self._bypass(bsz, params, sel.numel()):
                self.bypassed += 1
                return sel, w
            n = sel.numel()
            self.ing.seq += 1
            so, wo = self.sel_out[:n], self.w_out[:n]
            _native.split(sel.contiguous(), w.contiguous(), zz, self.E, self.first, self.slotof, self.score, self.pol,
                          self.ing.ctrl.data_ptr(), self.ing.hx.data_ptr(), self.ing.picks.data_ptr(), self.ing.seq,
                          self.li, int(bsz > 8), so, wo, self.ing.dflag, self.ing.stats, self.rres)
            shape_s, shape_w = sel.shape, w.shape
            topk = n // bsz
        else:
            logits = (zz.float() @ self.W.t()).contiguous()
            n = bsz * self.topk
            if self._bypass(bsz, params, n):
                self.bypassed += 1
                return _native.route(logits, self.topk)
            self.ing.seq += 1
            sel, w = self.sel[:n].view(bsz, self.topk), self.w[:n].view(bsz, self.topk)
            so, wo = self.sel_out[:n], self.w_out[:n]
            _native.route_split(logits, self.topk, zz, self.E, self.first, self.slotof, self.score, self.pol,
                                self.ing.ctrl.data_ptr(), self.ing.hx.data_ptr(), self.ing.picks.data_ptr(),
                                self.ing.seq, self.li, int(bsz > 8), sel, w, so, wo, self.ing.dflag, self.ing.stats,
                                self.rres)
            shape_s = shape_w = (bsz, self.topk)
            topk = self.topk
        if self.ctx is not None:
            self.ctx.ingress_serve(self.li, bsz, topk, self.ing.ctrl.data_ptr(), self.ing.hx.data_ptr(),
                                   self.ing.picks.data_ptr(), self.ing.hout.data_ptr(), self.mode, self.act_limit)
        self.pending = True
        return so.view(shape_s), wo.view(shape_w)

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
