"""The CPU-tier extension surface of the reference, backed by the gfx950 library.

The reference builds kernels/cpu_avx2/ft_tier_ext.cpp + ft_tier_cu.cu into one torch extension and reaches it as
`cpu_tier._H` (tier_* calls) and `cpu_tier._CU` (ft_split / ft_combine) (glm53/cpu_tier.py:67-84). This module
exports the same names, argument lists and error behaviour (a failed check raises RuntimeError, as TORCH_CHECK
does), so callers written against that extension run unchanged:

  tier_init / tier_add_layer / tier_start / tier_stop / tier_forward / tier_stats / tier_set_act_limit
      (ft_tier_ext.cpp:137-211, 814-914, 629-636)
  ft_split / ft_combine (ft_tier_cu.cu:238-294)
  tier_lut_build_grouped_rows (ft_tier_ext.cpp:1047-1097)

With every expert resident in HBM there is no host worker: tier_forward runs the experts on the GPU (gfl_moe_forward,
EXACT arithmetic, bit-identical to the reference's EXACT mode), and trellis pointers passed to tier_add_layer are
device addresses of the resident tiles. threads / cpus / swz are accepted and recorded, nothing more.
"""
import _native

__all__ = ["tier_init", "tier_add_layer", "tier_start", "tier_stop", "tier_forward", "tier_stats",
           "tier_set_act_limit", "ft_split", "ft_combine", "tier_lut_build_grouped_rows", "tier_shutdown"]


def _check(cond, msg):
    if not cond:
        raise RuntimeError(msg)


class _Tier:
    def __init__(self, ctx, mode, H, I, nlayers, keep, threads, cpus, swz):
        self.ctx, self.mode, self.H, self.I = ctx, mode, H, I
        self.layers = [None] * nlayers
        self.keep = list(keep)
        self.threads, self.cpus, self.swz = threads, list(cpus), swz
        self.running = False
        self.act_limit = 0.0
        self.jobs = self.experts = self.tokens = self.empty = 0


T = None                 # the singleton, like `Tier* T` (ft_tier_ext.cpp:122)
_ACT_LIMIT = [0.0]       # tier_set_act_limit may precede tier_init (ACT_LIMIT is a global in the reference)


def tier_init(threads, cpus, ctrl, hx, picks, hout, mode, H, I, nlayers, swz):
    """ft_tier_ext.cpp:137-157. ctrl/hx/picks/hout are the ingress buffers the split/combine pair shares with a host
    job (kept alive here); the expert computation itself has no host side."""
    global T
    import torch
    _check(T is None, "tier already initialised")
    _check(int(mode) in (-1, 0, 1, 2), "tier_init: mode must be -1, 0, 1 or 2")
    _check(H >= 256 and I >= 256 and H % 256 == 0 and I % 256 == 0, "tier_init: H and I must be multiples of 256")
    _check(torch.cuda.is_available(), "tier_init: no GPU (the expert path runs on the device)")
    ctx = _native.Context(torch.cuda.current_device())
    T = _Tier(ctx, int(mode), int(H), int(I), int(nlayers), (ctrl, hx, picks, hout), int(threads), cpus, int(swz))
    T.act_limit = _ACT_LIMIT[0]


def tier_shutdown():
    """Release the singleton (the reference process never does; tests and re-initialisation do)."""
    global T
    if T is not None:
        T.ctx.close()
        T = None


def tier_add_layer(li, ptrs, suh_g, svh_g, suh_u, svh_u, suh_d, svh_d, bits=(3, 3, 3)):
    """ft_tier_ext.cpp:160-211. ptrs int64 [E, 3]: device addresses of the gate/up/down trellis (native [k/16][n/16]
    tile layout); scales fp16 [E, .] on the CPU (copied to the device) or already on the device. `bits` extends the
    reference's fixed K=3 to the mixed-bitrate layers (2..5 per matrix)."""
    import torch
    _check(T is not None, "init first")
    _check(0 <= li < len(T.layers), "tier_add_layer: layer index out of range")
    _check(ptrs.dtype == torch.int64 and ptrs.dim() == 2 and ptrs.size(1) == 3, "ptrs: int64 [E, 3]")
    E, H, I = int(ptrs.size(0)), T.H, T.I
    dev = torch.device("cuda", T.ctx.device)
    sc = []
    for t in (suh_g, svh_g, suh_u, svh_u, suh_d, svh_d):
        _check(t.dtype == torch.float16 and t.is_contiguous() and t.dim() == 2 and t.size(0) == E,
               "scales: CPU fp16 contiguous [E, .]")
        sc.append(t.to(dev).contiguous())
    _check(suh_g.size(1) == H and svh_g.size(1) == I and suh_u.size(1) == H and svh_u.size(1) == I
           and suh_d.size(1) == I and svh_d.size(1) == H, "scale shapes")
    p = ptrs.cpu().tolist()
    table = []
    for e in range(E):
        table += [int(p[e][0]), int(p[e][1]), int(p[e][2])]
        table += [sc[k].data_ptr() + e * sc[k].size(1) * 2 for k in range(6)]
    try:
        T.ctx.register_layer(int(li), E, H, I, bits, table, keep=(ptrs, *sc))
    except _native.NativeError as err:
        raise RuntimeError(str(err)) from None
    T.layers[li] = E


def tier_start(cpu0):
    """ft_tier_ext.cpp:814-842: marks the tier running (no host worker thread exists)."""
    _check(T is not None, "init first")
    T.running = True


def tier_stop():
    """ft_tier_ext.cpp:844-862."""
    if T is not None:
        T.running = False


def tier_set_act_limit(limit):
    """ft_tier_ext.cpp:629-636: the SwiGLU clamp (exllamav3 semantics), 0 = off."""
    _ACT_LIMIT[0] = float(limit)
    if T is not None:
        T.act_limit = float(limit)


def tier_forward(li, x, sel, w, mode):
    """ft_tier_ext.cpp:865-904: x fp32 [m, H], sel int32 [m, k] (sel < 0 skipped), w fp32 [m, k] -> fp32 [m, H],
    sum over picks of w * expert(x) in the reference's job order. Tensors may live on the CPU (as the reference's)
    or on the device; the result is on x's device.

    Every mode number of the reference is accepted. Mode 1 (EXACT) is bit-identical to the reference's EXACT mode at
    every size up to 65536 picks. Modes -1 (auto), 0 (AFFINE) and 2 (I16) name the reference CPU engine's speed
    choices (ft_tier_ext.cpp:900): up to 1024 picks they compute EXACT too (it costs nothing more on the device and lies
    closer to the fp64 expert, ref_expert, ft_core.h:1674-1691, than AFFINE or I16 do); above 1024 picks they take the
    MFMA grouped path (the exact weights, rounding points and combine order, with the hidden-dimension sums formed in
    MFMA order: at the config-4 shape, M=2048, 3.6e-4 RMS and 2.9e-3 max-abs of the output RMS from EXACT)."""
    import torch
    _check(T is not None and not T.running, "tier_forward: worker running")
    _check(0 <= li < len(T.layers) and T.layers[li] is not None, "tier_forward: layer not registered")
    _check(int(mode) in (-1, 0, 1, 2), "tier_forward: mode must be -1, 0, 1 or 2")
    _check(x.dtype == torch.float32 and x.dim() == 2 and x.size(1) == T.H, "x: float32 [m, H]")
    _check(sel.dtype in (torch.int32, torch.int64) and sel.dim() == 2 and sel.size(0) == x.size(0), "sel: int32 [m, k]")
    _check(w.dtype == torch.float32 and tuple(w.shape) == tuple(sel.shape), "w: float32 [m, k]")
    m, k = sel.shape
    grouped = m * k > 1024 and int(mode) != 1
    _check(k <= 16 and m * k <= 65536, "tier_forward: k <= 16 and m * k <= 65536 picks")
    dev = torch.device("cuda", T.ctx.device)
    x16 = x.to(dev).half()
    _check(bool(torch.equal(x16.float(), x.to(dev))), "tier_forward: x must be fp16-valued (the expert input is fp16)")
    E = T.layers[li]
    _check(bool((sel < E).all()), "tier_forward: expert id out of range")
    seld = sel.to(dev).long()
    seld = torch.where(seld < 0, torch.full_like(seld, -1), seld).contiguous()
    out = torch.empty((m, T.H), dtype=torch.float32, device=dev)
    try:
        if grouped:
            T.ctx.grouped_forward(int(li), x16.contiguous(), seld, w.to(dev).contiguous(), out, act_limit=T.act_limit)
        else:
            T.ctx.moe_forward(int(li), x16.contiguous(), seld, w.to(dev).contiguous(), out,
                              mode=_native.MODE_EXACT, act_limit=T.act_limit)
    except _native.NativeError as err:
        raise RuntimeError(str(err)) from None
    valid = int((sel >= 0).sum())
    T.jobs += 1
    T.experts += valid
    T.tokens += m
    T.empty += int(valid == 0)
    return out if x.is_cuda else out.cpu()


def tier_stats():
    """ft_tier_ext.cpp:906-914: [jobs, experts, tokens, empty, busy_ns, swz_bytes, phase ns x5, prep ns]; the
    per-phase host wall times have no counterpart (device stage times come from the context's profiler)."""
    if T is None:
        return []
    return [T.jobs, T.experts, T.tokens, T.empty, 0, 0, 0, 0, 0, 0, 0, 0]


def ft_split(sel, w, z, E, first, slotof, score, pol, ctrl, hx, hpicks, seq, li, keep_ids, sel_out, w_out, dflag,
             stats, rres):
    """ft_tier_cu.cu:238-271 (and the fast kernel, ft_split_fast.cu:200-235): same arguments; ctrl / hx / hpicks
    are integer addresses the device can write (pinned host memory mapped into the GPU's address space, or device
    memory). Launches on the current stream."""
    import torch
    _check(pol.numel() >= 20, "ft_split: policy needs 20 entries")
    _check(rres.numel() == 0 or (rres.dtype == torch.int32 and rres.numel() >= E), "ft_split: rres int32 [E] or empty")
    _check(sel.dtype == torch.int64 and w.dtype == torch.float16 and z.dtype == torch.float16 and z.is_contiguous(),
           "dtypes")
    _check(z.dim() == 2, "ft_split: z [bsz, H]")
    bsz, H, n = int(z.size(0)), int(z.size(1)), int(sel.numel())
    _check(E <= 1024 and H % 8 == 0, "ft_split: E <= 1024")
    _check(n % bsz == 0 and n <= 1024, "ft_split: sel holds bsz * topk <= 1024 picks")
    for t in (sel, w, slotof, score, pol, sel_out, w_out, dflag, stats):
        _check(t.is_cuda and t.device == sel.device and t.is_contiguous(), "ft_split: buffers on one device, contiguous")
    _check(slotof.dtype == torch.int32 and slotof.numel() >= E and score.dtype == torch.float32 and score.numel() >= E
           and pol.dtype == torch.float32 and sel_out.dtype == torch.int64 and sel_out.numel() >= n
           and w_out.dtype == torch.float16 and w_out.numel() >= n and dflag.dtype == torch.int64
           and stats.dtype == torch.int64 and stats.numel() >= 8, "ft_split: buffer dtype/capacity mismatch")
    with torch.cuda.device(sel.device):
        try:
            _native.split(sel, w, z, E, first, slotof, score, pol, ctrl, hx, hpicks, seq, li, keep_ids, sel_out,
                          w_out, dflag, stats, rres)
        except _native.NativeError as err:
            raise RuntimeError(str(err)) from None


def ft_combine(out, dflag, ctrl, hout, stats, timeout_ns):
    """ft_tier_cu.cu:273-294: wait (at most timeout_ns) for ctrl[1] >= dflag, then out += hout (fp32 or fp16 out)."""
    import torch
    _check(out.dtype in (torch.float32, torch.float16) and out.is_contiguous(), "ft_combine: out fp32/fp16 contiguous")
    _check(dflag.dtype == torch.int64 and stats.dtype == torch.int64 and stats.numel() >= 8, "ft_combine: dtypes")
    with torch.cuda.device(out.device):
        try:
            _native.combine(out, dflag, ctrl, hout, stats, timeout_ns)
        except _native.NativeError as err:
            raise RuntimeError(str(err)) from None


def tier_lut_build_grouped_rows(sel, w, take, E):
    """ft_tier_ext.cpp:1047-1097 -> (experts int32, offsets int32 [n+1], row_token int32, row_weight float32), CPU."""
    import numpy as np
    import torch
    _check(1 <= E < 2 ** 31 - 1, "grouped E must fit a positive int32 expert count")
    _check(sel.device.type == "cpu" and sel.dtype == torch.int64 and sel.is_contiguous() and sel.dim() == 2,
           "grouped sel must be contiguous CPU int64 [T,K] with int32-sized rows")
    _check(w.device.type == "cpu" and w.dtype in (torch.float16, torch.float32) and w.is_contiguous()
           and tuple(w.shape) == tuple(sel.shape), "grouped weights must match sel as contiguous CPU fp16 or float32")
    _check(take.device.type == "cpu" and take.dtype == torch.uint8 and take.is_contiguous() and take.dim() == 1
           and take.numel() == E, "grouped take must be contiguous CPU uint8 [E]")
    try:
        ex, off, rt, rw = _native.grouped_rows(sel.numpy(), w.float().numpy(), take.numpy(), int(E))
    except ValueError as err:
        raise RuntimeError(str(err)) from None
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(dt)
    return t(ex, torch.int32), t(off, torch.int32), t(rt, torch.int32), t(rw, torch.float32)


def install(cpu_tier):
    """Make a reference cpu_tier module use this library: `_H` (the tier_* extension) and `_CU` (split/combine)."""
    import sys
    import types
    cpu_tier._H = sys.modules[__name__]
    cpu_tier._CU = types.SimpleNamespace(ft_split=ft_split, ft_combine=ft_combine)
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
