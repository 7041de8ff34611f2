"""EXL3 checkpoint -> HBM-resident expert arenas -> gfl_register_layer (full residency, no host tier).

The reference loads every routed expert's `.trellis` through exllamav3's SafetensorsCollection and, for the experts
it keeps off the GPU, copies them into exact-size pinned host arenas (glm53/exl3_tiers.py:99-160); expert_cache lays
a GPU slot out as gate | up | down trellis, each 256-byte aligned (rec = al(g) + al(u) + al(d),
glm53/expert_cache.py:550-555). On one MI355X all experts fit in HBM, so here every layer's experts go into one device
arena with that slot record, the suh/svh vectors into a second one, and the layer's [E][9] address table is
registered with a context.

Checkpoint keys (exllamav3 EXL3 linears): `<prefix>.layers.<L>.mlp.experts.<e>.<gate|up|down>_proj.<trellis|suh|svh>`
and, for the shared expert, `<prefix>.layers.<L>.mlp.shared_experts.<gate|up|down>_proj.<...>`. A linear [k -> n]
holds suh fp16 [k], svh fp16 [n] and its trellis as (k/16) * (n/16) tiles of 32*K bytes, row-major [k/16][n/16] (any
dtype/shape with that byte count); K follows from the byte count.

`self_test` repeats the reference's tier self-test (glm53/cpu_tier.py:738-770): fp64 truth from the effective weights
(this build's dequant, then the 128-wide Hadamards and suh/svh) against the device forward, as a relative RMS error.
"""
import math
import re
from dataclasses import dataclass, field

import numpy as np

_ROUTED = re.compile(r"^(?P<pre>.*?)\.layers\.(?P<layer>\d+)\.mlp\.experts\.(?P<e>\d+)\."
                     r"(?P<proj>gate|up|down)_proj\.(?P<kind>trellis|suh|svh)$")
_SHARED = re.compile(r"^(?P<pre>.*?)\.layers\.(?P<layer>\d+)\.mlp\.shared_experts\."
                     r"(?P<proj>gate|up|down)_proj\.(?P<kind>trellis|suh|svh)$")
PROJ = ("gate", "up", "down")
HAD = 1.0 / math.sqrt(128.0)


def _al(x, a):
    return (x + a - 1) // a * a


@dataclass
class LayerSpec:
    """Where layer L's expert tensors live: entries[(expert, proj, kind)] = (file, key, nbytes); expert -1 is the
    shared expert."""
    layer: int
    E: int = 0
    H: int = 0
    I: int = 0
    Ks: tuple = ()
    entries: dict = field(default_factory=dict)
    has_shared: bool = False

    @property
    def tile_bytes(self):
        """trellis bytes of gate, up, down"""
        return tuple((k // 16) * (n // 16) * 32 * K for (k, n), K in zip(self.dims, self.Ks))

    @property
    def dims(self):
        return ((self.H, self.I), (self.H, self.I), (self.I, self.H))

    @property
    def record(self):
        """expert slot record: (offset of up, offset of down, record bytes), each part 256-byte aligned"""
        sg, su, sd = self.tile_bytes
        off_u = _al(sg, 256)
        off_d = off_u + _al(su, 256)
        return off_u, off_d, off_d + _al(sd, 256)

    @property
    def scale_offsets(self):
        """fp16-element offsets of suh_g, svh_g, suh_u, svh_u, suh_d, svh_d inside one expert's scale record (each
        16-byte aligned) and the record length in elements"""
        lens = (self.H, self.I, self.H, self.I, self.I, self.H)
        offs, o = [], 0
        for n in lens:
            offs.append(o)
            o += _al(n, 8)
        return tuple(offs), o


def scan(paths):
    """Index the expert tensors of one or more .safetensors files -> {layer: LayerSpec}. Raises ValueError on a
    checkpoint this build cannot serve (missing tensors, sizes that are not EXL3 tiles, K outside 2..5, layers whose
    experts disagree in shape or bitrate)."""
    from safetensors import safe_open
    if isinstance(paths, str):
        paths = [paths]
    raw = {}
    for path in paths:
        with safe_open(path, framework="pt", device="cpu") as f:
            for key in f.keys():
                m = _ROUTED.match(key) or _SHARED.match(key)
                if not m:
                    continue
                L = int(m.group("layer"))
                e = int(m.group("e")) if "e" in m.groupdict() and m.group("e") is not None else -1
                sl = f.get_slice(key)
                shape = sl.get_shape()
                dt = sl.get_dtype()
                nbytes = int(np.prod(shape)) * _DT_BYTES[dt]
                raw.setdefault(L, {})[(e, m.group("proj"), m.group("kind"))] = (path, key, nbytes, dt, tuple(shape))
    specs = {}
    for L, ent in sorted(raw.items()):
        experts = sorted({e for (e, _, _) in ent if e >= 0})
        if not experts or experts != list(range(len(experts))):
            raise ValueError(f"layer {L}: routed experts must be numbered 0..E-1 (found {experts[:8]}...)")
        sp = LayerSpec(layer=L, E=len(experts), entries=ent, has_shared=any(e < 0 for (e, _, _) in ent))
        for who in ([-1] if sp.has_shared else []) + experts:
            for proj in PROJ:
                for kind in ("trellis", "suh", "svh"):
                    if (who, proj, kind) not in ent:
                        raise ValueError(f"layer {L}: expert {who} {proj}_proj.{kind} missing")
        # dims from expert 0's vectors: gate/up k = H, n = I
        def vec_len(e, proj, kind):
            _, _, nb, dt, shape = ent[(e, proj, kind)]
            if dt != "F16" or len(shape) != 1:
                raise ValueError(f"layer {L}: expert {e} {proj}_proj.{kind} must be a 1-d fp16 vector")
            return shape[0]
        sp.H, sp.I = vec_len(0, "gate", "suh"), vec_len(0, "gate", "svh")
        if sp.H % 256 or sp.I % 256:
            raise ValueError(f"layer {L}: hidden {sp.H} and intermediate {sp.I} must be multiples of 256")
        Ks = []
        for p, proj in enumerate(PROJ):
            k, n = sp.dims[p]
            tiles = (k // 16) * (n // 16)
            nb = ent[(0, proj, "trellis")][2]
            if nb % (tiles * 32) or not 2 <= nb // (tiles * 32) <= 5:
                raise ValueError(f"layer {L}: {proj}_proj.trellis has {nb} bytes, not {tiles} tiles of 32*K (K 2..5)")
            Ks.append(nb // (tiles * 32))
        sp.Ks = tuple(Ks)
        for who in ([-1] if sp.has_shared else []) + experts:
            for p, proj in enumerate(PROJ):
                k, n = sp.dims[p]
                if (vec_len(who, proj, "suh"), vec_len(who, proj, "svh")) != (k, n):
                    raise ValueError(f"layer {L}: expert {who} {proj}_proj vectors disagree with [{k} -> {n}]")
                if ent[(who, proj, "trellis")][2] != sp.tile_bytes[p]:
                    raise ValueError(f"layer {L}: expert {who} {proj}_proj.trellis size differs from expert 0's")
        specs[L] = sp
    return specs


_DT_BYTES = {"F16": 2, "BF16": 2, "F32": 4, "I16": 2, "U16": 2, "I32": 4, "U32": 4, "I8": 1, "U8": 1, "I64": 8,
             "U64": 8, "F64": 8}


class ResidentLayer:
    """One layer's experts in HBM: `arena` uint8 [E * record] (gate | up | down trellis per expert, 256-byte aligned)
    and `scales` fp16 [E * scale record]; `ptr_table` is gfl_register_layer's [E][9] address table. The shared
    expert, when the checkpoint has one, sits in a one-expert arena of its own (`shared`)."""

    def __init__(self, spec, device, experts):
        import torch
        self.spec = spec
        self.E = len(experts)
        self.off_u, self.off_d, self.rec = spec.record
        self.soffs, self.srec = spec.scale_offsets
        self.arena = torch.empty(self.E * self.rec, dtype=torch.uint8, device=device)
        self.scales = torch.zeros(self.E * self.srec, dtype=torch.float16, device=device)
        self.experts = experts
        self.shared = None

    def trellis_ptr(self, i, p):
        return self.arena.data_ptr() + i * self.rec + (0, self.off_u, self.off_d)[p]

    def scale_ptr(self, i, j):
        return self.scales.data_ptr() + 2 * (i * self.srec + self.soffs[j])

    @property
    def ptr_table(self):
        return [self.trellis_ptr(i, j) if j < 3 else self.scale_ptr(i, j - 3) for i in range(self.E) for j in range(9)]


def _copy_expert(res, i, who, spec, handles):
    import torch
    for p, proj in enumerate(PROJ):
        path, key, nb, _, _ = spec.entries[(who, proj, "trellis")]
        t = handles[path].get_tensor(key).contiguous().view(torch.uint8).reshape(-1)
        base = i * res.rec + (0, res.off_u, res.off_d)[p]
        res.arena[base: base + nb].copy_(t)
        for j, kind in enumerate(("suh", "svh")):
            path, key, _, _, _ = spec.entries[(who, proj, kind)]
            v = handles[path].get_tensor(key).contiguous().view(torch.float16)
            o = i * res.srec + res.soffs[2 * p + j]
            res.scales[o: o + v.numel()].copy_(v)


def load(paths, ctx, layers=None, device=0, shared=None):
    """Copy the routed experts of `layers` (default: all layers found) into HBM and register each as context layer
    index L. With `shared` (a k_overlap.SharedOverlap), shared experts are registered there under the same index,
    and with the routed layer in ctx too (gfl_register_shared), so that both can run in one call's launches.
    Returns {L: ResidentLayer}."""
    import torch
    from safetensors import safe_open
    if isinstance(paths, str):
        paths = [paths]
    specs = scan(paths)
    want = sorted(specs) if layers is None else list(layers)
    dev = torch.device("cuda", device)
    out = {}
    handles = {}
    try:
        for path in paths:
            handles[path] = safe_open(path, framework="pt", device="cpu").__enter__()
        for L in want:
            if L not in specs:
                raise ValueError(f"layer {L} not in the checkpoint")
            sp = specs[L]
            res = ResidentLayer(sp, dev, list(range(sp.E)))
            for e in range(sp.E):
                _copy_expert(res, e, e, sp, handles)
            ctx.register_layer(L, sp.E, sp.H, sp.I, sp.Ks, res.ptr_table, keep=res)
            if sp.has_shared:
                sh = ResidentLayer(sp, dev, [-1])
                _copy_expert(sh, 0, -1, sp, handles)
                res.shared = sh
                if shared is not None:
                    shared.register(L, sp.H, sp.I, sp.Ks, sh.ptr_table, keep=sh, routed=ctx)
            out[L] = res
    finally:
        for h in handles.values():
            h.__exit__(None, None, None)
    torch.cuda.synchronize(dev)
    return out


def _fwht_blocks(a):
    """128-wide Sylvester Hadamard along the last axis, per block, scaled by 1/sqrt(128) (float64)."""
    from scipy.linalg import hadamard
    Hm = hadamard(128).astype(np.float64) * HAD
    sh = a.shape
    return (a.reshape(-1, sh[-1] // 128, 128) @ Hm).reshape(sh)


def effective_weight(W16, suh, svh):
    """W_eff [k][n] (float64) of an EXL3 linear: x @ W_eff = ((x * suh) H) W H * svh with H the block Hadamard / sqrt(128)
    (prep_block / out_block of kernels/cpu_avx2/ft_core.h:96-110 without their fp16 rounding points)."""
    W = np.asarray(W16, dtype=np.float64)
    Wl = _fwht_blocks(W.T).T                    # H W   (H symmetric)
    Wr = _fwht_blocks(Wl)                       # (H W) H
    return suh.astype(np.float64)[:, None] * Wr * svh.astype(np.float64)[None, :]


def self_test(ctx, res, li, n_exp=4, mtok=(1, 3), seed=0):
    """The reference's tier self-test (glm53/cpu_tier.py:738-770) on one resident layer: x ~ 0.35 N(0,1) in fp16,
    n_exp random experts at weight 0.25, truth in float64 from the effective weights, SwiGLU output rounded to fp16;
    returns the largest relative RMS error of gfl_moe_forward (EXACT) over the token counts."""
    import torch
    import _native
    sp = res.spec
    g = np.random.default_rng(seed)
    errs = []
    weights = {}

    def weff(e, p):
        if (e, p) not in weights:
            k, n = sp.dims[p]
            W = torch.empty((k, n), dtype=torch.float16, device=res.arena.device)
            _native.check(_native.load().gfl_dequant(res.trellis_ptr(e, p), k, n, sp.Ks[p], _native.ptr(W),
                                                     _native._stream()))
            o = e * res.srec
            suh = res.scales[o + res.soffs[2 * p]: o + res.soffs[2 * p] + k].float().cpu().numpy()
            svh = res.scales[o + res.soffs[2 * p + 1]: o + res.soffs[2 * p + 1] + n].float().cpu().numpy()
            weights[(e, p)] = effective_weight(W.float().cpu().numpy(), suh, svh)
        return weights[(e, p)]

    for mt in mtok:
        x = (g.standard_normal((mt, sp.H)) * 0.35).astype(np.float16)
        exps = g.permutation(sp.E)[:n_exp].tolist()
        xd = x.astype(np.float64)
        ref = np.zeros((mt, sp.H), np.float64)
        for e in exps:
            gt, ut = xd @ weff(e, 0), xd @ weff(e, 1)
            a = ((gt / (1.0 + np.exp(-gt))) * ut).astype(np.float16).astype(np.float64)
            ref += 0.25 * (a @ weff(e, 2))
        xt = torch.from_numpy(x.view(np.int16)).view(torch.float16).to(res.arena.device)
        sel = torch.tensor([exps] * mt, dtype=torch.int64, device=res.arena.device)
        w = torch.full((mt, n_exp), 0.25, dtype=torch.float32, device=res.arena.device)
        out = torch.empty((mt, sp.H), dtype=torch.float32, device=res.arena.device)
        ctx.moe_forward(li, xt, sel, w, out)
        torch.cuda.synchronize()
        got = out.cpu().numpy().astype(np.float64)
        errs.append(float(np.linalg.norm(got - ref) / np.linalg.norm(ref)))
    return {"EXACT": round(max(errs), 6)}
