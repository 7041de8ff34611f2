"""Synthetic GLM-shaped routed-expert layers resident in HBM (benchmark and test inputs).

Every routed expert is an EXL3 SwiGLU MLP: gate/up [H -> I], down [I -> H], K bits per weight in 16x16 tiles. Any bit
stream is a valid trellis tile, so tiles are splitmix64 bytes (generated on the device by gfl_synth_trellis); suh is
Rademacher +-1 and svh is +-U(0.5, 1.5)/sqrt(fan_in) rounded to fp16 (generated here, bit-identical to the CPU
checker's generator). Seeds: 0x6A11F1A5 ^ (layer << 20 | expert << 4 | proj), proj 0/1/2 = gate/up/down; the
scale stream uses seed ^ 0x5C41E50000000000.

One layer's trellis lives in one device arena (per expert: gate, up, down blobs, each 256-byte aligned) and its sign and
scale vectors in a second one; `ptr_table` lists the 9 device addresses per expert that gfl_register_layer takes.
"""
import numpy as np

import _native

SCALE_SALT = 0x5C41E50000000000
_M64 = 0xFFFFFFFFFFFFFFFF


def seed(layer, expert, proj):
    return 0x6A11F1A5 ^ ((layer << 20) | (expert << 4) | proj)


def splitmix64_at(seed_, idx):
    """Output idx (uint64 array) of the splitmix64 sequence seeded with seed_ (counter form)."""
    idx = np.asarray(idx, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed_ & _M64) + (idx + np.uint64(1)) * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def scales(seed_, k, n, fan_in):
    """suh [k], svh [n] as fp16 bit patterns (uint16)."""
    s2 = (seed_ ^ SCALE_SALT) & _M64
    r = splitmix64_at(s2, np.arange(k, dtype=np.uint64))
    suh = np.where((r & np.uint64(1)) != 0, np.uint16(0xBC00), np.uint16(0x3C00)).astype(np.uint16)
    r = splitmix64_at(s2, np.arange(k, k + n, dtype=np.uint64))
    u = (r >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    sign = np.where((r & np.uint64(1)) != 0, -1.0, 1.0)
    v = sign * (0.5 + u) * (1.0 / np.sqrt(np.float64(fan_in)))
    svh = v.astype(np.float32).astype(np.float16).view(np.uint16)
    return suh, svh


def trellis_bytes(k, n, K):
    return (k // 16) * (n // 16) * 32 * K


def _al(x):
    return (x + 255) // 256 * 256


class SynthLayer:
    """E synthetic experts of one layer: trellis in one HBM arena (per expert: gate, up, down, each 256-byte aligned),
    sign/scale vectors in a second, small arena."""

    def __init__(self, layer, E, H, I, Ks=(3, 3, 3), device=0):
        import torch
        self.layer, self.E, self.H, self.I, self.Ks = layer, E, H, I, tuple(Ks)
        self.dims = dims = [(H, I, Ks[0]), (H, I, Ks[1]), (I, H, Ks[2])]
        self.tbytes = [trellis_bytes(k, n, K) for k, n, K in dims]
        self.toffs, o = [], 0
        for tb in self.tbytes:
            self.toffs.append(o)
            o += _al(tb)
        self.trec = o
        self.soffs, o = [], 0
        for k, n, _ in dims:
            self.soffs.append(o); o += _al(2 * k)
            self.soffs.append(o); o += _al(2 * n)
        self.srec = o
        self.quant_bytes_per_expert = sum(self.tbytes) + 2 * sum(k + n for k, n, _ in dims)
        dev = f"cuda:{device}"
        self.arena = torch.empty(self.trec * E, dtype=torch.uint8, device=dev)
        host = np.zeros((E, self.srec), np.uint8)
        for e in range(E):
            for p, (k, n, _) in enumerate(dims):
                suh, svh = scales(seed(layer, e, p), k, n, k)
                host[e, self.soffs[2 * p]: self.soffs[2 * p] + 2 * k] = suh.view(np.uint8)
                host[e, self.soffs[2 * p + 1]: self.soffs[2 * p + 1] + 2 * n] = svh.view(np.uint8)
        self.sarena = torch.from_numpy(host.reshape(-1)).to(dev)
        for e in range(E):
            for p in range(3):
                base = e * self.trec + self.toffs[p]
                _native.synth_trellis(self.arena[base: base + self.tbytes[p]], seed(layer, e, p))
        torch.cuda.synchronize(device)

    def ptr(self, e, which):
        """which 0..2: trellis gate/up/down; 3..8: suh_g, svh_g, suh_u, svh_u, suh_d, svh_d"""
        if which < 3:
            return self.arena.data_ptr() + e * self.trec + self.toffs[which]
        return self.sarena.data_ptr() + e * self.srec + self.soffs[which - 3]

    @property
    def ptr_table(self):
        return [self.ptr(e, i) for e in range(self.E) for i in range(9)]

    def register(self, ctx, li):
        ctx.register_layer(li, self.E, self.H, self.I, self.Ks, self.ptr_table, keep=self)

    def matrix(self, e, p):
        """(trellis uint8, suh uint16, svh uint16) of expert e, proj p, copied to host numpy."""
        k, n, _ = self.dims[p]
        tb = self.arena[e * self.trec + self.toffs[p]: e * self.trec + self.toffs[p] + self.tbytes[p]]
        sc = self.sarena[e * self.srec: (e + 1) * self.srec].cpu().numpy()
        suh = sc[self.soffs[2 * p]: self.soffs[2 * p] + 2 * k].view(np.uint16).copy()
        svh = sc[self.soffs[2 * p + 1]: self.soffs[2 * p + 1] + 2 * n].view(np.uint16).copy()
        return tb.cpu().numpy().copy(), suh, svh


def route_uniform(M, E, topk, rng):
    """fp32 N(0,1) router logits -> sigmoid top-k, renormalised weights in fp16."""
    logits = rng.standard_normal((M, E)).astype(np.float32)
    return route(logits, topk), logits


def route(logits, topk):
    """Sigmoid scores s = 1 / (1 + e), e = exp(-x) correctly rounded to fp32, top-k (lower index on ties),
    w = s / sum(s) (summed in pick order) rounded to fp16. Returns (sel int64, w fp16)."""
    logits = np.asarray(logits, dtype=np.float32)
    ex = np.exp(-logits.astype(np.float64)).astype(np.float32)      # correctly rounded fp32 exp(-x)
    s = (np.float32(1.0) / (np.float32(1.0) + ex)).astype(np.float32)
    order = np.argsort(-s, axis=1, kind="stable")[:, :topk]
    picked = np.take_along_axis(s, order, axis=1).astype(np.float32)
    tot = np.zeros(picked.shape[0], np.float32)
    for j in range(topk):
        tot = (tot + picked[:, j]).astype(np.float32)
    w = (picked / tot[:, None]).astype(np.float32).astype(np.float16)
    return order.astype(np.int64), w


def zipf_logits(M, E, s, rng, perm_seed=7):
    """Zipf-skewed router logits: -s*ln(rank_e) + Gumbel(0,1) with rank a seeded permutation of 1..E."""
    rank = np.random.default_rng(perm_seed).permutation(E) + 1
    g = rng.gumbel(size=(M, E))
    return (-s * np.log(rank)[None, :] + g).astype(np.float32)
