"""Expert residency with every expert in HBM (the lookups of glm53/expert_cache.py:540-1046 of the reference).

The reference keeps a VRAM arena of expert slots in front of pinned host copies: `slotof[li, e] >= 0` means resident,
`home[li, e]` holds the host (UVA) addresses of the three trellis matrices, `step(li, sel, admit)` counts hits and
misses and admits misses over PCIe, `verify()` compares every owned slot with its home copy and the pointer tables
with slotof. One MI355X holds all 42 x 288 experts (~125 GB of 288 GB), so here every expert's home copy *is* its
slot: slotof[li, e] = li * E + e, home[li, e] = the device addresses of its trellis, the pointer tables the fused
kernels read equal home, and a step is all hits. The lookup surface (Pool, slotof, home, E, first, step, verify,
summary; attach_modules / find_moe / summary / verify at module level) keeps the reference's names so its callers
(cpu_tier.routed reads pool.slotof[li], pool.E, pool.first) run unchanged.

Modules are duck-typed like exllamav3's BlockSparseMLP as the reference reads them: num_local_experts or
num_experts, routing_first, routing_fn, and multi_gate / multi_up / multi_down each with ptrs_trellis (int64 [E]
device addresses) and linears[e].inner.{trellis, suh, svh}.
"""
import torch

POOLS = []


def _E(m):
    return int(getattr(m, "num_local_experts", None) or m.num_experts)


class Pool:
    def __init__(self, device, mods, reserve=0, max_slots=None, admit_max=64, stage_bytes=0, stage_min=8192):
        """reserve / max_slots / admit_max / stage_* are the reference's arena knobs; with full residency there is
        no arena to size, so they are recorded only."""
        self.device = torch.device(device)
        self.mods = list(mods)
        self.admit_max = admit_max
        m0 = self.mods[0]
        self.E = _E(m0)
        self.first = int(getattr(m0, "routing_first", 0) or 0)
        if not all(_E(m) == self.E and int(getattr(m, "routing_first", 0) or 0) == self.first for m in self.mods):
            raise ValueError("expert_cache: every MoE layer needs the same expert count and routing_first")
        L = len(self.mods)
        self.S = L * self.E
        i32 = dict(dtype=torch.int32, device=self.device)
        self.slotof = (torch.arange(L, **i32)[:, None] * self.E + torch.arange(self.E, **i32)[None, :]).contiguous()
        home, tabs = [], []
        for m in self.mods:
            pg, pu, pd = m.multi_gate.ptrs_trellis, m.multi_up.ptrs_trellis, m.multi_down.ptrs_trellis
            for t in (pg, pu, pd):
                if not (t.dtype == torch.long and t.is_contiguous() and t.device == self.device and t.numel() == self.E):
                    raise ValueError("expert_cache: ptrs_trellis must be contiguous int64 [E] on the pool's device")
            home.append(torch.stack([pg, pu, pd], dim=1))
            tabs.append([pg.data_ptr(), pu.data_ptr(), pd.data_ptr(), 0])
        self.home = torch.stack(home).contiguous()                 # [L, E, 3] device addresses
        self.tabs = torch.tensor(tabs, dtype=torch.int64, device=self.device)
        self.home_cpu = self.home.cpu()
        self.stats = torch.zeros(16, dtype=torch.int64, device=self.device)
        self.size_hist = {}
        self._sums = self._checksums()
        for li, m in enumerate(self.mods):
            m._ec = (self, li)

    def _checksums(self):
        """Per-layer, per-matrix wrapping int64 word sums of every expert's trellis (the bytes verify() re-reads)."""
        out = []
        for m in self.mods:
            row = []
            for mm in (m.multi_gate, m.multi_up, m.multi_down):
                row.append(torch.stack([_word_sum(l.inner.trellis) for l in mm.linears]))
            out.append(torch.stack(row))
        return torch.stack(out)                                     # [L, 3, E]

    def step(self, li, sel, admit):
        """ec_step: count the layer's picks; every local pick is a hit (stats[0]), ids of other layers' ranges and the
        -1 sentinel are ignored. No admission, no copies."""
        n = sel.numel()
        b = 1 << max(0, (n - 1).bit_length())
        self.size_hist[b] = self.size_hist.get(b, 0) + 1
        s = sel.reshape(-1).long() - self.first
        self.stats[0] += ((s >= 0) & (s < self.E)).sum()

    def warm(self, scores):
        """Nothing to warm: every expert is resident."""
        self.stats.zero_()

    def verify(self):
        """ec_verify: bad_slots = experts whose trellis bytes changed since attach, bad_tables = pointer-table entries
        that differ from home or slotof entries that are not the expert's own slot, owned = slots held."""
        if self.device.type == "cuda":
            torch.cuda.synchronize(self.device)
        bad_slots = int((self._checksums() != self._sums).sum())
        L = len(self.mods)
        want = torch.arange(L, device=self.device)[:, None] * self.E + torch.arange(self.E, device=self.device)[None, :]
        bad_tables = int((self.slotof.long() != want).sum())
        for li, m in enumerate(self.mods):
            cur = torch.stack([m.multi_gate.ptrs_trellis, m.multi_up.ptrs_trellis, m.multi_down.ptrs_trellis], dim=1)
            bad_tables += int((cur != self.home[li]).any(dim=1).sum())
        return {"device": str(self.device), "bad_slots": bad_slots, "bad_tables": bad_tables, "owned": self.S}

    def summary(self):
        s = self.stats.tolist()
        rec = sum(int(l.inner.trellis.numel() * l.inner.trellis.element_size())
                  for mm in (self.mods[0].multi_gate, self.mods[0].multi_up, self.mods[0].multi_down)
                  for l in mm.linears[:1])
        return {"device": str(self.device), "layers": len(self.mods), "slots": self.S, "slot_bytes": rec,
                "arena_gb": round(self.S * rec / 1e9, 2), "elastic": None,
                "mem_alloc_gb": round(torch.cuda.memory_allocated(self.device) / 1e9, 2)
                if self.device.type == "cuda" else 0.0,
                "hits": s[0], "misses": 0, "admitted": 0, "no_victim": 0, "evictions": 0,
                "hit_rate": 1.0 if s[0] else 0.0, "stage": None, "bg": None,
                "picks_hist": dict(sorted(self.size_hist.items())), "residency": "full"}


def _word_sum(t):
    flat = t.reshape(-1).view(torch.uint8)
    pad = (-flat.numel()) % 8
    if pad:
        flat = torch.cat([flat, torch.zeros(pad, dtype=torch.uint8, device=flat.device)])
    return flat.view(torch.int64).sum()


def find_moe(modules):
    """The MoE layers among `modules` (an iterable, or a callable returning one, like model.modules)."""
    it = modules() if callable(modules) else modules
    return [m for m in it if hasattr(m, "routing_fn") and hasattr(m, "multi_gate") and hasattr(m, "multi_down")]


def attach_modules(mods):
    """expert_cache.py:993-1031: one Pool per device; the router is wrapped so each routed call steps the pool."""
    by_dev = {}
    for m in mods:
        by_dev.setdefault(str(m.device), []).append(m)
    for dev, ms in by_dev.items():
        p = Pool(torch.device(dev), ms)
        POOLS.append(p)
        for m in ms:
            orig = m.routing_fn

            def routed(bsz, cfg, z, params, _orig=orig, _m=m):
                sel, w = _orig(bsz, cfg, z, params)
                pool, li = _m._ec
                if not params.get("autosplit_measure") and not params.get("tp_warmup"):
                    pool.step(li, sel, sel.numel() <= pool.admit_max)
                return sel, w
            m.routing_fn = routed
    return POOLS


def attach(model):
    return attach_modules(find_moe(model.modules))


def summary():
    return [p.summary() for p in POOLS]


def verify():
    return [p.verify() for p in POOLS]
