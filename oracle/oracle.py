"""ctypes bindings over the CPU checker libraries -- TEST INFRASTRUCTURE ONLY.

`Oracle` wraps oracle/_build/libgfl_oracle.so (the C restatement of the reference path, oracle/gfl_oracle.c).
`RefEngine` wraps oracle/_ref/libftref.so, the reference's own AVX2 expert engine (kernels/cpu_avx2/ft_core.h)
compiled from the reference tree by oracle/Makefile. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg use this module; the product package never imports it.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libgfl_oracle.so")
REFLIB = os.path.join(HERE, "_ref", "libftref.so")
REFLIB_SERVER = os.path.join(HERE, "_ref", "libftref_server.so")   # the server's flags, default contraction

_P = C.c_void_p


def build(ref=True):
    """Compile the oracle (and the reference shim when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", HERE, "all" if ref else os.path.join(HERE, "_build", "libgfl_oracle.so")],
                   check=True)


def _ptr(a):
    return a.ctypes.data_as(_P) if a is not None else None


class Mat:
    """One quantized matrix: trellis bytes [k/16 * n/16 * 32K], suh fp16 bits [k], svh fp16 bits [n]."""

    def __init__(self, tr, suh, svh, k, n, K):
        self.tr = np.ascontiguousarray(tr, dtype=np.uint8)
        self.suh = np.ascontiguousarray(suh, dtype=np.uint16)
        self.svh = np.ascontiguousarray(svh, dtype=np.uint16)
        self.k, self.n, self.K = int(k), int(n), int(K)
        assert self.tr.size == (k // 16) * (n // 16) * 32 * K


class _CMat(C.Structure):
    _fields_ = [("tr", _P), ("suh", _P), ("svh", _P), ("k", C.c_int), ("n", C.c_int), ("K", C.c_int)]


class _CExpert(C.Structure):
    _fields_ = [("g", _CMat), ("u", _CMat), ("d", _CMat)]


def _cmat(m):
    return _CMat(_ptr(m.tr), _ptr(m.suh), _ptr(m.svh), m.k, m.n, m.K)


class Oracle:
    def __init__(self, path=LIB):
        if not os.path.exists(path):
            build(ref=False)
        L = self.L = C.CDLL(path)
        L.gflo_h2f.restype = C.c_float
        L.gflo_h2f.argtypes = [C.c_uint16]
        L.gflo_f2h.restype = C.c_uint16
        L.gflo_f2h.argtypes = [C.c_float]
        L.gflo_state.restype = C.c_uint16
        L.gflo_state.argtypes = [_P, C.c_int, C.c_int]
        L.gflo_perm.restype = C.c_int
        L.gflo_bytesum.restype = C.c_int
        L.gflo_bytesum.argtypes = [C.c_uint16]
        L.gflo_weight_bits.restype = C.c_uint16
        L.gflo_weight_bits.argtypes = [C.c_uint16]
        L.gflo_dequant.argtypes = [_P, C.c_int, C.c_int, C.c_int, _P]
        L.gflo_had128.argtypes = [_P]
        L.gflo_prep_block.argtypes = [_P, _P, _P]
        L.gflo_out_block.argtypes = [_P, _P]
        L.gflo_act_mul.restype = C.c_float
        L.gflo_act_mul.argtypes = [C.c_float, C.c_float, C.c_float]
        L.gflo_gemv.argtypes = [_P, C.c_int, C.c_int, C.c_int, _P, C.c_int, _P, C.c_int, _P]
        L.gflo_expert_forward.argtypes = [C.POINTER(_CExpert), _P, C.c_int, _P, C.c_int, C.c_float]
        L.gflo_expert_ref64.argtypes = [C.POINTER(_CExpert), _P, _P, C.c_float]
        L.gflo_moe_forward.restype = C.c_int
        L.gflo_moe_forward.argtypes = [C.POINTER(_CExpert), C.c_int, _P, C.c_int, _P, _P, C.c_int, _P, C.c_int,
                                       C.c_float]
        L.gflo_moe_forward_rows.restype = C.c_int
        L.gflo_moe_forward_rows.argtypes = [C.POINTER(_CExpert), C.c_int, _P, C.c_int, _P, _P, C.c_int, _P, _P,
                                            C.c_int, C.c_float]
        L.gflo_build_jobs.restype = C.c_int
        L.gflo_build_jobs.argtypes = [C.c_int, C.c_int, _P, _P, C.c_int, _P, _P, _P, _P]
        L.gflo_split.argtypes = [_P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P,
                                 _P, _P, C.c_int64, C.c_int, C.c_int, _P, _P, _P, _P, _P]
        L.gflo_combine.restype = C.c_int
        L.gflo_combine.argtypes = [_P, C.c_int, C.c_int, C.c_int64, _P, _P]
        L.gflo_grouped_rows.restype = C.c_int
        L.gflo_grouped_rows.argtypes = [_P, _P, C.c_int, C.c_int, _P, C.c_int, _P, _P, _P, _P, C.POINTER(C.c_int)]
        L.gflo_route.argtypes = [_P, C.c_int, C.c_int, C.c_int, _P, _P]
        L.gflo_splitmix64_at.restype = C.c_uint64
        L.gflo_splitmix64_at.argtypes = [C.c_uint64, C.c_uint64]
        L.gflo_seed.restype = C.c_uint64
        L.gflo_seed.argtypes = [C.c_int, C.c_int, C.c_int]
        L.gflo_synth_trellis.argtypes = [C.c_uint64, _P, C.c_size_t]
        L.gflo_synth_scales.argtypes = [C.c_uint64, _P, C.c_int, _P, C.c_int, C.c_int]

    # ---- fp16 / format ----
    def f2h(self, f):
        return self.L.gflo_f2h(float(f))

    def h2f(self, h):
        return self.L.gflo_h2f(int(h))

    def state(self, tile, K, t):
        tile = np.ascontiguousarray(tile, dtype=np.uint8)
        return self.L.gflo_state(_ptr(tile), K, t)

    def perm(self, i):
        return self.L.gflo_perm(i)

    def weight_bits(self, st):
        return self.L.gflo_weight_bits(int(st))

    def dequant(self, tr, k, n, K):
        """fp16 bits W[k][n]"""
        tr = np.ascontiguousarray(tr, dtype=np.uint8)
        W = np.empty((k, n), dtype=np.uint16)
        self.L.gflo_dequant(_ptr(tr), k, n, K, _ptr(W))
        return W

    # ---- transforms ----
    def had128(self, v):
        v = np.array(v, dtype=np.float32)
        self.L.gflo_had128(_ptr(v))
        return v

    def prep_block(self, x, suh):
        x = np.ascontiguousarray(x, dtype=np.float32)
        suh = np.ascontiguousarray(suh, dtype=np.uint16)
        xt = np.empty(128, dtype=np.float32)
        self.L.gflo_prep_block(_ptr(x), _ptr(suh), _ptr(xt))
        return xt

    def out_block(self, y, svh):
        y = np.array(y, dtype=np.float32)
        svh = np.ascontiguousarray(svh, dtype=np.uint16)
        self.L.gflo_out_block(_ptr(y), _ptr(svh))
        return y

    def gemv(self, m, xt, mode=1, sumx=None):
        xt = np.ascontiguousarray(xt, dtype=np.float32).reshape(-1, m.k)
        y = np.empty((xt.shape[0], m.n), dtype=np.float32)
        sx = None if sumx is None else np.ascontiguousarray(sumx, dtype=np.float32)
        self.L.gflo_gemv(_ptr(m.tr), m.k, m.n, m.K, _ptr(xt), xt.shape[0], _ptr(y), mode, _ptr(sx))
        return y

    # ---- experts ----
    def expert_forward(self, ex, x, mode=1, act_limit=0.0):
        g, u, d = ex
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, g.k)
        y = np.empty((x.shape[0], g.k), dtype=np.float32)
        ce = _CExpert(_cmat(g), _cmat(u), _cmat(d))
        self.L.gflo_expert_forward(C.byref(ce), _ptr(x), x.shape[0], _ptr(y), mode, act_limit)
        return y

    def expert_ref64(self, ex, x, act_limit=0.0):
        g, u, d = ex
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(g.k)
        y = np.empty(g.k, dtype=np.float32)
        ce = _CExpert(_cmat(g), _cmat(u), _cmat(d))
        self.L.gflo_expert_ref64(C.byref(ce), _ptr(x), _ptr(y), act_limit)
        return y

    def moe_forward(self, experts, x, sel, w, mode=1, act_limit=0.0):
        """experts: list of (g, u, d) Mats; x fp32 [T][H]; sel int [T][topk] (<0 skipped); w fp32 [T][topk]"""
        H = experts[0][0].k
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, H)
        sel = np.ascontiguousarray(sel, dtype=np.int32).reshape(x.shape[0], -1)
        w = np.ascontiguousarray(w, dtype=np.float32).reshape(sel.shape)
        arr = (_CExpert * len(experts))(*[_CExpert(_cmat(g), _cmat(u), _cmat(d)) for g, u, d in experts])
        out = np.empty_like(x)
        self.L.gflo_moe_forward(arr, len(experts), _ptr(x), x.shape[0], _ptr(sel), _ptr(w), sel.shape[1], _ptr(out),
                                mode, act_limit)
        return out

    def moe_forward_rows(self, experts, x, sel, w, rows, mode=1, act_limit=0.0):
        """moe_forward with the jobs of the whole batch (each token's combine order as in the full call) but only the
        given rows evaluated: returns fp32 [len(rows)][H]. experts: a list over all expert ids; entries of experts no
        wanted row picks are never read (any Mat tuple will do)."""
        H = experts[0][0].k
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, H)
        sel = np.ascontiguousarray(sel, dtype=np.int32).reshape(x.shape[0], -1)
        w = np.ascontiguousarray(w, dtype=np.float32).reshape(sel.shape)
        want = np.zeros(x.shape[0], np.uint8)
        want[list(rows)] = 1
        arr = (_CExpert * len(experts))(*[_CExpert(_cmat(g), _cmat(u), _cmat(d)) for g, u, d in experts])
        out = np.empty_like(x)
        self.L.gflo_moe_forward_rows(arr, len(experts), _ptr(x), x.shape[0], _ptr(sel), _ptr(w), sel.shape[1],
                                     _ptr(want), _ptr(out), mode, act_limit)
        return out[list(rows)]

    def build_jobs(self, E, sel, w):
        sel = np.ascontiguousarray(sel, dtype=np.int32)
        w = np.ascontiguousarray(w, dtype=np.float32).reshape(sel.shape)
        T, K = sel.shape
        cap = T * K + 1
        je = np.zeros(cap, np.int32); jm = np.zeros(cap, np.int32)
        jt = np.zeros(cap * 8, np.int32); jw = np.zeros(cap * 8, np.float32)
        nj = self.L.gflo_build_jobs(E, T, _ptr(sel), _ptr(w), K, _ptr(je), _ptr(jm), _ptr(jt), _ptr(jw))
        return [(int(je[j]), [(int(jt[j * 8 + i]), float(jw[j * 8 + i])) for i in range(jm[j])]) for j in range(nj)]

    # ---- split / combine / grouped rows / router ----
    def split(self, sel, w_bits, z_bits, E, first, slotof, score, pol, seq, li, keep_ids, rres=None, ctrl=None,
              stats=None):
        sel = np.ascontiguousarray(sel, dtype=np.int64).reshape(-1)
        w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16).reshape(-1)
        z_bits = np.ascontiguousarray(z_bits, dtype=np.uint16)
        bsz, H = z_bits.shape
        n = sel.size
        topk = n // bsz
        slotof = np.ascontiguousarray(slotof, dtype=np.int32)
        score = np.ascontiguousarray(score, dtype=np.float32)
        pol = np.ascontiguousarray(pol, dtype=np.float32)
        ctrl = np.zeros(16, np.int64) if ctrl is None else ctrl
        stats = np.zeros(8, np.int64) if stats is None else stats
        hx = np.zeros(bsz * H, np.uint16)
        hpicks = np.full(n * 3, -7, np.int32)
        sel_out = np.empty(n, np.int64)
        w_out = np.empty(n, np.uint16)
        dflag = np.zeros(1, np.int64)
        rr = None if rres is None else np.ascontiguousarray(rres, dtype=np.int32)
        self.L.gflo_split(_ptr(sel), _ptr(w_bits), _ptr(z_bits), n, bsz, topk, H, E, first, _ptr(slotof),
                          _ptr(score), _ptr(pol), _ptr(ctrl), _ptr(hx), _ptr(hpicks), seq, li, keep_ids,
                          _ptr(sel_out), _ptr(w_out), _ptr(dflag), _ptr(stats), _ptr(rr))
        npk = int(ctrl[4]) if dflag[0] != 0 else 0
        return dict(sel_out=sel_out, w_out=w_out, hpicks=hpicks[:3 * npk].reshape(-1, 3).copy(), ctrl=ctrl,
                    dflag=int(dflag[0]), stats=stats, hx=hx)

    def combine(self, out, dflag, ctrl, hout):
        is_half = out.dtype == np.uint16
        ctrl = np.ascontiguousarray(ctrl, dtype=np.int64)
        hout = np.ascontiguousarray(hout, dtype=np.float32)
        return self.L.gflo_combine(_ptr(out), int(is_half), out.size, int(dflag), _ptr(ctrl), _ptr(hout))

    def grouped_rows(self, sel, w, take, E):
        sel = np.ascontiguousarray(sel, dtype=np.int64)
        w = np.ascontiguousarray(w, dtype=np.float32).reshape(sel.shape)
        take = np.ascontiguousarray(take, dtype=np.uint8)
        T, K = sel.shape
        ex = np.zeros(E, np.int32); off = np.zeros(E + 1, np.int32)
        rt = np.zeros(T * K, np.int32); rw = np.zeros(T * K, np.float32)
        rows = C.c_int(0)
        nexp = self.L.gflo_grouped_rows(_ptr(sel), _ptr(w), T, K, _ptr(take), E, _ptr(ex), _ptr(off), _ptr(rt),
                                        _ptr(rw), C.byref(rows))
        if nexp < 0:
            raise ValueError("grouped rows rejected the routing")
        r = rows.value
        return ex[:nexp].copy(), off[:nexp + 1].copy(), rt[:r].copy(), rw[:r].copy()

    def route(self, logits, topk):
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        M, E = logits.shape
        sel = np.empty((M, topk), np.int64)
        w = np.empty((M, topk), np.uint16)
        self.L.gflo_route(_ptr(logits), M, E, topk, _ptr(sel), _ptr(w))
        return sel, w

    # ---- synthetic ----
    def seed(self, layer, expert, proj):
        return self.L.gflo_seed(layer, expert, proj)

    def synth_trellis(self, seed, nbytes):
        tr = np.empty(nbytes, np.uint8)
        self.L.gflo_synth_trellis(seed, _ptr(tr), nbytes)
        return tr

    def synth_scales(self, seed, k, n, fan_in):
        suh = np.empty(k, np.uint16); svh = np.empty(n, np.uint16)
        self.L.gflo_synth_scales(seed, _ptr(suh), k, _ptr(svh), n, fan_in)
        return suh, svh

    def synth_mat(self, layer, expert, proj, k, n, K):
        s = self.seed(layer, expert, proj)
        tr = self.synth_trellis(s, (k // 16) * (n // 16) * 32 * K)
        suh, svh = self.synth_scales(s, k, n, k)
        return Mat(tr, suh, svh, k, n, K)

    def synth_expert(self, layer, expert, H, I, Ks=(3, 3, 3)):
        return (self.synth_mat(layer, expert, 0, H, I, Ks[0]), self.synth_mat(layer, expert, 1, H, I, Ks[1]),
                self.synth_mat(layer, expert, 2, I, H, Ks[2]))


class RefEngine:
    """The reference's ft_core.h engine (K=3 only), for golden vectors and the CPU baseline."""

    def __init__(self, threads=1, cpus=None, path=REFLIB):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.L = C.CDLL(path)
        L.ref_init.restype = C.c_int
        L.ref_init.argtypes = [C.c_int, _P, C.c_int]
        L.ref_dense_weights.argtypes = [_P, C.c_int, C.c_int, _P]
        L.ref_state.restype = C.c_uint16
        L.ref_state.argtypes = [_P, C.c_int]
        L.ref_w_gpu.restype = C.c_float
        L.ref_w_gpu.argtypes = [C.c_uint16]
        L.ref_prep_block.argtypes = [_P, _P, _P]
        L.ref_out_block.argtypes = [_P, _P]
        L.ref_moe_forward.restype = C.c_int
        L.ref_moe_forward.argtypes = [C.c_int, C.c_int, C.c_int, _P, _P, _P, C.c_int, _P, _P, C.c_int, _P, C.c_int,
                                      C.c_float]
        L.ref_expert64.argtypes = [C.c_int, C.c_int, _P, _P, _P, _P]
        L.ref_time_decode.restype = C.c_int
        L.ref_time_decode.argtypes = [C.c_int, C.c_int, C.c_int, _P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int,
                                      C.c_int, _P]
        cpus = list(cpus) if cpus else [0]
        arr = np.array(cpus, np.int32)
        self.threads = L.ref_init(int(threads), _ptr(arr), len(cpus))
        self._keep = []

    @staticmethod
    def _tables(experts):
        trs = (C.c_void_p * (3 * len(experts)))()
        scs = (C.c_void_p * (6 * len(experts)))()
        for e, (g, u, d) in enumerate(experts):
            for j, m in enumerate((g, u, d)):
                assert m.K == 3, "the reference engine is K=3 only"
                trs[3 * e + j] = m.tr.ctypes.data
                scs[6 * e + 2 * j] = m.suh.ctypes.data
                scs[6 * e + 2 * j + 1] = m.svh.ctypes.data
        return trs, scs

    def dense_weights(self, m):
        W = np.empty((m.k, m.n), np.float32)
        self.L.ref_dense_weights(_ptr(m.tr), m.k, m.n, _ptr(W))
        return W

    def moe_forward(self, experts, x, sel, w, mode=1, act_limit=0.0):
        g0 = experts[0][0]
        H, I = g0.k, g0.n
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, H)
        sel = np.ascontiguousarray(sel, dtype=np.int32).reshape(x.shape[0], -1)
        w = np.ascontiguousarray(w, dtype=np.float32).reshape(sel.shape)
        out = np.empty_like(x)
        trs, scs = self._tables(experts)
        rc = self.L.ref_moe_forward(len(experts), H, I, trs, scs, _ptr(x), x.shape[0], _ptr(sel), _ptr(w),
                                    sel.shape[1], _ptr(out), mode, act_limit)
        assert rc == 0
        return out

    def expert64(self, ex, x):
        g = ex[0]
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(g.k)
        y = np.empty(g.k, np.float32)
        trs, scs = self._tables([ex])
        self.L.ref_expert64(g.k, g.n, trs, scs, _ptr(x), _ptr(y))
        return y

    def time_decode(self, experts, x, topk, iters, warmup, mode):
        """Per-call wall seconds of `iters` decode calls of x.shape[0] tokens (x fp32 [H] or [M][H]) x topk experts,
        expert sets cycling through the pool (ref_time_decode)."""
        g0 = experts[0][0]
        trs, scs = self._tables(experts)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, g0.k)
        secs = np.zeros(iters, np.float64)
        rc = self.L.ref_time_decode(len(experts), g0.k, g0.n, trs, scs, _ptr(x), x.shape[0], topk, iters, warmup,
                                    mode, _ptr(secs))
        assert rc == 0
        return secs
