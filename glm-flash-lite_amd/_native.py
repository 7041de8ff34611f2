"""ctypes binding of libgfl_moe.so (the C ABI declared in include/gfl_moe.h).

The native library is the product: there is no Python or CPU fallback. If the shared object is missing or cannot be
loaded, every entry point raises NativeUnavailable (build it with `python glm-flash-lite_amd/build.py`).
Tensor arguments are torch tensors on the context's device; the current torch stream is used.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgfl_moe.so")

# exported symbols of include/gfl_moe.h (checked by tests/test_abi.py against the header)
SYMBOLS = ("gfl_last_error", "gfl_version", "gfl_ctx_create", "gfl_ctx_destroy", "gfl_register_layer",
           "gfl_moe_forward", "gfl_grouped_forward", "gfl_dequant", "gfl_split", "gfl_combine", "gfl_grouped_rows",
           "gfl_synth_trellis", "gfl_route",
           "gfl_stats", "gfl_profile_enable", "gfl_profile_read", "gfl_exp_table", "gfl_silu_table",
           "gfl_grouped_plan", "gfl_grouped_reserve", "gfl_layer_info", "gfl_route_split", "gfl_moe_forward_noalloc",
           "gfl_ctx_set_shared", "gfl_ctx_check", "gfl_ingress_serve", "gfl_register_shared",
           "gfl_moe_forward_shared")

EUNSUPPORTED = 4   # GFL_EUNSUPPORTED: gfl_moe_forward_shared cannot fuse this call (nothing was launched)

# layout limits of gfl_moe_forward_noalloc's static scratch array (GFL_NOALLOC_MAX_* in include/gfl_moe.h)
NOALLOC_MAX_PICKS, NOALLOC_MAX_H, NOALLOC_MAX_I = 64, 8192, 4096

MODE_AUTO, MODE_AFFINE, MODE_EXACT, MODE_I16, MODE_MFMA = -1, 0, 1, 2, 3


class NativeUnavailable(RuntimeError):
    pass


class NativeError(RuntimeError):
    pass


_LIB = None
_P = C.c_void_p


def load(path=LIB_PATH):
    """Load and type the library once; raise NativeUnavailable when it is absent."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise NativeUnavailable(f"{path} is missing: build it with `python glm-flash-lite_amd/build.py`")
    try:
        L = C.CDLL(path)
    except OSError as e:
        raise NativeUnavailable(f"cannot load {path}: {e}") from e
    L.gfl_last_error.restype = C.c_char_p
    L.gfl_version.restype = C.c_int
    L.gfl_ctx_create.argtypes = [C.c_int, C.POINTER(_P)]
    L.gfl_ctx_destroy.argtypes = [_P]
    L.gfl_register_layer.argtypes = [_P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _P]
    L.gfl_moe_forward.argtypes = [_P, C.c_int, _P, _P, _P, C.c_int, C.c_int, C.c_int, _P, C.c_int, C.c_float, _P]
    L.gfl_moe_forward_noalloc.argtypes = L.gfl_moe_forward.argtypes
    L.gfl_moe_forward_shared.argtypes = L.gfl_moe_forward.argtypes
    L.gfl_register_shared.argtypes = [_P, C.c_int, C.c_int, C.c_int, C.c_int, _P]
    L.gfl_grouped_forward.argtypes = [_P, C.c_int, _P, _P, _P, C.c_int, C.c_int, C.c_int, _P, C.c_float, _P]
    L.gfl_grouped_reserve.argtypes = [_P, C.c_int]
    L.gfl_layer_info.argtypes = [_P, C.c_int, _P]
    L.gfl_grouped_plan.argtypes = [_P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P, _P, _P, _P, _P]
    L.gfl_dequant.argtypes = [_P, C.c_int, C.c_int, C.c_int, _P, _P]
    L.gfl_split.argtypes = [_P, _P, _P, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P, _P, _P,
                            C.c_int64, C.c_int, C.c_int, _P, _P, _P, _P, _P, _P]
    L.gfl_route_split.argtypes = [_P, C.c_int, C.c_int, C.c_int, _P, _P, _P, C.c_int, C.c_int, C.c_int, _P, _P, _P,
                                  _P, _P, _P, C.c_int64, C.c_int, C.c_int, _P, _P, _P, _P, _P, _P]
    L.gfl_combine.argtypes = [_P, C.c_int, C.c_int, _P, _P, _P, _P, C.c_int64, _P]
    L.gfl_grouped_rows.argtypes = [_P, _P, C.c_int, C.c_int, _P, C.c_int, _P, _P, _P, _P, C.POINTER(C.c_int)]
    L.gfl_synth_trellis.argtypes = [_P, C.c_size_t, C.c_uint64, _P]
    L.gfl_route.argtypes = [_P, C.c_int, C.c_int, C.c_int, _P, _P, _P]
    L.gfl_stats.argtypes = [_P, _P, C.c_int]
    L.gfl_profile_enable.argtypes = [_P, C.c_int]
    L.gfl_ctx_set_shared.argtypes = [_P, C.c_int]
    L.gfl_ctx_check.argtypes = [_P]
    L.gfl_ingress_serve.argtypes = [_P, C.c_int, C.c_int, C.c_int, _P, _P, _P, _P, C.c_int, C.c_float, _P]
    L.gfl_profile_read.argtypes = [_P, _P, _P]
    L.gfl_exp_table.argtypes = [_P, C.c_int]
    L.gfl_silu_table.argtypes = [_P, C.c_int]
    for name in SYMBOLS:
        if name != "gfl_last_error":
            getattr(L, name).restype = C.c_int
    _LIB = L
    return L


def check(rc):
    if rc != 0:
        raise NativeError(load().gfl_last_error().decode() or f"gfl error {rc}")


def _stream():
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


class Context:
    """One gfl_ctx on a device (layer registry + workspace)."""

    def __init__(self, device=0):
        L = load()
        h = _P()
        check(L.gfl_ctx_create(int(device), C.byref(h)))
        self.h = h
        self.device = int(device)
        self._keep = {}
        self._shape = {}

    def close(self):
        if self.h:
            load().gfl_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def register_layer(self, li, E, H, I, ks, ptr_table, keep=None):
        """ptr_table: sequence of E*9 device addresses (see gfl_register_layer)."""
        arr = (C.c_uint64 * (9 * E))(*[int(p) for p in ptr_table])
        check(load().gfl_register_layer(self.h, li, E, H, I, int(ks[0]), int(ks[1]), int(ks[2]), arr))
        self._shape[li] = self.layer_info(li)
        if keep is not None:
            self._keep[li] = keep

    def register_shared(self, li, ks, ptr_row, keep=None):
        """The shared expert of registered layer li: ptr_row = its 9 device addresses (gfl_register_shared)."""
        arr = (C.c_uint64 * 9)(*[int(p) for p in ptr_row])
        check(load().gfl_register_shared(self.h, int(li), int(ks[0]), int(ks[1]), int(ks[2]), arr))
        if keep is not None:
            self._keep[("shared", li)] = keep

    def layer_info(self, li):
        """(E, H, I, k_gate, k_up, k_down) of a registered layer (gfl_layer_info)."""
        info = (C.c_int * 6)()
        check(load().gfl_layer_info(self.h, int(li), info))
        return tuple(info)

    def grouped_reserve(self, max_picks):
        """Size the grouped-path workspace for calls of up to max_picks picks (gfl_grouped_reserve)."""
        check(load().gfl_grouped_reserve(self.h, int(max_picks)))

    def _check_width(self, li, x):
        shape = self._shape.get(li)
        if shape is None:
            shape = self._shape[li] = self.layer_info(li)
        if x.shape[1] != shape[1]:
            raise ValueError(f"x is [M, {x.shape[1]}] but layer {li} has H = {shape[1]}")

    def moe_forward(self, li, x, sel, w, out, mode=MODE_EXACT, act_limit=0.0):
        """x fp16 [M,H], sel int64 [M,topk], w fp16|fp32 [M,topk], out fp32 [M,H] (all on the context device)."""
        return self._decode_forward(load().gfl_moe_forward, li, x, sel, w, out, mode, act_limit)

    def moe_forward_shared(self, li, x, sel, w, out, mode=MODE_EXACT, act_limit=0.0):
        """out = routed layer li + its shared expert in the routed call's own launches (gfl_moe_forward_shared).
        Returns False, with nothing launched, when the call cannot take that form (GFL_EUNSUPPORTED)."""
        return self._decode_forward(load().gfl_moe_forward_shared, li, x, sel, w, out, mode, act_limit,
                                    allow=(EUNSUPPORTED,)) is not None

    def moe_forward_noalloc(self, li, x, sel, w, out, mode=MODE_EXACT, act_limit=0.0):
        """moe_forward on the library's static scratch array: allocates nothing (M*topk <= NOALLOC_MAX_PICKS)."""
        return self._decode_forward(load().gfl_moe_forward_noalloc, li, x, sel, w, out, mode, act_limit)

    def _decode_forward(self, fn, li, x, sel, w, out, mode, act_limit, allow=()):
        import torch
        if sel.dim() != 2:
            raise ValueError("sel must be int64 [M, topk]")
        M, topk = sel.shape
        if not (x.dtype == torch.float16 and x.is_contiguous() and x.dim() == 2 and x.shape[0] == M):
            raise ValueError("x must be contiguous fp16 [M, H]")
        if not (sel.dtype == torch.int64 and sel.is_contiguous()):
            raise ValueError("sel must be contiguous int64 [M, topk]")
        if not (w.dtype in (torch.float16, torch.float32) and w.is_contiguous() and tuple(w.shape) == (M, topk)):
            raise ValueError("w must be contiguous fp16 or fp32 [M, topk]")
        if not (out.dtype == torch.float32 and out.is_contiguous() and tuple(out.shape) == tuple(x.shape)):
            raise ValueError("out must be contiguous fp32 [M, H]")
        for t in (x, sel, w, out):
            if not (t.is_cuda and t.device.index == self.device):
                raise ValueError(f"all tensors must be on cuda:{self.device}")
        self._check_width(li, x)
        rc = fn(self.h, li, ptr(x), ptr(sel), ptr(w), int(w.dtype == torch.float16), M, topk, ptr(out), int(mode),
                float(act_limit), _stream())
        if rc in allow:
            return None
        check(rc)
        return out

    def grouped_forward(self, li, x, sel, w, out, act_limit=0.0):
        """Prefill-sized forward (MFMA grouped GEMMs): same tensors as moe_forward, M*topk <= 65536."""
        import torch
        if sel.dim() != 2:
            raise ValueError("sel must be int64 [M, topk]")
        M, topk = sel.shape
        if not (x.dtype == torch.float16 and x.is_contiguous() and x.dim() == 2 and x.shape[0] == M):
            raise ValueError("x must be contiguous fp16 [M, H]")
        if not (sel.dtype == torch.int64 and sel.is_contiguous()):
            raise ValueError("sel must be contiguous int64 [M, topk]")
        if not (w.dtype in (torch.float16, torch.float32) and w.is_contiguous() and tuple(w.shape) == (M, topk)):
            raise ValueError("w must be contiguous fp16 or fp32 [M, topk]")
        if not (out.dtype == torch.float32 and out.is_contiguous() and tuple(out.shape) == tuple(x.shape)):
            raise ValueError("out must be contiguous fp32 [M, H]")
        for t in (x, sel, w, out):
            if not (t.is_cuda and t.device.index == self.device):
                raise ValueError(f"all tensors must be on cuda:{self.device}")
        self._check_width(li, x)
        check(load().gfl_grouped_forward(self.h, li, ptr(x), ptr(sel), ptr(w), int(w.dtype == torch.float16), M, topk,
                                         ptr(out), float(act_limit), _stream()))
        return out

    def grouped_plan(self, sel, w, E):
        """The device routing plan of grouped_forward alone, for sel int64 [M, topk] and w fp16/fp32 [M, topk] on this
        context's device: dict of tensors hdr [2], off [E+1], slot_pick / slot_e [M*topk], tok_slot / tok_w [M, topk],
        tok_npk [M] (layout of gfl_grouped_plan)."""
        import torch
        if not (sel.dim() == 2 and sel.dtype == torch.int64 and sel.is_contiguous()):
            raise ValueError("sel must be contiguous int64 [M, topk]")
        M, topk = sel.shape
        if not (w.dtype in (torch.float16, torch.float32) and w.is_contiguous() and tuple(w.shape) == (M, topk)):
            raise ValueError("w must be contiguous fp16 or fp32 [M, topk]")
        for t in (sel, w):
            if not (t.is_cuda and t.device.index == self.device):
                raise ValueError(f"all tensors must be on cuda:{self.device}")
        dev, i32 = sel.device, torch.int32
        r = dict(hdr=torch.zeros(2, dtype=i32, device=dev), off=torch.zeros(E + 1, dtype=i32, device=dev),
                 slot_pick=torch.full((M * topk,), -1, dtype=i32, device=dev),
                 slot_e=torch.full((M * topk,), -1, dtype=i32, device=dev),
                 tok_slot=torch.full((M, topk), -1, dtype=i32, device=dev),
                 tok_w=torch.zeros((M, topk), dtype=torch.float32, device=dev),
                 tok_npk=torch.zeros(M, dtype=i32, device=dev))
        check(load().gfl_grouped_plan(self.h, ptr(sel), ptr(w), int(w.dtype == torch.float16), M, topk, E,
                                      ptr(r["hdr"]), ptr(r["off"]), ptr(r["slot_pick"]), ptr(r["slot_e"]),
                                      ptr(r["tok_slot"]), ptr(r["tok_w"]), ptr(r["tok_npk"]), _stream()))
        return r

    STAGES = ("plan", "gate_up", "grouped", "down", "combine")

    def set_shared(self, shared):
        """Tell the context whether other GPU work runs beside its decode calls (gfl_ctx_set_shared): with shared set,
        calls of 769..1,536 gate|up tile columns keep the per-slot launches, which leave SIMDs free."""
        check(load().gfl_ctx_set_shared(self.h, int(bool(shared))))
        self._shared = bool(shared)

    @property
    def shared(self):
        """The flag set_shared last set on this context (False until then)."""
        return getattr(self, "_shared", False)

    def check(self):
        """Synchronise the device and raise NativeError when a device-side condition was counted since the last check
        (an expired relay hand-off wait, a published job the device worker refused): gfl_ctx_check."""
        check(load().gfl_ctx_check(self.h))

    def ingress_serve(self, li, bsz, topk, ctrl, hx, hpicks, hout, mode=MODE_AUTO, act_limit=0.0):
        """The device worker (gfl_ingress_serve): compute the job the split published to ctrl / hx / hpicks (integer
        addresses, as the split takes them) into hout and answer it, on the current stream."""
        check(load().gfl_ingress_serve(self.h, int(li), int(bsz), int(topk), C.c_void_p(int(ctrl)),
                                       C.c_void_p(int(hx)), C.c_void_p(int(hpicks)), C.c_void_p(int(hout)), int(mode),
                                       float(act_limit), _stream()))

    def profile(self, enable):
        check(load().gfl_profile_enable(self.h, int(bool(enable))))

    def profile_read(self):
        """{stage: (total device ms, launches)} since the last read (synchronises the recorded events)."""
        ms = (C.c_double * 5)()
        n = (C.c_int64 * 5)()
        check(load().gfl_profile_read(self.h, ms, n))
        return {s: (ms[i], n[i]) for i, s in enumerate(self.STAGES)}

    def stats(self):
        out = (C.c_int64 * 4)()
        check(load().gfl_stats(self.h, out, 4))
        return list(out)


def dequant(trellis, k, n, K, out):
    check(load().gfl_dequant(ptr(trellis), k, n, K, ptr(out), _stream()))
    return out


def synth_trellis(dst, seed, nbytes=None):
    nb = dst.numel() * dst.element_size() if nbytes is None else int(nbytes)
    check(load().gfl_synth_trellis(ptr(dst), nb, C.c_uint64(seed & 0xFFFFFFFFFFFFFFFF), _stream()))
    return dst


def route(logits, topk=8, sel=None, w=None):
    """Router (gfl_route): logits fp32 [M, E] on the device -> (sel int64 [M, topk], w fp16 [M, topk]), the routing_fn
    contract ft_split consumes. sel / w may be given (contiguous, on the device) to write in place."""
    import torch
    if not (logits.dtype == torch.float32 and logits.dim() == 2 and logits.is_contiguous() and logits.is_cuda):
        raise ValueError("logits must be contiguous fp32 [M, E] on the device")
    M, E = logits.shape
    if sel is None:
        sel = torch.empty((M, topk), dtype=torch.int64, device=logits.device)
    if w is None:
        w = torch.empty((M, topk), dtype=torch.float16, device=logits.device)
    if not (sel.dtype == torch.int64 and sel.is_contiguous() and tuple(sel.shape) == (M, topk)):
        raise ValueError("sel must be contiguous int64 [M, topk]")
    if not (w.dtype == torch.float16 and w.is_contiguous() and tuple(w.shape) == (M, topk)):
        raise ValueError("w must be contiguous fp16 [M, topk]")
    check(load().gfl_route(ptr(logits), M, E, int(topk), ptr(sel), ptr(w), _stream()))
    return sel, w


def split(sel, w, z, E, first, slotof, score, pol, ctrl, hx, hpicks, seq, li, keep_ids, sel_out, w_out, dflag,
          stats, rres):
    """ft_split with the reference's argument list (ctrl/hx/hpicks as integer addresses)."""
    bsz, H = z.shape
    n = sel.numel()
    check(load().gfl_split(ptr(sel), ptr(w), ptr(z), bsz, n, H, int(E), int(first), ptr(slotof), ptr(score),
                           ptr(pol), C.c_void_p(int(ctrl)), C.c_void_p(int(hx)), C.c_void_p(int(hpicks)), int(seq),
                           int(li), int(keep_ids), ptr(sel_out), ptr(w_out), ptr(dflag), ptr(stats),
                           ptr(rres) if rres is not None and rres.numel() else None, _stream()))


def route_split(logits, topk, z, E, first, slotof, score, pol, ctrl, hx, hpicks, seq, li, keep_ids, sel, w, sel_out,
                w_out, dflag, stats, rres):
    """Router and ft_split in one launch (gfl_route_split): logits fp32 [M, E_route] on the device; sel int64 and w fp16
    [M, topk] receive the routing, sel_out / w_out the split's selection; other arguments as split()."""
    M, ER = logits.shape
    H = z.shape[1]
    check(load().gfl_route_split(ptr(logits), M, ER, int(topk), ptr(sel), ptr(w), ptr(z), H, int(E), int(first),
                                 ptr(slotof), ptr(score), ptr(pol), C.c_void_p(int(ctrl)), C.c_void_p(int(hx)),
                                 C.c_void_p(int(hpicks)), int(seq), int(li), int(keep_ids), ptr(sel_out), ptr(w_out),
                                 ptr(dflag), ptr(stats), ptr(rres) if rres is not None and rres.numel() else None,
                                 _stream()))


def combine(out, dflag, ctrl, hout, stats, timeout_ns):
    """ft_combine with the reference's argument list (ctrl/hout as integer addresses)."""
    import torch
    check(load().gfl_combine(ptr(out), int(out.dtype == torch.float16), out.numel(), ptr(dflag),
                             C.c_void_p(int(ctrl)), C.c_void_p(int(hout)), ptr(stats), int(timeout_ns), _stream()))


def exp_table():
    """Host copy of the SwiGLU exponential table: expf(-g) for every fp16 bit pattern of g (float32 [65536])."""
    import numpy as np
    out = np.empty(65536, np.float32)
    check(load().gfl_exp_table(out.ctypes.data_as(C.c_void_p), out.size))
    return out


def silu_table():
    """Host copy of the SwiGLU gate table the device reads: g / (1 + expf(-g)) in fp32 for every fp16 bit pattern of g
    (float32 [65536])."""
    import numpy as np
    out = np.empty(65536, np.float32)
    check(load().gfl_silu_table(out.ctypes.data_as(C.c_void_p), out.size))
    return out


def grouped_rows(sel, w, take, E):
    """Host routine over numpy arrays (tier_lut_build_grouped_rows)."""
    import numpy as np
    sel = np.ascontiguousarray(sel, dtype=np.int64)
    T, K = sel.shape
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(T, K)
    take = np.ascontiguousarray(take, dtype=np.uint8)
    if take.size != E:
        raise ValueError("grouped take must be contiguous CPU uint8 [E]")
    ex = np.zeros(E, np.int32); off = np.zeros(E + 1, np.int32)
    rt = np.zeros(max(1, T * K), np.int32); rw = np.zeros(max(1, T * K), np.float32)
    rows = C.c_int(0)
    P = lambda a: a.ctypes.data_as(C.c_void_p)
    n = load().gfl_grouped_rows(P(sel), P(w), T, K, P(take), int(E), P(ex), P(off), P(rt), P(rw), C.byref(rows))
    if n < 0:
        raise ValueError(load().gfl_last_error().decode())
    r = rows.value
    return ex[:n].copy(), off[:n + 1].copy(), rt[:r].copy(), rw[:r].copy()
