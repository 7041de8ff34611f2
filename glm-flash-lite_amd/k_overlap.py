"""The shared expert on a side HIP stream, overlapped with the routed-expert path (glm53/k_overlap.py:1-16).

The reference takes the shared GatedMLP out of exllamav3's fused decode kernel and launches it on a side stream right
after routing, on the MoE input; it joins at the stock add `final_hidden_states += shared_experts.forward(x)`
(glm53/k_overlap.py:61-90). Here the shared expert is a one-expert layer of its own context (so its workspace never
races the routed call's), run through the same bit-exact expert path with weight 1.0 (o = 0 + 1.0 * y = y exactly),
on a side stream at the default priority. The routed layer call stays on the caller's stream; the join is one fp32
add, so the result equals routed + shared computed one after the other, bit for bit. All work is stream-ordered and
captures into HIP graphs (events are created once, up front).

Best of all, the shared expert rides on the routed call's own launches as one more pick per token
(gfl_moe_forward_shared), when the routed context holds it (register(..., routed=ctx)) and the call takes the relay
launches (up to 64 routed picks) with the same bit widths: config 1 M = 1 routed + shared 69.6 -> about 51 us per
token. Otherwise the two calls run as follows.

Whether the overlap pays depends on how the routed call fills the GPU (measured on MI355X, config 1 routed + one
config-0-shaped shared expert, us per token; gate|up tile columns = tokens x top-k x 2 x I / 16):
- up to 1,536 routed gate|up columns (M = 1 at top-8) the routed relay launches fill every SIMD with waves that yield
  to each other as they progress, and any overlapped form was slower than the stock order (69.6 sequential; 71.7
  with the routed call on narrower launches beside the shared expert, 73.1 with both on their own launches): such
  calls run in the stock order;
- up to 3,072 (M = 2) both run on their own launches, overlapped: 44.2 against 48.2 sequential (52.2 with the shared
  expert on narrow launches);
- above that the routed call fills every SIMD for longer, and the shared expert's context is told so
  (gfl_ctx_set_shared), so that its launches leave SIMDs free: 40.0 against 40.5 sequential at M = 4.
"""
import torch

import _native


class SharedOverlap:
    """Shared experts of a model (one per MoE layer) on a side stream of `device`."""

    def __init__(self, device=0):
        self.device = torch.device("cuda", device)
        self.ctx = _native.Context(device)
        self.side = torch.cuda.Stream(self.device)
        self.fork = torch.cuda.Event()
        self.join = torch.cuda.Event()
        self._sel = {}
        self._w = {}
        self._y = {}
        self._I = {}
        self.overlapped = 0
        self.sequential = 0
        self.fused = 0
        self._attached = set()   # (routed context, layer) pairs that hold the shared expert

    def register(self, li, H, I, ks, ptr_row, keep=None, routed=None):
        """Register layer li's shared expert: ptr_row = its 9 device addresses (trellis g/u/d, suh/svh g/u/d), as one
        row of gfl_register_layer's table; ks = (K gate, K up, K down). routed: the context that holds the routed
        layer li, registered already; it then also holds the shared expert, so that forward can run both in one
        call's launches (gfl_register_shared)."""
        self.ctx.register_layer(li, 1, H, I, ks, list(ptr_row), keep=keep)
        if routed is not None:
            routed.register_shared(li, ks, list(ptr_row), keep=keep)
            self._attached.add((id(routed), li))

    def _bufs(self, M, H):
        if M not in self._sel:
            self._sel[M] = torch.zeros((M, 1), dtype=torch.int64, device=self.device)
            self._w[M] = torch.ones((M, 1), dtype=torch.float32, device=self.device)
            self._y[M] = torch.empty((M, H), dtype=torch.float32, device=self.device)
        return self._sel[M], self._w[M], self._y[M]

    def forward(self, routed, li, x, sel, w, out, overlap=True):
        """out = routed layer li (context `routed`, picks sel / w) + shared expert of layer li, for x fp16 [M, H].
        With overlap, both run in the routed call's launches where that context holds the shared expert and the call
        allows it (gfl_moe_forward_shared), else on two streams, or in the stock order for a routed call of at most
        1,536 gate|up tile columns, where the overlap measured slower. overlap=False runs the shared expert after the
        routed call on the caller's stream (the reference's stock order), for comparison. Every order gives the same
        bits."""
        M, H = x.shape
        s1, w1, y = self._bufs(M, H)
        main = torch.cuda.current_stream(self.device)
        if overlap and (id(routed), li) in self._attached and routed.moe_forward_shared(li, x, sel, w, out):
            self.fused += 1
            return out
        cols = M * sel.shape[1] * 2 * (self._inter(routed, li) // 16)   # the routed call's gate|up tile columns
        if not overlap or cols <= 1536:
            routed.moe_forward(li, x, sel, w, out)
            self.ctx.set_shared(False)
            self.ctx.moe_forward(li, x, s1, w1, y)
            out.add_(y)
            self.sequential += 1
            return out
        self.fork.record(main)                   # MoE input ready
        self.side.wait_event(self.fork)
        # beside a routed call of more than 3,072 gate|up tile columns the shared expert takes narrower launches
        # that leave SIMDs free (M = 4: 40.0 against 40.5 us per token with its own launches); beside a smaller one its
        # own launches are faster (M = 2: 44.2 against 52.2)
        narrow = cols > 3072
        with torch.cuda.stream(self.side):
            self.ctx.set_shared(narrow)
            self.ctx.moe_forward(li, x, s1, w1, y)
            self.join.record(self.side)
        # the routed call is told that the side stream runs beside it (above 1,536 gate|up columns this changes no
        # launch shape, and results never change); the caller's own setting is restored afterwards
        prev = routed.shared
        routed.set_shared(True)
        try:
            routed.moe_forward(li, x, sel, w, out)
        finally:
            routed.set_shared(prev)
        main.wait_event(self.join)
        out.add_(y)
        self.overlapped += 1
        return out

    def _inter(self, routed, li):
        """The routed layer's intermediate size (gfl_layer_info), cached per layer."""
        if li not in self._I:
            self._I[li] = routed.layer_info(li)[2]
        return self._I[li]

    def summary(self):
        return {"overlapped": self.overlapped, "sequential": self.sequential, "fused": self.fused}
