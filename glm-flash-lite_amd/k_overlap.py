"""The shared expert on a side HIP stream, overlapped with the routed-expert path (glm53/k_overlap.py:1-16).

The reference takes the shared GatedMLP out of exllamav3's fused decode kernel and launches it on a side stream right
after routing, on the MoE input; it joins at the stock add `final_hidden_states += shared_experts.forward(x)`
(glm53/k_overlap.py:61-90). Here the shared expert is a one-expert layer of its own context (so its workspace never
races the routed call's), run through the same bit-exact expert path with weight 1.0 (o = 0 + 1.0 * y = y exactly),
on a side stream at the default priority. The routed layer call stays on the caller's stream; the join is one fp32
add, so the result equals routed + shared computed one after the other, bit for bit. All work is stream-ordered and
captures into HIP graphs (events are created once, up front).

At decode sizes the routed launches leave compute units idle (1,536 gate|up column-waves on 1,024 SIMDs at M=1), which
is the room the shared expert's 48 + 40 workgroups run in. The routed context is told so for the overlapped call
(gfl_ctx_set_shared): on its own it runs such calls with launches that fill every SIMD. A larger routed call fills
every SIMD anyway; beside it the shared expert's own context is told so, and its launches leave SIMDs free instead.
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

    def register(self, li, H, I, ks, ptr_row, keep=None):
        """Register layer li's shared expert: ptr_row = its 9 device addresses (trellis g/u/d, suh/svh g/u/d), as one
        row of gfl_register_layer's table; ks = (K gate, K up, K down)."""
        self.ctx.register_layer(li, 1, H, I, ks, list(ptr_row), keep=keep)

    def _bufs(self, M, H):
        if M not in self._sel:
            self._sel[M] = torch.zeros((M, 1), dtype=torch.int64, device=self.device)
            self._w[M] = torch.ones((M, 1), dtype=torch.float32, device=self.device)
            self._y[M] = torch.empty((M, H), dtype=torch.float32, device=self.device)
        return self._sel[M], self._w[M], self._y[M]

    def forward(self, routed, li, x, sel, w, out, overlap=True):
        """out = routed layer li (context `routed`, picks sel / w) + shared expert of layer li, for x fp16 [M, H].
        overlap=False runs the shared expert after the routed call on the caller's stream (the reference's stock
        order), for comparison."""
        M, H = x.shape
        s1, w1, y = self._bufs(M, H)
        main = torch.cuda.current_stream(self.device)
        if not overlap:
            routed.moe_forward(li, x, sel, w, out)
            self.ctx.set_shared(False)
            self.ctx.moe_forward(li, x, s1, w1, y)
            out.add_(y)
            self.sequential += 1
            return out
        self.fork.record(main)                   # MoE input ready
        self.side.wait_event(self.fork)
        # beside a routed call of more than 1,536 gate|up tile columns (it fills every SIMD: 2 or more tokens at
        # top-8 and I = 1536) the shared expert takes narrower launches that leave SIMDs free (routed + shared at M = 4
        # 41.1 -> 38.8 us per token); beside a smaller routed call the default launches are faster (69.9 against 72.5
        # at M = 1)
        I = self._inter(routed, li)
        narrow = M * sel.shape[1] * 2 * (I // 16) > 1536
        with torch.cuda.stream(self.side):
            self.ctx.set_shared(narrow)
            self.ctx.moe_forward(li, x, s1, w1, y)
            self.join.record(self.side)
        # the routed call keeps launch shapes that leave SIMDs free for the side stream (same results); the caller's
        # own setting is restored afterwards
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
        return {"overlapped": self.overlapped, "sequential": self.sequential}
