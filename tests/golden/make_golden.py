"""Write tests/golden/ref_vectors.npz from the reference's own AVX2 engine.

The engine is kernels/cpu_avx2/ft_core.h of the reference, compiled in this container by oracle/Makefile into
oracle/_ref/libftref.so (the reference tree is needed to build it; the GPU box only ever reads the .npz). Inputs are
regenerated from seeds by the checker's splitmix64 generator, so only seeds and reference outputs are stored:

  state_K3        state_scalar (ft_core.h:65-73) of all 256 stream indices of 4 seeded K=3 tiles
  dense_K3_*      dense_weights (ft_core.h:1657-1672) of seeded matrices, fp16 bit patterns
  prep / outb     prep_block / out_block (ft_core.h:97-110) of seeded vectors
  moe_*           moe_forward (ft_core.h:1338-1407) EXACT and AFFINE outputs: H=512 I=256 E=6 with the reference
                  harness routing ((t + 2k) % E, weight 0.25; kernel-ab-harness.cpp:115-116), ntok 1/3/4/16
                  (16 tokens put 10-11 tokens on each expert: two jobs per expert)
  expert_c0_*     config-0 expert (H=5120 I=1536 K=3) one token: EXACT moe_forward with weight 1, and ref_expert fp64

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

OUT = os.path.join(HERE, "ref_vectors.npz")


def main():
    import oracle as om
    om.build(ref=True)
    O = om.Oracle()
    R = om.RefEngine(threads=4, cpus=sorted(os.sched_getaffinity(0))[:4])
    out = {}
    # states
    st = []
    for s in range(4):
        tile = O.synth_trellis(1000 + s, 96)
        st.append([R.L.ref_state(tile.ctypes.data_as(om._P), t) for t in range(256)])
    out["state_K3_seeds"] = np.arange(1000, 1004)
    out["state_K3"] = np.array(st, np.uint16)
    # dense weights
    for name, (k, n, seed) in {"a": (64, 32, 2001), "b": (256, 128, 2002)}.items():
        m = O.synth_mat(0, 0, 0, k, n, 3)
        tr = O.synth_trellis(seed, (k // 16) * (n // 16) * 96)
        m = om.Mat(tr, m.suh, m.svh, k, n, 3)
        out[f"dense_K3_{name}"] = R.dense_weights(m).astype(np.float16).view(np.uint16)
        out[f"dense_K3_{name}_meta"] = np.array([k, n, seed])
    # transforms
    rng = np.random.default_rng(3001)
    xs = (rng.standard_normal((4, 128)) * 0.5).astype(np.float16).astype(np.float32)
    suh = np.where(rng.random((4, 128)) < 0.5, np.uint16(0xBC00), np.uint16(0x3C00)).astype(np.uint16)
    svh = (rng.uniform(0.5, 1.5, (4, 128)) * 0.03).astype(np.float16).view(np.uint16)
    prep, outb = [], []
    for i in range(4):
        xt = np.empty(128, np.float32)
        R.L.ref_prep_block(xs[i].ctypes.data_as(om._P), suh[i].ctypes.data_as(om._P), xt.ctypes.data_as(om._P))
        prep.append(xt)
        y = (xs[i] * 40.0).astype(np.float32)
        R.L.ref_out_block(y.ctypes.data_as(om._P), svh[i].ctypes.data_as(om._P))
        outb.append(y)
    out["tf_x"], out["tf_suh"], out["tf_svh"] = xs, suh, svh
    out["prep"], out["outb"] = np.array(prep), np.array(outb)
    # small MoE layer, harness routing
    H, I, E = 512, 256, 6
    ex = [O.synth_expert(7, e, H, I) for e in range(E)]
    for nt in (1, 3, 4, 16):
        r2 = np.random.default_rng(777 + nt)
        x = (r2.standard_normal((nt, H)) * 0.35).astype(np.float16).astype(np.float32)
        sel = np.array([[(t + 2 * k) % E for k in range(4)] for t in range(nt)], np.int32)
        w = np.full(sel.shape, 0.25, np.float32)
        out[f"moe_x_{nt}"], out[f"moe_sel_{nt}"] = x, sel
        out[f"moe_exact_{nt}"] = R.moe_forward(ex, x, sel, w, mode=1)
        out[f"moe_affine_{nt}"] = R.moe_forward(ex, x, sel, w, mode=0)
    # config-0 expert
    H, I = 5120, 1536
    e0 = O.synth_expert(8, 0, H, I)
    x = np.random.default_rng(4001).standard_normal((1, H)).astype(np.float16).astype(np.float32)
    out["c0_x"] = x
    out["expert_c0_exact"] = R.moe_forward([e0], x, np.zeros((1, 1), np.int32), np.ones((1, 1), np.float32), mode=1)
    out["expert_c0_ref64"] = R.expert64(e0, x[0])
    np.savez_compressed(OUT, **out)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
