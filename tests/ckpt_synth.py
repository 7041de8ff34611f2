"""A small synthetic EXL3 checkpoint in the exllamav3 key layout, for the loader tests (not a reference file: random
trellis bits and the package's seeded sign/scale vectors, written with safetensors)."""
import numpy as np

PREFIX = "model"


def expert_tensors(layer, e, H, I, Ks, rng):
    """{suffix: array} of one expert (e = -1: the shared expert); trellis as int16 [k/16, n/16, 16K]."""
    import synth
    out = {}
    for p, (proj, (k, n)) in enumerate(zip(("gate", "up", "down"), ((H, I), (H, I), (I, H)))):
        K = Ks[p]
        tb = rng.integers(0, 2 ** 16, size=(k // 16, n // 16, 16 * K), dtype=np.uint16).view(np.int16)
        suh, svh = synth.scales(synth.seed(layer, e % 4096, p), k, n, k)
        out[f"{proj}_proj.trellis"] = tb
        out[f"{proj}_proj.suh"] = suh.view(np.float16)
        out[f"{proj}_proj.svh"] = svh.view(np.float16)
    return out


def write(tmpdir, layers, E, H, I, Ks_by_layer, shared=True, seed=5):
    """Write one shard per layer (model-0000L.safetensors) plus unrelated tensors; returns the shard paths."""
    from safetensors.numpy import save_file
    rng = np.random.default_rng(seed)
    paths = []
    for L in layers:
        d = {f"{PREFIX}.layers.{L}.self_attn.q_proj.weight": np.zeros((4, 4), np.float16)}
        for e in ([-1] if shared else []) + list(range(E)):
            for suf, a in expert_tensors(L, e, H, I, Ks_by_layer[L], rng).items():
                mid = "shared_experts" if e < 0 else f"experts.{e}"
                d[f"{PREFIX}.layers.{L}.mlp.{mid}.{suf}"] = np.ascontiguousarray(a)
        path = str(tmpdir / f"model-{L:05d}.safetensors")
        save_file(d, path)
        paths.append(path)
    return paths


def host_experts(paths, L, E, H, I, Ks, shared=False):
    """oracle Mats of layer L's experts (or its shared expert) read back from the files."""
    from oracle import Mat
    from safetensors.numpy import load_file
    t = {}
    for p in paths:
        t.update(load_file(p))
    out = []
    for e in ([-1] if shared else range(E)):
        mid = "shared_experts" if e < 0 else f"experts.{e}"
        mats = []
        for p, (proj, (k, n)) in enumerate(zip(("gate", "up", "down"), ((H, I), (H, I), (I, H)))):
            base = f"{PREFIX}.layers.{L}.mlp.{mid}.{proj}_proj"
            mats.append(Mat(t[base + ".trellis"].view(np.uint8).reshape(-1).copy(), t[base + ".suh"].view(np.uint16),
                            t[base + ".svh"].view(np.uint16), k, n, Ks[p]))
        out.append(tuple(mats))
    return out
