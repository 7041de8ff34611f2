"""EXL3 checkpoint scan (exl3_loader.scan) on the CPU: key parsing, shapes and bitrates inferred from the tensors,
the expert slot record (expert_cache.py:550-555 rule), and refusals of checkpoints the device path cannot serve."""
import numpy as np
import pytest

import ckpt_synth


def test_scan_finds_layers_experts_and_bitrates(tmp_path):
    import exl3_loader
    paths = ckpt_synth.write(tmp_path, [0, 3], E=4, H=512, I=256, Ks_by_layer={0: (3, 3, 3), 3: (4, 4, 5)})
    specs = exl3_loader.scan(paths)
    assert sorted(specs) == [0, 3]
    s0, s3 = specs[0], specs[3]
    assert (s0.E, s0.H, s0.I, s0.Ks, s0.has_shared) == (4, 512, 256, (3, 3, 3), True)
    assert s3.Ks == (4, 4, 5)
    sg, su, sd = s3.tile_bytes
    assert (sg, su, sd) == (512 * 32 * 4, 512 * 32 * 4, 512 * 32 * 5)   # 512 tiles of 32*K bytes each
    off_u, off_d, rec = s3.record
    al = lambda x: (x + 255) // 256 * 256
    assert (off_u, off_d, rec) == (al(sg), al(sg) + al(su), al(sg) + al(su) + al(sd))
    offs, srec = s0.scale_offsets
    assert offs == (0, 512, 768, 1280, 1536, 1792) and srec == 2304


def test_scan_refuses_what_it_cannot_serve(tmp_path):
    import exl3_loader
    from safetensors.numpy import save_file, load_file
    paths = ckpt_synth.write(tmp_path, [1], E=3, H=512, I=256, Ks_by_layer={1: (3, 3, 3)}, shared=False)
    t = load_file(paths[0])
    bad = dict(t)
    del bad["model.layers.1.mlp.experts.2.up_proj.svh"]
    p1 = str(tmp_path / "missing.safetensors")
    save_file(bad, p1)
    with pytest.raises(ValueError, match="missing"):
        exl3_loader.scan([p1])
    bad = dict(t)
    bad["model.layers.1.mlp.experts.0.down_proj.trellis"] = np.zeros((16, 32, 16 * 6), np.int16)   # K = 6
    p2 = str(tmp_path / "k6.safetensors")
    save_file(bad, p2)
    with pytest.raises(ValueError, match="K 2..5"):
        exl3_loader.scan([p2])
    bad = {k.replace("experts.2.", "experts.5."): v for k, v in t.items()}
    p3 = str(tmp_path / "gap.safetensors")
    save_file(bad, p3)
    with pytest.raises(ValueError, match="numbered"):
        exl3_loader.scan([p3])


def test_effective_weight_matches_transforms():
    """x @ effective_weight == out_block(prep(x) @ W) without the fp16 rounding points (float64 transforms)."""
    import exl3_loader
    from scipy.linalg import hadamard
    rng = np.random.default_rng(3)
    k, n = 256, 384
    W = rng.standard_normal((k, n)).astype(np.float16)
    suh = rng.choice([-1.0, 1.0], k).astype(np.float16)
    svh = rng.random(n).astype(np.float16)
    x = rng.standard_normal((2, k))
    Hm = hadamard(128) / np.sqrt(128.0)
    Hk = np.kron(np.eye(k // 128), Hm)
    Hn = np.kron(np.eye(n // 128), Hm)
    want = (((x * suh.astype(np.float64)) @ Hk) @ W.astype(np.float64) @ Hn) * svh.astype(np.float64)
    got = x @ exl3_loader.effective_weight(W, suh, svh)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
