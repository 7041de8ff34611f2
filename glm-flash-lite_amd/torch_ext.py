"""The PyTorch-ROCm extension _torch_ext/gfl_torch_ext.so (csrc/torch_ext.cpp, built in place by build.py): the
reference's torch-extension names (tier_*, ft_split, ft_combine) over libgfl_moe.so. Loading fails loudly when the
extension has not been built; there is no fallback."""
import importlib.util
import os

HERE = os.path.dirname(os.path.abspath(__file__))
PATH = os.path.join(HERE, "_torch_ext", "gfl_torch_ext.so")
_MOD = None


def load():
    global _MOD
    if _MOD is not None:
        return _MOD
    import torch  # noqa: F401  (the extension links torch's libraries; torch initialises HIP first)
    import _native
    _native.load()   # libgfl_moe.so: the extension's dependency, bound by soname to this loaded copy
    if not os.path.exists(PATH):
        raise _native.NativeUnavailable(f"{PATH} is missing: build it with `python glm-flash-lite_amd/build.py`")
    spec = importlib.util.spec_from_file_location("gfl_torch_ext", PATH)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    _MOD = mod
    return mod
