"""Loader for the native operator library and the capability queries.

Mirrors tvdcn/extension.py (``has_ops``, ``with_cuda``, ``cuda_version``,
``cuda_arch_list``, ``_assert_has_ops``; tvdcn/extension.py:61-188). The library
is ``tvdcn_amd/_C.so``, built in-tree by ``tvdcn_amd/_build.py`` and found as the
reference finds its ``_C`` (tvdcn/extension.py:19-51): the import system's extension
finder over this directory, so ``_C`` + any extension suffix of the interpreter
(``.cpython-*.so``, ``.abi3.so``, ``.so``) is taken; it registers the
``torch.ops.tvdcn`` operators (the reference's namespace and schemas) and links
``libtvdcn_hip.so`` (the gfx950 HIP kernels behind the C ABI in
``include/tvdcn_hip.h``). There is no fallback: if the library is missing every op
raises.

``_has_ops`` is a function whose body is a constant, rebound once the library loads
(as tvdcn/extension.py:55-82 does), so that TorchScript can compile
``_assert_has_ops`` into scripted modules.
"""
import importlib.machinery
import os
from typing import List

import torch

_LIB_DIR = os.path.dirname(os.path.abspath(__file__))
HIP_LIB_PATH = os.path.join(_LIB_DIR, "libtvdcn_hip.so")


def _get_extension_path(lib_name: str) -> str:
    """Path of library ``lib_name`` in this package's directory under any of the interpreter's
    extension-module suffixes (the import system's own file finder); ImportError when absent."""
    finder = importlib.machinery.FileFinder(
        _LIB_DIR, (importlib.machinery.ExtensionFileLoader, importlib.machinery.EXTENSION_SUFFIXES))
    spec = finder.find_spec(lib_name)
    if spec is None or spec.origin is None:
        raise ImportError(f"no {lib_name} library in {_LIB_DIR}")
    return spec.origin

_HAS_OPS = False
_LOAD_ERROR = None


def _has_ops() -> bool:
    return False


def _has_ops_loaded() -> bool:
    return True


def _load() -> bool:
    """Loads ``_C.so`` once it exists; safe to call again (e.g. right after a build)."""
    global _HAS_OPS, _LOAD_ERROR, _has_ops
    if _HAS_OPS:
        return True
    try:
        torch.ops.load_library(_get_extension_path("_C"))
        _HAS_OPS = True
        _has_ops = _has_ops_loaded
        _LOAD_ERROR = None
    except (ImportError, OSError, RuntimeError) as e:  # pragma: no cover - reported by _assert_has_ops
        _LOAD_ERROR = str(e)
    return _HAS_OPS


_load()


def _assert_has_ops() -> None:
    if not _has_ops():
        raise RuntimeError(
            "Couldn't load the tvdcn native ops (tvdcn_amd/_C.so). Build them with:\n"
            "\tpython -m tvdcn_amd._build")


def has_ops() -> bool:
    """True when the native operator library is loaded."""
    return _HAS_OPS


def cuda_version() -> int:
    """HIP runtime version the kernels were built against (HIP_VERSION), -1 without ops.

    Named after the reference's ``cuda_version`` (on ROCm, torch's "cuda" device is HIP).
    """
    if not _HAS_OPS:
        return -1
    return torch.ops.tvdcn._cuda_version()


def with_cuda() -> bool:
    """True when the library carries GPU kernels (always, once loaded)."""
    return cuda_version() != -1


def cuda_arch_list() -> List[str]:
    """Offload targets the kernels were compiled for (``['gfx950']``)."""
    if not _HAS_OPS:
        return []
    return torch.ops.tvdcn._cuda_arch_flags().split()


def set_keep_channels_last_copy(enabled: bool) -> bool:
    """Opt-in memory-for-time trade of the float32 convolutions (no counterpart in the reference):
    when enabled, the forward keeps the channels-last copy of its input that the kernels sample, and
    the autograd node saves it instead of the input (the reference saves the input,
    autograd/deform_conv2d_kernel.cpp:35), so that the backward skips its own layout copy (about 1%
    of a forward + backward at BASELINE configs[1]). It holds one more |input| of device memory per
    layer until the backward runs, and an in-place change of the input after the forward goes
    undetected. Off by default. Returns the previous setting."""
    _assert_has_ops()
    return torch.ops.tvdcn._set_keep_input_copy(bool(enabled))

