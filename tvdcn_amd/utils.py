from types import FunctionType
from typing import Any, List, Tuple, Union

import torch

_NAMESPACE = "tvdcn_amd"


def _log_api_usage_once(obj: Any) -> None:
    """Record one API-usage event per call site through torch's (default no-op) logger.

    Same role as tvdcn/utils.py:11-32.
    """
    module = obj.__module__
    if not module.startswith(_NAMESPACE):
        module = f"{_NAMESPACE}.internal.{module}"
    name = obj.__name__ if isinstance(obj, FunctionType) else obj.__class__.__name__
    torch._C._log_api_usage_once(f"{module}.{name}")


# int-or-tuple arguments as the int lists the operator schemas take (``SymInt[N]``).
# Written for TorchScript as well: the parameters are annotated with explicit unions
# (torch.nn.common_types' ``_size_Nt`` aliases script as ``int[]`` without broadcasting
# an int default). In eager mode any sequence passes through and the operator checks
# its length, as it does for the reference's ``_single`` / ``_pair`` / ``_triple``.
def _ints1(v: Union[int, Tuple[int]]) -> List[int]:
    if isinstance(v, int):
        return [v]
    if torch.jit.is_scripting():
        return [v[0]]
    return [int(e) for e in v]


def _ints2(v: Union[int, Tuple[int, int]]) -> List[int]:
    if isinstance(v, int):
        return [v, v]
    if torch.jit.is_scripting():
        return [v[0], v[1]]
    return [int(e) for e in v]


def _ints3(v: Union[int, Tuple[int, int, int]]) -> List[int]:
    if isinstance(v, int):
        return [v, v, v]
    if torch.jit.is_scripting():
        return [v[0], v[1], v[2]]
    return [int(e) for e in v]
