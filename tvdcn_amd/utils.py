from types import FunctionType
from typing import Any

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
