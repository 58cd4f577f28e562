"""MI355X-native (gfx950) activation-compression hot path of Deep_Optimization.

Importing the package registers the ``torch.ops.act_lib`` operators (see ``act_lib``); the HIP
library ``libdopt.so`` is loaded on the first operator call and must have been built with
``python -m deep_optimization_amd.build``.
"""
from . import act_lib  # noqa: F401  (registers torch.ops.act_lib.*)
from . import bn_lib  # noqa: F401  (registers the BatchNorm act_lib operators)
from . import dw_lib  # noqa: F401  (registers act_lib::dw_gemm)
from .act_lib import _bits_consts  # noqa: F401

__all__ = ["act_lib", "bn_lib", "dw_lib"]
