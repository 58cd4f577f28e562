"""ctypes binding of libdopt.so (the C ABI declared in include/dopt.h).

There is no fallback: if the library is missing, or a call fails, an exception is raised.
Bad ``bits`` raise ``ValueError`` (as act_triton_kernel.py:329-330 does); every other failure
raises ``RuntimeError`` carrying the library's dopt_last_error() message.
"""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libdopt.so")

F32, F16, BF16 = 0, 1, 2
ROUND_NEAREST, ROUND_STOCH_NOISE, ROUND_STOCH_PHILOX = 0, 1, 2
FLAG_CLAMP, FLAG_SQUASH = 1, 2
ACT_RELU, ACT_RELU6, ACT_GELU, ACT_SILU = 0, 1, 2, 3
BN_NORM, BN_QUANT, BN_RELU_QUANT, BN_RELU6_QUANT = 0, 1, 2, 3

OK, EBITS, EINVAL, EUNSUPPORTED, EHIP = 0, -1, -2, -3, -4

EXPORTS = (
    "dopt_abi_version",
    "dopt_last_error",
    "dopt_quant_pack",
    "dopt_dequant_unpack",
    "dopt_pack_codes",
    "dopt_unpack_codes",
    "dopt_fp8_gemm_nt",
    "dopt_fp8_pack_kmajor",
    "dopt_relu_pack",
    "dopt_relu_unpack",
    "dopt_act_forward",
    "dopt_pact_clamp_forward",
    "dopt_pact_clamp_backward",
    "dopt_act_quant_pack",
    "dopt_act_dequant_mul",
    "dopt_act_dequant_mul_alam",
    "dopt_bn_workspace_floats",
    "dopt_bn_reduce",
    "dopt_bn_norm_quant",
    "dopt_bn_train_forward",
    "dopt_bn_train_forward_noalloc",
    "dopt_bn_train_backward",
    "dopt_bn_bwd_reduce",
    "dopt_bn_bwd_dx",
    "dopt_bn_norm_quant_alam",
    "dopt_bn_bwd_reduce_alam",
    "dopt_bn_bwd_dx_alam",
    "dopt_dw_gemm_workspace_floats",
    "dopt_dw_gemm",
    "dopt_graph_node_counts",
    "dopt_graph_replace_memsets",
    "dopt_alam_quant_pack",
    "dopt_alam_dequant_unpack",
)

_lib = None


class DoptError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


def lib() -> ctypes.CDLL:
    """Load libdopt.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: the HIP kernels are not built. "
                "Run `python -m deep_optimization_amd.build` (or __graft_entry__.build())."
            )
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32, u64, f32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_uint64, ctypes.c_float
        L.dopt_abi_version.argtypes = []
        L.dopt_abi_version.restype = i32
        L.dopt_last_error.argtypes = []
        L.dopt_last_error.restype = ctypes.c_char_p
        L.dopt_quant_pack.argtypes = [vp, i32, i64, i32, i32, vp, i32, vp, u64, u64, i32, f32, vp, vp, vp, i32, vp]
        L.dopt_quant_pack.restype = i32
        L.dopt_dequant_unpack.argtypes = [vp, vp, vp, i32, i64, i32, i32, vp, vp, i32, vp]
        L.dopt_dequant_unpack.restype = i32
        L.dopt_pack_codes.argtypes = [vp, i64, i32, i32, vp, vp]
        L.dopt_pack_codes.restype = i32
        L.dopt_unpack_codes.argtypes = [vp, i64, i32, i32, vp, vp]
        L.dopt_unpack_codes.restype = i32
        L.dopt_fp8_gemm_nt.argtypes = [vp, vp, i64, i64, i64, i64, i64, f32, vp, i64, vp]
        L.dopt_fp8_gemm_nt.restype = i32
        L.dopt_fp8_pack_kmajor.argtypes = [vp, i64, i64, i64, i64, vp, i64, vp]
        L.dopt_fp8_pack_kmajor.restype = i32
        L.dopt_relu_pack.argtypes = [vp, i32, i64, i32, i32, vp, vp, vp]
        L.dopt_relu_pack.restype = i32
        L.dopt_relu_unpack.argtypes = [vp, vp, i32, i64, i32, vp, vp]
        L.dopt_relu_unpack.restype = i32
        L.dopt_act_forward.argtypes = [vp, i32, i64, i32, vp, vp, vp]
        L.dopt_act_forward.restype = i32
        L.dopt_pact_clamp_forward.argtypes = [vp, i32, i64, f32, vp, vp, vp]
        L.dopt_pact_clamp_forward.restype = i32
        L.dopt_pact_clamp_backward.argtypes = [vp, vp, i32, i64, vp, vp]
        L.dopt_pact_clamp_backward.restype = i32
        L.dopt_act_quant_pack.argtypes = [vp, i32, i32, i64, i32, i32, vp, vp, vp, vp, vp, i32, vp]
        L.dopt_act_quant_pack.restype = i32
        L.dopt_act_dequant_mul.argtypes = [vp, vp, vp, i32, i64, i32, i32, vp, vp, i32, vp, vp]
        L.dopt_act_dequant_mul.restype = i32
        L.dopt_act_dequant_mul_alam.argtypes = [vp, vp, vp, i32, i64, i32, i32, vp, vp, i32, u64, vp, vp]
        L.dopt_act_dequant_mul_alam.restype = i32
        L.dopt_bn_workspace_floats.argtypes = [i64, i64, i64]
        L.dopt_bn_workspace_floats.restype = i64
        L.dopt_bn_reduce.argtypes = [vp, i32, i64, i64, i64, i64, i64, vp, vp, vp, vp]
        L.dopt_bn_reduce.restype = i32
        L.dopt_bn_norm_quant.argtypes = [vp, i32, i64, i64, i64, i64, i64, vp, vp, vp, vp, i32, vp, vp, f32, i32, i32,
                                         i32, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        L.dopt_bn_norm_quant.restype = i32
        # x, dt, N, C, HW, stride_n, stride_c, workspace, weight, bias, eps, mode, group, bits,
        # y, x_hat, packed, relu_packed, scale, min, mean_out, var_out, running_mean, running_var, momentum, stream
        L.dopt_bn_train_forward.argtypes = [vp, i32, i64, i64, i64, i64, i64, vp, vp, vp, f32, i32, i32, i32,
                                            vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, f32, vp]
        L.dopt_bn_train_forward.restype = i32
        L.dopt_bn_train_forward_noalloc.argtypes = [vp, i32, i64, i64, i64, i64, i64, vp, vp, f32, i32, i32, i32,
                                                    vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, f32, vp]
        L.dopt_bn_train_forward_noalloc.restype = i32
        # mode, packed, relu_packed, scale, min, dy, dy_dt, N, C, HW, stride_n, stride_c, group, bits, workspace,
        # weight, var, eps, dweight, dbias, dx, stream
        L.dopt_bn_train_backward.argtypes = [i32, vp, vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, i32, i32, vp,
                                             vp, vp, f32, vp, vp, vp, vp]
        L.dopt_bn_train_backward.restype = i32
        L.dopt_bn_bwd_reduce.argtypes = [i32, vp, vp, vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, i32, i32, vp, vp, vp,
                                         vp]
        L.dopt_bn_bwd_reduce.restype = i32
        L.dopt_bn_bwd_dx.argtypes = [i32, vp, vp, vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, i32, i32, vp, vp, vp, vp,
                                     f32, i32, vp, vp]
        L.dopt_bn_bwd_dx.restype = i32
        # x, dt, N, C, HW, stride_n, stride_c, sum, sumsq, mean_in, invstd_in, sync, weight, bias, eps, group,
        # bits, alam_bits, y, packed, scale, min, mean_out, var_out, stream
        L.dopt_bn_norm_quant_alam.argtypes = [vp, i32, i64, i64, i64, i64, i64, vp, vp, vp, vp, i32, vp, vp, f32, i32,
                                              i32, i32, vp, vp, vp, vp, vp, vp, vp]
        L.dopt_bn_norm_quant_alam.restype = i32
        # packed, scale, min, dy, dy_dt, N, C, HW, stride_n, stride_c, group, bits, alam_bits, workspace, dweight,
        # dbias, stream
        L.dopt_bn_bwd_reduce_alam.argtypes = [vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, i32, i32, i32, vp, vp, vp,
                                              vp]
        L.dopt_bn_bwd_reduce_alam.restype = i32
        # packed, scale, min, dy, dy_dt, N, C, HW, stride_n, stride_c, group, bits, alam_bits, dweight, dbias,
        # weight, var, eps, var_is_invstd, dx, stream
        L.dopt_bn_bwd_dx_alam.argtypes = [vp, vp, vp, vp, i32, i64, i64, i64, i64, i64, i32, i32, i32, vp, vp, vp, vp,
                                          f32, i32, vp, vp]
        L.dopt_bn_bwd_dx_alam.restype = i32
        L.dopt_dw_gemm_workspace_floats.argtypes = [i64, i64, i64]
        L.dopt_dw_gemm_workspace_floats.restype = i64
        L.dopt_dw_gemm.argtypes = [vp, i64, vp, i64, vp, vp, vp, i32, i32, i64, i64, i64, vp, vp, vp, vp, vp]
        L.dopt_dw_gemm.restype = i32
        L.dopt_graph_node_counts.argtypes = [vp, vp, i32]
        L.dopt_graph_node_counts.restype = i32
        L.dopt_graph_replace_memsets.argtypes = [vp, vp]
        L.dopt_graph_replace_memsets.restype = i32
        L.dopt_alam_quant_pack.argtypes = [vp, i32, i64, i32, i32, i32, i32, ctypes.c_float, vp, vp, vp, vp]
        L.dopt_alam_quant_pack.restype = i32
        L.dopt_alam_dequant_unpack.argtypes = [vp, vp, vp, i64, i32, i32, i32, ctypes.c_uint64, vp, vp]
        L.dopt_alam_dequant_unpack.restype = i32
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc == OK:
        return
    msg = lib().dopt_last_error().decode(errors="replace")
    if rc == EBITS:
        raise ValueError(msg)
    raise DoptError(rc, f"{what} failed ({rc}): {msg}")
