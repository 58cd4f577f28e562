"""The act_lib operators as PyTorch sees them: torch.library.opcheck (schema, fake kernel against
the real one, dispatch under functionalization / AOT), and a torch.compile trace (aot_eager, so no
code is generated) of a quantize -> dequantize round trip whose results equal eager's. The
reference registers its operators with triton_op for the same traceability
(Activation_Compression/act_triton_kernel.py:336, :372, :398, :419)."""
import pytest
import torch

import deep_optimization_amd  # noqa: F401

pytestmark = pytest.mark.gpu
DEV = "cuda"
ops = torch.ops.act_lib


def _x(shape, seed=0, dtype=torch.bfloat16):
    return torch.randn(shape, generator=torch.Generator(device=DEV).manual_seed(seed), device=DEV).to(dtype)


# opcheck's autograd-registration test expects an autograd formula; these operators are
# forward-only building blocks (the layers' autograd Functions call them), so it is left out
TESTS = ("test_schema", "test_faketensor", "test_aot_dispatch_static", "test_aot_dispatch_dynamic")


@pytest.mark.parametrize("case", [
    "quant_pack", "quant_pack_triton", "dequant_unpack", "dequant_unpack_triton", "quant_pack_triton_alam",
    "dequant_unpack_triton_alam", "quant_pack_tiles",
    "pack_triton", "unpack_triton", "fp8_gemm_nt", "fp8_linear", "relu_fwd_fused_pack", "dw_gemm"])
def test_opcheck(case):
    x = _x((2, 8, 256))
    if case == "quant_pack":
        args = (x, 2, 256, False, 0.0, False, 0, None, 0, 0, torch.float32)
    elif case == "quant_pack_triton":
        args = (x, 2, 256, False, 0, True, 3.0)
    elif case == "dequant_unpack":
        p, s, m = ops.quant_pack(x, 2, 256, False, 0.0, False, 0, None, 0, 0, torch.float32)
        args = (p, s, m, 2, 256, torch.bfloat16)
    elif case == "dequant_unpack_triton":
        p, s, m = ops.quant_pack_triton(x, 4, 256, False, 0, True, 3.0)
        args = (p, s, m, 4, 256, False, 0)
    elif case == "quant_pack_triton_alam":
        args = (x, 2, 256, True, 4, True, 3.0)
    elif case == "dequant_unpack_triton_alam":
        p, s, m = ops.quant_pack_triton(x, 4, 256, True, 2, True, 3.0)
        args = (p, s, m, 4, 256, True, 2)
    elif case == "quant_pack_tiles":
        args = (_x((2, 4, 32, 48)), 2, 256, False, 0.0, False, 0, None, 0, 0, torch.float32)
    elif case == "pack_triton":
        args = ((x > 0).to(torch.int8), 1, 256)
    elif case == "unpack_triton":
        args = (ops.pack_triton((x > 0).to(torch.int8), 1, 256), 1, 2, 8, 256)
    elif case == "fp8_gemm_nt":
        args = (_x((256, 128), 1).to(torch.float8_e4m3fn), _x((256, 128), 2).to(torch.float8_e4m3fn), 0.5)
    elif case == "fp8_linear":
        args = (_x((200, 100), 1).to(torch.float8_e4m3fn), _x((100, 72), 2).to(torch.float8_e4m3fn), 0.5)
    elif case == "relu_fwd_fused_pack":
        args = (_x((4, 8, 16, 16)), True, False, 1, 256)
    else:
        args = (_x((512, 256), 3), _x((512, 256), 4), None, None, None, 256, 0, 0, True, torch.float32)
    # test_schema mutates-and-compares its inputs with arithmetic torch lacks for fp8 tensors
    tests = TESTS[1:] if case.startswith("fp8") else TESTS
    name = case[:-len("_alam")] if case.endswith("_alam") else case  # the avg_alam cases of the same op
    torch.library.opcheck(getattr(ops, name).default, args, test_utils=tests)


def test_compile_round_trip_matches_eager():
    def round_trip(x):
        p, s, m = ops.quant_pack(x, 2, 256, False, 0.0, True, 0, None, 0, 0, torch.float32)
        return ops.dequant_unpack(p, s, m, 2, 256, torch.bfloat16) * 2 + 1

    x = _x((4, 16, 256), 5)
    eager = round_trip(x)
    compiled = torch.compile(round_trip, backend="aot_eager", fullgraph=True)(x)
    assert torch.equal(eager, compiled)
