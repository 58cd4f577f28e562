"""GPU parity of the weight-gradient GEMM act_lib::dw_gemm (dopt_dw_gemm): dW = dy^T . x_hat and
db = sum_k dy, x_hat read in bf16 or decoded from packed codes inside the kernel.

Bar:
  * dW and db against float64 products of the same bf16 operands: |err| <= 1e-4 of the sum of the
    terms' magnitudes (fp32 accumulation over up to 25k terms) plus 1e-6;
  * the packed path bit-exact equal to the bf16 path fed with act_lib::dequant_unpack_triton's
    x_hat (itself bit-exact against the CPU oracle): the in-kernel decode produces the same bf16
    values, and every kernel (the pipelined one for bf16 and for 1/2/4-bit codes, the
    register-decoding one for 8-bit codes) splits K at the same token boundaries and accumulates
    the same 16-token MFMA steps in the same order;
  * the bf16 output is the round-to-nearest-even of the fp32 output; repeated calls are bit-equal.
"""
import pytest
import torch

import deep_optimization_amd  # noqa: F401

pytestmark = pytest.mark.gpu
DEV = "cuda"
ops = torch.ops.act_lib


def operands(K, M, N, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    dy = torch.randn((K, M), generator=g, device=DEV).to(torch.bfloat16)
    x = (torch.randn((K, N), generator=g, device=DEV) * 2).to(torch.bfloat16)
    return dy, x


def check_close(got, dy, x):
    ref = dy.double().t() @ x.double()
    mag = dy.double().abs().t() @ x.double().abs()
    err = (got.double() - ref).abs()
    assert bool((err <= 1e-4 * mag + 1e-6).all()), float((err / (mag + 1e-30)).max())


@pytest.mark.parametrize("K,M,N", [(25216, 768, 768), (1000, 256, 512), (64, 512, 256), (4100, 1024, 256), (2048, 2304, 768)])
def test_bf16_operand(K, M, N):
    dy, x = operands(K, M, N, K + M)
    dw, db = ops.dw_gemm(dy, x, None, None, None, N, 0, 0, True, torch.float32)
    torch.cuda.synchronize()
    check_close(dw, dy, x)
    dbr = dy.double().sum(0)
    assert bool(((db.double() - dbr).abs() <= 1e-4 * dy.double().abs().sum(0) + 1e-6).all())
    dw16, none = ops.dw_gemm(dy, x, None, None, None, N, 0, 0, False, torch.bfloat16)
    assert none is None and torch.equal(dw16, dw.to(torch.bfloat16))
    dw2, db2 = ops.dw_gemm(dy, x, None, None, None, N, 0, 0, True, torch.float32)
    assert torch.equal(dw, dw2) and torch.equal(db, db2)


# the flat activation must split into whole groups (777 x 256 does not at g = 512)
PACKED_CASES = [(bits, g, K, M, N) for K, M, N in [(2048, 512, 768), (777, 256, 256), (25216, 768, 3072)]
                for bits, g in [(1, 64), (2, 256), (4, 128), (8, 512), (2, 512)] if (K * N) % g == 0]


@pytest.mark.parametrize("bits,g,K,M,N", PACKED_CASES)
def test_packed_operand_equals_dequantized(bits, g, K, M, N):
    dy, x = operands(K, M, N, 3 * bits + K)
    # the reference quantizer on the flat activation (one sample: groups of g consecutive elements)
    packed, scale, xmin = ops.quant_pack_triton(x.reshape(1, -1, g), bits, g, False, 0, True, 3.0)
    x_hat = ops.dequant_unpack_triton(packed, scale, xmin, bits, g, False, 0).reshape(K, N)
    want, wdb = ops.dw_gemm(dy, x_hat, None, None, None, N, 0, 0, True, torch.float32)
    got, gdb = ops.dw_gemm(dy, None, packed, scale, xmin, N, bits, g, True, torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    # db: both sum the same dy, in the two kernels' own orders
    assert bool(((gdb.double() - wdb.double()).abs() <= 1e-4 * dy.double().abs().sum(0) + 1e-6).all())
    check_close(got, dy, x_hat)


def test_no_tokens_and_errors():
    dy = torch.empty((0, 256), device=DEV, dtype=torch.bfloat16)
    x = torch.empty((0, 256), device=DEV, dtype=torch.bfloat16)
    dw, db = ops.dw_gemm(dy, x, None, None, None, 256, 0, 0, True, torch.float32)
    assert not dw.any() and not db.any()
    dy = torch.randn((64, 200), device=DEV).to(torch.bfloat16)
    x = torch.randn((64, 256), device=DEV).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="multiples of 256"):
        ops.dw_gemm(dy, x, None, None, None, 256, 0, 0, False, torch.float32)
    # packed operands: the per-group scale/min must cover every group (the kernel reads them unchecked)
    dy = torch.randn((64, 256), device=DEV).to(torch.bfloat16)
    x = torch.randn((1, 64 * 256 // 128, 128), device=DEV).to(torch.bfloat16)
    p, sc, mn = ops.quant_pack_triton(x, 2, 128, False, 0, True, 3.0)
    with pytest.raises(RuntimeError, match="one value per group"):
        ops.dw_gemm(dy, None, p, sc.reshape(-1)[:-2], mn, 256, 2, 128, False, torch.float32)
    with pytest.raises(RuntimeError, match="packed holds"):
        ops.dw_gemm(dy, None, p.reshape(-1)[:-1], sc, mn, 256, 2, 128, False, torch.float32)
