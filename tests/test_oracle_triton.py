"""The oracle's Triton random streams against Triton itself.

The ALAM dequant noise is ``tl.randn(42 + program_id, element)`` and the SiLU ALAM backward's
``tl.rand(42 + program_id, element)`` (Activation_Compression/act_triton_kernel.py:212-219;
activations/kernel_implementation.py). ``oracle_triton_rand`` / ``oracle_triton_randn`` restate
them in C from the Philox-4x32-10 words. Here a tiny ``@triton.jit`` kernel runs both under
Triton's CPU interpreter (``TRITON_INTERPRET=1``, in a child process, since the switch must be
set before triton is imported) for seeds 42, 43, 1042, just above 2^32 and 2^40, at offsets 0-511
and 511 random offsets up to 2^31 - 1 plus 2^31 - 1 itself: ``tl.rand`` must match bit for bit and
``tl.randn`` to 4 fp32 ulps of max(1, |value|) (the interpreter's log / cos are numpy's, the
oracle's the C library's).
"""
import json
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest

import oracle

SEEDS = (42, 43, 1042, 2**32 + 5, 2**40 + 3)

_CHILD = textwrap.dedent("""
    import json, os, sys
    os.environ["TRITON_INTERPRET"] = "1"
    import torch
    import triton
    import triton.language as tl

    @triton.jit
    def rand_kernel(offs_ptr, out_u, out_n, seed, N: tl.constexpr):
        i = tl.arange(0, N)
        offs = tl.load(offs_ptr + i)
        tl.store(out_u + i, tl.rand(seed, offs))
        tl.store(out_n + i, tl.randn(seed, offs))

    req = json.loads(sys.stdin.read())
    offs = torch.tensor(req["offsets"], dtype=torch.int32)
    res = {"triton": triton.__version__, "u": {}, "n": {}}
    for seed in req["seeds"]:
        u = torch.empty(offs.numel(), dtype=torch.float32)
        n = torch.empty(offs.numel(), dtype=torch.float32)
        rand_kernel[(1,)](offs, u, n, seed, N=offs.numel())
        res["u"][str(seed)] = u.view(torch.int32).tolist()
        res["n"][str(seed)] = n.tolist()
    print(json.dumps(res))
""")


def test_triton_rand_and_randn_match_the_oracle():
    pytest.importorskip("triton")
    rng = np.random.default_rng(0)
    offsets = np.concatenate([np.arange(512), rng.integers(512, 2**31 - 1, 511), [2**31 - 1]]).astype(np.int64)
    env = dict(os.environ, TRITON_INTERPRET="1")
    proc = subprocess.run([sys.executable, "-c", _CHILD], input=json.dumps({"offsets": offsets.tolist(),
                                                                            "seeds": list(SEEDS)}),
                          env=env, capture_output=True, text=True, timeout=600)
    assert proc.returncode == 0, proc.stderr[-2000:]
    res = json.loads(proc.stdout.strip().splitlines()[-1])
    for seed in SEEDS:
        got_u = np.array(res["u"][str(seed)], np.int32).view(np.float32)
        got_n = np.array(res["n"][str(seed)], np.float32)
        want_u = np.array([oracle.triton_rand(seed, int(o)) for o in offsets], np.float32)
        want_n = np.array([oracle.triton_randn(seed, int(o)) for o in offsets], np.float32)
        np.testing.assert_array_equal(got_u.view(np.int32), want_u.view(np.int32), err_msg=f"tl.rand seed {seed}")
        tol = 2.0 ** -21 * np.maximum(1.0, np.abs(want_n))
        bad = np.abs(got_n.astype(np.float64) - want_n) > tol
        assert not bad.any(), (seed, offsets[bad][:5], got_n[bad][:5], want_n[bad][:5])
