"""c3hip_linear_fwd_noalloc (workspace in the library's static scratch) against
c3hip_linear_fwd (workspace from the stream-ordered pool), through the C ABI.

Both run the same kernels with the same launch plan, so their outputs must be
identical bit for bit, on real-valued inputs too.  The shapes are ones the
size heuristic splits over k, so the split-K partials go through the scratch:
bf16 1024x8192x1024 splits 8 ways (32 MiB of partials, the whole scratch) and
576x8192x576 16 ways (21 MiB); fp32 128x784x256 splits 6 ways.  Each pair
runs twice in a row, the second call on a smaller problem, so the second
call sees the scratch holding the first call's partials.
"""
import numpy as np
import pytest
import torch

from c3_amd import native as N
from oracle import oracle as O
from tests.parity import dev, dev_bf16, empty, host, ptr

pytestmark = pytest.mark.gpu


def _pair(dtype, M, K, Nn, act, seed, stream):
    bf = dtype == N.BF16
    X = O.normal(seed, (M, K))
    W = O.normal(seed + 1, (K, Nn), 0.0, 1.0 / np.sqrt(K))
    b = O.normal(seed + 2, Nn, 0.0, 0.1)
    up = dev_bf16 if bf else dev
    X_, W_, b_ = up(X), up(W), dev(b)
    tdt = torch.bfloat16 if bf else torch.float32
    Y_pool = empty((M, Nn), dtype=tdt)
    Y_static = empty((M, Nn), dtype=tdt)
    N.linear_fwd_noalloc(dtype, ptr(X_), ptr(W_), ptr(b_), ptr(Y_static), M, K, Nn, act, stream)
    N.linear_fwd(dtype, ptr(X_), ptr(W_), ptr(b_), ptr(Y_pool), M, K, Nn, act, stream)
    got, ref = host(Y_static), host(Y_pool)
    assert np.all(np.isfinite(got)), "unwritten or non-finite outputs"
    bad = got.view(np.int32) != ref.view(np.int32)
    assert not bad.any(), f"{M}x{K}x{Nn}: {int(bad.sum())} elements differ from c3hip_linear_fwd"


@pytest.mark.parametrize("act", [N.ACT_RELU, N.ACT_NONE])
def test_noalloc_bf16_split_k_matches_pool_workspace(gpu, stream, act):
    _pair(N.BF16, 1024, 8192, 1024, act, 0x0A11, stream)   # 8-way split: 32 MiB, the whole scratch
    _pair(N.BF16, 576, 8192, 576, act, 0x0A12, stream)     # then a smaller one (16-way, 21 MiB)


def test_noalloc_fp32_split_k_matches_pool_workspace(gpu, stream):
    _pair(N.F32, 128, 784, 256, N.ACT_RELU, 0x0A21, stream)
    _pair(N.F32, 64, 784, 128, N.ACT_RELU, 0x0A22, stream)


def test_noalloc_without_split_matches(gpu, stream):
    _pair(N.F32, 1024, 512, 1024, N.ACT_RELU, 0x0A31, stream)
    _pair(N.BF16, 2048, 1024, 2048, N.ACT_RELU, 0x0A32, stream)


def test_noalloc_rejects_workspace_beyond_scratch(gpu, stream):
    # A forced 256x256 split tile plans 8 x 1024 x 2048 fp32 partials (64 MiB):
    # more than the scratch, so the call fails before launching anything.
    M, K, Nn = 1024, 8192, 2048
    X_ = dev_bf16(O.normal(1, (M, K)))
    W_ = dev_bf16(O.normal(2, (K, Nn), 0.0, 0.01))
    Y = empty((M, Nn), dtype=torch.bfloat16)
    N.set_gemm_tile(N.BF16, "d256w8")
    try:
        with pytest.raises(N.C3HipError) as ei:
            N.linear_fwd_noalloc(N.BF16, ptr(X_), ptr(W_), None, ptr(Y), M, K, Nn, N.ACT_NONE, stream)
    finally:
        N.set_gemm_tile(N.BF16, None)
    assert ei.value.code == N.ERR_TOO_LARGE
    assert "workspace" in str(ei.value)
    assert np.all(np.isnan(host(Y))), "a rejected call wrote its output"
