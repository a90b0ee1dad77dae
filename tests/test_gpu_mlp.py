"""GPU train step of an MLP through C3's dispatch flow (c3_amd/trainer.py over
MlpTrainer), checked against the oracle.

Each step's intermediates are read back and every stage is checked on the
GPU's own inputs to it ("teacher forcing"), with the GEMM bounds of
tests/parity.py: forward layer l from activation l, CE from the logits,
backward layer l from the gradient arriving at its output, SGD bit-exact from
the GPU's dW/db.  The whole chain is also compared with a pure oracle chain
(normwise rel-err).  The first step runs eagerly (nothing installed yet);
after warm-up every ReLU layer runs as a region kernel and every layer
backward as a fused kernel, and the same checks hold.
"""
import numpy as np
import pytest
import torch

from c3_amd import native as N
from c3_amd import trainer as T
from oracle import oracle as O
from tests.parity import (U, assert_close_gemm, check_ce, dev, empty, gemm_bound, host, mask_flips, ptr)

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
BF16_TOL = 1e-2
BF16_ROUND = 2.0 ** -8  # one RNE rounding to bf16 is <= 2^-9 relative; twice that as slack


def kaiming_uniform(seed, fan_in, fan_out):
    bound = np.sqrt(6.0 / fan_in)
    return O.uniform(seed, (fan_in, fan_out), -bound, bound)


def fetch(p, shape, dtype, stream):
    """Copy a device buffer of the trainer into a host fp32 array (bf16 widened exactly)."""
    n = int(np.prod(shape))
    out = empty(n)
    N.cast(dtype, N.F32, p, ptr(out), n, stream)
    return host(out).reshape(shape)


def upload_params(tr, Ws, bs, stream):
    for l, (W, b) in enumerate(zip(Ws, bs)):
        wp, bp = tr.params(l)
        N.cast(N.F32, tr.dtype, ptr(dev(W)), wp, W.size, stream)
        N.cast(N.F32, N.F32, ptr(dev(b)), bp, b.size, stream)
    torch.cuda.synchronize()


def make_problem(dims, batch, seed, dtype):
    X = O.uniform(seed, (batch, dims[0]))
    Ws = [kaiming_uniform(seed + 1 + l, dims[l], dims[l + 1]) for l in range(len(dims) - 1)]
    bs = [O.normal(seed + 20 + l, dims[l + 1], 0.0, 0.1) for l in range(len(dims) - 1)]
    if dtype == N.BF16:
        X = O.round_bf16(X)
        Ws = [O.round_bf16(W) for W in Ws]
    lbl = O.labels(seed + 40, batch, dims[-1])
    return X, Ws, bs, lbl


def upload_input(X, dtype):
    if dtype == N.BF16:
        from tests.parity import dev_bf16

        return dev_bf16(X)
    return dev(X)


def check_step(tr, X, Ws, bs, lbl, lr, loss, stream):
    """Teacher-forced checks of one step whose parameters before the step were Ws, bs."""
    dt = tr.dtype
    L = tr.num_layers
    dims = tr.dims
    B = tr.batch
    tol = FP32_TOL if dt == N.F32 else BF16_TOL
    out_round = 0.0 if dt == N.F32 else BF16_ROUND
    acts = [fetch(tr.tensor(T.ACTIVATION, l), (B, dims[l]), dt, stream) for l in range(L + 1)]
    assert np.array_equal(acts[0], X)
    # Forward, layer by layer.
    for l in range(L):
        relu = l + 1 < L
        t = O.matmul(acts[l], Ws[l])
        z = O.bias_act(t, bs[l], act=0)
        ref = O.bias_act(t, bs[l], act=1 if relu else 0)
        bound = gemm_bound(acts[l], Ws[l], dims[l])
        assert_close_gemm(acts[l + 1], ref, bound, tol, out_round, what=f"Y{l}")
        if relu:
            mask_flips(acts[l + 1], z, bound + out_round * np.abs(z))
    # Loss and its gradient from the GPU's logits.
    g = [fetch(tr.tensor(T.OUTPUT_GRAD, l), (B, dims[l + 1]), dt, stream) for l in range(L)]
    ref_loss, ref_d, ref_rows = O.softmax_ce(acts[L], lbl, want_rows=True)
    check_ce(None, g[L - 1], acts[L], lbl, ref_rows, ref_d, d_round=out_round)
    assert abs(loss - ref_loss) <= 1e-5 * max(1.0, abs(ref_loss)), (loss, ref_loss)
    # Backward, layer by layer, from the gradient arriving at each output.
    for l in range(L):
        relu = l + 1 < L
        rX, rW, rb = O.linear_bwd(acts[l], Ws[l], acts[l + 1], g[l], 1 if relu else 0)
        dZ = O.relu_mask_mul(acts[l + 1], g[l]) if relu else g[l]
        dW = fetch(tr.tensor(T.WEIGHT_GRAD, l), (dims[l], dims[l + 1]), N.F32, stream)
        db = fetch(tr.tensor(T.BIAS_GRAD, l), (dims[l + 1],), N.F32, stream)
        assert_close_gemm(dW, rW, gemm_bound(acts[l].T, dZ, B), tol, what=f"dW{l}")
        assert_close_gemm(db, rb, 2.02 * B * U * np.abs(dZ.astype(np.float64)).sum(0), tol, what=f"db{l}")
        if l > 0:
            assert_close_gemm(g[l - 1], rX, gemm_bound(dZ, Ws[l].T, dims[l + 1]), tol, out_round, what=f"dX{l}")
        # SGD from the GPU's gradients: bit-exact.
        wp, bp = tr.params(l)
        W_after = fetch(wp, (dims[l], dims[l + 1]), dt, stream)
        b_after = fetch(bp, (dims[l + 1],), N.F32, stream)
        if dt == N.BF16:
            ref_w = O.bf16_bits_to_f32(O.sgd_update(O.pack_bf16(Ws[l]), dW, lr))
        else:
            ref_w = O.sgd_update(Ws[l], dW, lr)
        assert np.array_equal(W_after, ref_w.reshape(W_after.shape)), f"W{l} after SGD"
        assert np.array_equal(b_after, O.sgd_update(bs[l], db, lr)), f"b{l} after SGD"
    return acts, g


def oracle_chain(X, Ws, bs, lbl):
    """Pure oracle forward + CE + backward: (loss, [dW_l], [db_l])."""
    L = len(Ws)
    acts = [X]
    for l in range(L):
        acts.append(O.linear_fwd(acts[-1], Ws[l], bs[l], act=1 if l + 1 < L else 0))
    loss, d = O.softmax_ce(acts[L], lbl)
    dWs, dbs = [None] * L, [None] * L
    g = d
    for l in reversed(range(L)):
        dX, dWs[l], dbs[l] = O.linear_bwd(acts[l], Ws[l], acts[l + 1], g, 1 if l + 1 < L else 0)
        g = dX
    return loss, dWs, dbs


def run_checked_step(tr, X, Ws, bs, lbl, lr, stream):
    upload_params(tr, Ws, bs, stream)
    dX = upload_input(X, tr.dtype)
    dl = dev(np.ascontiguousarray(lbl, dtype=np.int32))
    loss = tr.step(ptr(dX), ptr(dl), lr, want_loss=True, stream=stream)
    check_step(tr, X, Ws, bs, lbl, lr, loss, stream)
    return loss


def test_mlp_784_256_128_10_fp32_train_step(gpu, stream):
    dims, batch, lr = [784, 256, 128, 10], 128, 0.05
    X, Ws, bs, lbl = make_problem(dims, batch, 0xC3, N.F32)
    tr = T.MlpTrainer(dims, batch, N.F32)
    tr.keep_gradients(True)
    # Step 1: nothing installed yet, every op eager.
    loss = run_checked_step(tr, X, Ws, bs, lbl, lr, stream)
    s = tr.stats()
    assert s["region_hits"] == 0 and s["backward_misses"] == 3 and s["fully_dispatched"] == 0
    # End-to-end against the pure oracle chain.
    ref_loss, rW, rb = oracle_chain(X, Ws, bs, lbl)
    assert abs(loss - ref_loss) <= 1e-5 * abs(ref_loss)
    for l in range(3):
        dW = fetch(tr.tensor(T.WEIGHT_GRAD, l), rW[l].shape, N.F32, stream)
        rel = np.max(np.abs(dW - rW[l])) / np.max(np.abs(rW[l]))
        assert rel <= FP32_TOL, f"dW{l} end-to-end rel err {rel:.2e}"
    # Warm up: regions and fused backwards compile in the background.
    dXb = dev(X)
    dl = dev(lbl.astype(np.int32))
    steps = tr.warm_up(ptr(dXb), ptr(dl), lr, 16, stream)
    assert steps < 16 and tr.stats()["fully_dispatched"] == 1
    # The same step on the fused path.
    before = tr.stats()
    loss2 = run_checked_step(tr, X, Ws, bs, lbl, lr, stream)
    after = tr.stats()
    assert after["region_hits"] - before["region_hits"] == 2
    assert after["backward_hits"] - before["backward_hits"] == 3
    assert after["fully_dispatched"] == 1
    assert abs(loss2 - ref_loss) <= 1e-5 * abs(ref_loss)
    # Training lowers the loss.
    first = tr.step(ptr(dXb), ptr(dl), lr, want_loss=True, stream=stream)
    for _ in range(20):
        last = tr.step(ptr(dXb), ptr(dl), lr, want_loss=True, stream=stream)
    assert last < first
    tr.close()


def test_mlp_bf16_train_step(gpu, stream):
    # 200 classes: a multiple of 8 (bf16 vector extents) but not of 64, so the
    # last layer's dX (inner extent 200) takes the register-staged kernels.
    dims, batch, lr = [256, 512, 384, 200], 256, 0.05
    X, Ws, bs, lbl = make_problem(dims, batch, 0xB16, N.BF16)
    tr = T.MlpTrainer(dims, batch, N.BF16)
    tr.keep_gradients(True)
    run_checked_step(tr, X, Ws, bs, lbl, lr, stream)
    assert tr.stats()["backward_misses"] == 3
    dXb = upload_input(X, N.BF16)
    dl = dev(lbl.astype(np.int32))
    steps = tr.warm_up(ptr(dXb), ptr(dl), lr, 16, stream)
    assert steps < 16 and tr.stats()["fully_dispatched"] == 1
    before = tr.stats()
    run_checked_step(tr, X, Ws, bs, lbl, lr, stream)
    after = tr.stats()
    assert after["region_hits"] - before["region_hits"] == 2
    assert after["backward_hits"] - before["backward_hits"] == 3
    tr.close()


def test_trainer_rejects_bad_arguments(gpu, stream):
    with pytest.raises(T.TrainerError):
        T.MlpTrainer([10], 4)
    with pytest.raises(T.TrainerError):
        T.MlpTrainer([10, 0, 3], 4)
    tr = T.MlpTrainer([8, 4], 2)
    with pytest.raises(T.TrainerError, match="not kept"):
        tr.tensor(T.WEIGHT_GRAD, 0)
    with pytest.raises(T.TrainerError):
        tr.params(5)
    tr.close()


def test_graph_replay_equals_eager_steps(gpu):
    # A captured train step replayed N times leaves the parameters bit for bit
    # where N eager steps do (same kernels, same launch shapes).
    dims, batch, lr = [784, 256, 128, 10], 128, 0.05
    X, Ws, bs, lbl = make_problem(dims, batch, 0xC5, N.F32)
    side = torch.cuda.Stream()
    s = side.cuda_stream
    dXb, dl = dev(X), dev(lbl.astype(np.int32))
    A = T.MlpTrainer(dims, batch, N.F32)
    B = T.MlpTrainer(dims, batch, N.F32)
    with torch.cuda.stream(side):
        upload_params(A, Ws, bs, s)
        upload_params(B, Ws, bs, s)
        warm = A.warm_up(ptr(dXb), ptr(dl), lr, 16, s)
        A.capture(ptr(dXb), ptr(dl), lr, s)       # one real step, then the recorded one
        for _ in range(5):
            A.replay(s)
        for _ in range(warm + 1 + 5):
            B.step(ptr(dXb), ptr(dl), lr, want_loss=False, stream=s)
        side.synchronize()
        for l in range(3):
            for which in range(2):
                pa, pb = A.params(l)[which], B.params(l)[which]
                n = dims[l] * dims[l + 1] if which == 0 else dims[l + 1]
                va, vb = fetch(pa, (n,), N.F32, s), fetch(pb, (n,), N.F32, s)
                assert np.array_equal(va.view(np.int32), vb.view(np.int32)), (l, which)
    assert A.stats()["graph_replays"] == 5
    with pytest.raises(T.TrainerError, match="default stream"):
        A.capture(ptr(dXb), ptr(dl), lr, 0)
    A.close()
    B.close()
