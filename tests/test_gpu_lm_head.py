"""Frozen LM head + exact chunked cross-entropy on the GPU: the row kernel
against the fp64 oracle, and the reference's own tests
(tests/kernels/test_frozen_linear_cross_entropy.py:11-186) restated."""
from __future__ import annotations

import numpy as np
import pytest
import torch
from torch.nn import functional as F

from oracle import nf4_oracle as O
from tests._util import assert_close_fro, np_f32

from molt_amd import ops
from molt_amd.errors import CapabilityError
from molt_amd.kernels.frozen_linear_cross_entropy import (_fused_frozen_head_forward, frozen_linear_cross_entropy,
                                                          frozen_linear_cross_entropy_loss_only)
from molt_amd.kernels.partitioned_loss import _AnalyticalHeadCrossEntropy, exact_partitioned_linear_cross_entropy

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,vocab,dtype", [(7, 317, torch.bfloat16), (16, 4096, torch.float32),
                                              (5, 151936, torch.bfloat16), (3, 64, torch.float32)])
def test_rows_kernel_matches_oracle(rows, vocab, dtype):
    print(f"cross-entropy rows R={rows} V={vocab} {dtype}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(rows + vocab)
    logits = (torch.randn(rows, vocab, generator=g) * 4.0).to("cuda", dtype)
    targets = torch.randint(0, vocab, (rows,), generator=g)
    targets[0] = -100            # ignored rows: zero loss, softmax gradient
    if rows > 2:
        targets[2] = vocab
    targets = targets.cuda()
    z = np_f32(logits).astype(np.float64)
    rl, rg = O.cross_entropy_rows(z, targets.cpu().numpy(), 11.0)
    work = logits.clone()
    loss = ops.cross_entropy_rows(work, targets, 11.0, True)
    np.testing.assert_allclose(np_f32(loss), rl, rtol=2e-6, atol=1e-7)
    if dtype == torch.float32:
        assert_close_fro(np_f32(work), rg, tol=1e-5, what="grad fp32")
    else:
        assert_close_fro(np_f32(work), rg, what="grad bf16")
    only = ops.cross_entropy_rows(logits.clone(), targets, 11.0, False)
    assert torch.equal(only, loss), "the loss-only pass must give the training loss bit for bit"


def test_large_vocabulary_repeated_calls_are_reproducible():
    torch.manual_seed(1337)
    hidden = torch.randn(256, 128, device="cuda", dtype=torch.bfloat16)
    weight = torch.randn(151936, 128, device="cuda", dtype=torch.bfloat16) * 0.1
    targets = torch.randint(151936, (256,), device="cuda")
    reference_loss, reference_grad = _fused_frozen_head_forward(hidden, weight, targets, 96)
    expected = F.cross_entropy(F.linear(hidden, weight).float(), targets)
    torch.testing.assert_close(reference_loss, expected, rtol=1e-5, atol=1e-5)
    with torch.enable_grad():
        h = hidden.detach().requires_grad_()
        analytical = _AnalyticalHeadCrossEntropy.apply(h, weight, targets, 96)
        analytical.backward()
    torch.testing.assert_close(reference_grad, h.grad, rtol=0, atol=2e-3)
    for _ in range(20):
        loss, grad = _fused_frozen_head_forward(hidden, weight, targets, 96)
        torch.testing.assert_close(loss, reference_loss, rtol=1e-6, atol=1e-6)
        assert torch.equal(grad, reference_grad)


def test_opcheck_cuda():
    h = torch.randn(8, 64, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    w = torch.randn(128, 64, device="cuda", dtype=torch.bfloat16)
    t = torch.randint(128, (8,), device="cuda")
    torch.library.opcheck(frozen_linear_cross_entropy, (h, w, t, 4))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_numerical_parity_against_unpartitioned_reference(dtype):
    torch.manual_seed(42)
    tokens, width, vocab, chunk = 128, 256, 4096, 64
    hidden = torch.randn(tokens, width, dtype=dtype)
    weight = torch.randn(vocab, width, dtype=dtype)
    targets = torch.randint(vocab, (tokens,))
    # reference: unpartitioned, same dtype, fp32 CE reduction (computed on the CPU)
    h_ref = hidden.clone().requires_grad_(True)
    loss_ref = F.cross_entropy(F.linear(h_ref, weight).float(), targets, reduction="mean")
    loss_ref.backward()
    h_test = hidden.cuda().requires_grad_(True)
    loss_test = frozen_linear_cross_entropy(h_test, weight.cuda(), targets.cuda(), chunk)
    loss_test.backward()
    assert abs(loss_test.item() - loss_ref.item()) / loss_ref.item() <= 1e-5
    assert (h_test.grad.cpu().float() - h_ref.grad.float()).abs().max().item() <= 2e-3


def test_chunked_loss_and_gradient_match_oracle():
    torch.manual_seed(7)
    tokens, width, vocab = 70, 96, 1000
    hidden = (torch.randn(tokens, width) * 0.5).to("cuda", torch.bfloat16).requires_grad_()
    weight = (torch.randn(vocab, width) * 0.1).to("cuda", torch.bfloat16)
    targets = torch.randint(vocab, (tokens,), device="cuda")
    loss = frozen_linear_cross_entropy(hidden, weight, targets, 32)
    loss.backward()
    hv, wv = np_f32(hidden).astype(np.float64), np_f32(weight).astype(np.float64)
    z = O.bf16_round((hv @ wv.T).astype(np.float32)).astype(np.float64)   # bf16 logits, as the GEMM stores them
    rl, rg = O.cross_entropy_rows(z, targets.cpu().numpy(), float(tokens))
    np.testing.assert_allclose(loss.item(), rl.sum(), rtol=1e-5)
    assert_close_fro(np_f32(hidden.grad), O.bf16_round(rg.astype(np.float32)).astype(np.float64) @ wv, what="dH")


def test_non_contiguous_and_batched_inputs():
    h = torch.randn(2, 8, 32, device="cuda", dtype=torch.bfloat16).transpose(0, 1).requires_grad_(True)
    assert not h.is_contiguous()
    w = torch.randn(64, 32, device="cuda", dtype=torch.bfloat16)
    t = torch.randint(64, (8, 2), device="cuda")
    loss = frozen_linear_cross_entropy(h, w, t, chunk_size=4)
    loss.backward()
    assert h.grad is not None and h.grad.shape == h.shape
    ref = F.cross_entropy(F.linear(h.detach().float().reshape(-1, 32).cpu(), w.float().cpu()),
                          t.reshape(-1).cpu())
    assert abs(loss.item() - ref.item()) / ref.item() < 2e-2


def test_adversarial_logits_stability():
    h = (torch.randn(4, 32, device="cuda", dtype=torch.float32) * 50.0).requires_grad_(True)
    w = torch.randn(64, 32, device="cuda", dtype=torch.float32) * 50.0
    t = torch.randint(64, (4,), device="cuda")
    loss = frozen_linear_cross_entropy(h, w, t, chunk_size=2)
    loss.backward()
    assert torch.isfinite(loss) and torch.isfinite(h.grad).all()


def test_odd_vocabulary_tail():
    h = torch.randn(5, 47, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    w = torch.randn(317, 47, device="cuda", dtype=torch.bfloat16)
    t = torch.randint(317, (5,), device="cuda")
    loss = frozen_linear_cross_entropy(h, w, t, chunk_size=2)
    loss.backward()
    assert torch.isfinite(loss) and torch.isfinite(h.grad).all()


def test_partitioned_loss_backend_dispatch():
    h = torch.randn(16, 64, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    w = torch.randn(128, 64, device="cuda", dtype=torch.bfloat16)
    t = torch.randint(128, (16,), device="cuda")
    kw = dict(precompute_frozen_gradient=True)
    l_auto = exact_partitioned_linear_cross_entropy(h, w, t, 8, backend="auto", **kw)
    l_fused = exact_partitioned_linear_cross_entropy(h, w, t, 8, backend="triton", **kw)
    l_anal = exact_partitioned_linear_cross_entropy(h, w, t, 8, backend="analytical", **kw)
    l_recompute = exact_partitioned_linear_cross_entropy(h, w, t, 8)
    assert abs(l_auto.item() - l_fused.item()) < 1e-5
    assert abs(l_fused.item() - l_anal.item()) < 1e-4
    assert abs(l_fused.item() - l_recompute.item()) < 1e-4
    l_recompute.backward()
    assert h.grad is not None and torch.isfinite(h.grad).all()


def test_fp32_hidden_with_bf16_frozen_head():
    h = torch.randn(8, 64, device="cuda", dtype=torch.float32, requires_grad=True)
    w = torch.randn(128, 64, device="cuda", dtype=torch.bfloat16)
    t = torch.randint(128, (8,), device="cuda")
    loss = exact_partitioned_linear_cross_entropy(h, w, t, 4, precompute_frozen_gradient=True, backend="triton")
    loss.backward()
    assert h.grad is not None and h.grad.dtype == torch.float32
    assert torch.isfinite(loss) and torch.isfinite(h.grad).all()


def test_loss_only_path_is_bit_exact_to_training_loss():
    torch.manual_seed(91)
    hidden = torch.randn(16, 64, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    weight = torch.randn(151936, 64, device="cuda", dtype=torch.bfloat16)
    targets = torch.randint(151936, (16,), device="cuda")
    training = exact_partitioned_linear_cross_entropy(hidden, weight, targets, 8, precompute_frozen_gradient=True,
                                                      backend="triton")
    with torch.no_grad():
        evaluation = exact_partitioned_linear_cross_entropy(hidden, weight, targets, 8,
                                                            precompute_frozen_gradient=True, backend="triton")
    assert torch.equal(evaluation, training.detach())
    assert torch.equal(frozen_linear_cross_entropy_loss_only(hidden.detach(), weight, targets, 8), evaluation)


@pytest.mark.parametrize("chunk_size", [1, 3, 8, 32])
def test_recomputing_backend_matches_unpartitioned_loss_and_both_gradients(chunk_size):
    """tests/test_molt_stream_partitioned_loss.py:7-25 in fp32 on the GPU (the
    row kernel reduces in fp32) against fp64 autograd on the CPU, with a
    trainable head: loss, hidden gradient and head gradient."""
    torch.manual_seed(17)
    hidden64 = torch.randn(2, 4, 7, dtype=torch.float64, requires_grad=True)
    weight64 = torch.randn(11, 7, dtype=torch.float64, requires_grad=True)
    targets = torch.randint(0, 11, (2, 4))
    reference = F.cross_entropy(F.linear(hidden64, weight64).flatten(0, 1), targets.flatten())
    reference.backward()
    hidden = hidden64.detach().float().cuda().requires_grad_()
    weight = weight64.detach().float().cuda().requires_grad_()
    loss = exact_partitioned_linear_cross_entropy(hidden, weight, targets.cuda(), chunk_size)
    loss.backward()
    torch.testing.assert_close(loss.double().cpu(), reference.detach(), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(hidden.grad.double().cpu(), hidden64.grad, rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(weight.grad.double().cpu(), weight64.grad, rtol=1e-4, atol=1e-6)
    with pytest.raises(CapabilityError, match="float64"):
        exact_partitioned_linear_cross_entropy(hidden64.detach().cuda(), weight64.detach().cuda(), targets.cuda(),
                                               chunk_size)


@pytest.mark.parametrize("grad_scale", [1.0, -0.5])
def test_recomputing_backend_ignored_targets_and_signed_upstream_gradient(grad_scale):
    """The exact path follows F.cross_entropy as the reference's exact path
    calls it (kernels/partitioned_loss.py:43-101: summed over chunks, divided by
    every token): targets of -100 add nothing to the loss and get a zero
    gradient, and the upstream gradient may be negative. Against fp64 autograd
    of that formulation on the CPU, with a trainable head."""
    torch.manual_seed(19)
    hidden64 = torch.randn(3, 5, 9, dtype=torch.float64, requires_grad=True)
    weight64 = torch.randn(13, 9, dtype=torch.float64, requires_grad=True)
    targets = torch.randint(0, 13, (3, 5))
    targets[0, 1] = targets[2, 4] = targets[1, 0] = -100
    ref = F.cross_entropy(F.linear(hidden64, weight64).flatten(0, 1), targets.flatten(), reduction="sum")
    ref = ref / targets.numel()
    (ref * grad_scale).backward()
    hidden = hidden64.detach().float().cuda().requires_grad_()
    weight = weight64.detach().float().cuda().requires_grad_()
    loss = exact_partitioned_linear_cross_entropy(hidden, weight, targets.cuda(), 4)
    (loss * grad_scale).backward()
    torch.testing.assert_close(loss.double().cpu(), ref.detach(), rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(hidden.grad.double().cpu(), hidden64.grad, rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(weight.grad.double().cpu(), weight64.grad, rtol=1e-4, atol=1e-6)
    assert torch.count_nonzero(hidden.grad[0, 1]) == 0 and torch.count_nonzero(hidden.grad[2, 4]) == 0


def test_recomputing_backend_rejects_out_of_range_targets():
    hidden = torch.randn(2, 3, 8, device="cuda", requires_grad=True)
    weight = torch.randn(5, 8, device="cuda")
    for bad in (5, -1, -7):
        targets = torch.zeros(2, 3, dtype=torch.long, device="cuda")
        targets[1, 2] = bad
        with pytest.raises(IndexError, match="out of bounds"):
            exact_partitioned_linear_cross_entropy(hidden, weight, targets, 2)
