"""Gathered-row consumers through the C ABI: the selected-row LM head
(candidate logits) and the embedding row gather, for Q4_K and Q6_K rows.

Bars: the embedding gather is bit-exact with the oracle dequant (the
reference's q3_quant.c order, pinned by the golden vectors); candidate
logits (fp32 weights times fp32 hidden, as the reference's
candidate_logits_kernel) are within 1e-3 * rms of the double-precision
oracle, and invalid ids give NaN.
"""
import sys

import numpy as np
import pytest

import q3q4
from oracle import oracle

pytestmark = pytest.mark.gpu
TOL = 1e-3


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as _t
    if not _t.cuda.is_available():
        pytest.fail("gpu test without a visible HIP device")
    q3q4.load()
    return _t


def dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def weights(rng, qtype, N, K):
    if qtype == 12:
        return oracle.quantize_q4k((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
    return oracle.q6k_weights(rng, N, K)


def dequant(qtype, W, N, K):
    return oracle.dequant(W, N, K) if qtype == 12 else oracle.dequant_q6k(W, N, K)


@pytest.mark.parametrize("qtype", [12, 14])
@pytest.mark.parametrize("N,K", [(300, 256), (1001, 5120), (77, 2304)])
def test_embedding_bit_exact(torch, qtype, N, K):
    say(f"case embedding qtype={qtype} N={N} K={K}")
    rng = np.random.default_rng(qtype * 1000 + N + K)
    W = weights(rng, qtype, N, K)
    ids = rng.integers(0, N, 37).astype(np.uint32)
    ids[5] = N + 3                                   # invalid: row left untouched
    out = torch.full((len(ids), K), 7.25, dtype=torch.float32, device="cuda")
    q3q4.embedding(qtype, dev(torch, W), N, K, dev(torch, ids.astype(np.int32)), out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    ref = dequant(qtype, W, N, K)
    for t, i in enumerate(ids):
        if i >= N:
            assert np.all(got[t] == 7.25)
        else:
            assert np.array_equal(got[t].view(np.uint32), ref[i].view(np.uint32)), t


@pytest.mark.parametrize("qtype", [12, 14])
@pytest.mark.parametrize("N,K,branches,per", [(500, 256, 1, 17), (2048, 5120, 16, 64), (333, 2304, 3, 5)])
def test_candidate_logits(torch, qtype, N, K, branches, per):
    say(f"case candidate logits qtype={qtype} N={N} K={K} branches={branches} per={per}")
    rng = np.random.default_rng(qtype + N * 3 + K + branches)
    W = weights(rng, qtype, N, K)
    hidden = rng.standard_normal((branches, K)).astype(np.float32)
    ids = rng.integers(0, N, branches * per).astype(np.uint32)
    ids[-1] = N                                      # invalid id -> NaN
    logits = torch.full((branches * per,), 3.0, dtype=torch.float32, device="cuda")
    q3q4.candidate_logits(qtype, dev(torch, W), N, K, dev(torch, hidden), dev(torch, ids.astype(np.int32)), per,
                          logits)
    torch.cuda.synchronize()
    got = logits.cpu().numpy()
    deq = dequant(qtype, W, N, K).astype(np.float64)
    ref = np.array([deq[i] @ hidden[b].astype(np.float64) if i < N else np.nan
                    for b in range(branches) for i in ids[b * per:(b + 1) * per]])
    assert np.isnan(got[-1])
    ok = ~np.isnan(ref)
    rms = float(np.sqrt(np.mean(ref[ok] ** 2)))
    err = float(np.max(np.abs(got[ok] - ref[ok])))
    say(f"  max|err| = {err:.3e}, rms = {rms:.3e}")
    assert np.all(np.isfinite(got[ok])) and err <= TOL * rms


def test_candidate_logits_full_lm_head(torch):
    """Q6_K output.weight shape 151936 x 5120 (the stock Q4_K_M LM head), 16
    branches x 128 candidates; weights made on the device, every logit
    checked."""
    say("case candidate logits full LM head")
    N, K = 151936, 5120
    gen = torch.Generator(device="cuda").manual_seed(11)
    Wd = torch.randint(0, 256, (N, K // 256, 210), generator=gen, device="cuda", dtype=torch.uint8)
    d = (torch.rand((N, K // 256), generator=gen, device="cuda") + 0.5) * 2e-5
    Wd[:, :, 208:210] = d.to(torch.float16).view(torch.uint8).view(N, K // 256, 2)
    rng = np.random.default_rng(12)
    branches, per = 16, 128
    hidden = rng.standard_normal((branches, K)).astype(np.float32)
    ids = rng.integers(0, N, branches * per).astype(np.uint32)
    logits = torch.empty(branches * per, dtype=torch.float32, device="cuda")
    q3q4.candidate_logits(14, Wd, N, K, dev(torch, hidden), dev(torch, ids.astype(np.int32)), per, logits)
    torch.cuda.synchronize()
    got = logits.cpu().numpy()
    rows = Wd.view(N, -1)[torch.from_numpy(ids.astype(np.int64)).cuda()].cpu().numpy()
    deq = oracle.dequant_q6k(rows, len(ids), K).astype(np.float64)
    ref = np.einsum("ik,ik->i", deq, np.repeat(hidden, per, axis=0).astype(np.float64))
    rms = float(np.sqrt(np.mean(ref ** 2)))
    err = float(np.max(np.abs(got - ref)))
    say(f"  max|err| = {err:.3e}, rms = {rms:.3e}")
    assert err <= TOL * rms
