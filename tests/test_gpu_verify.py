"""GPU parity of the fused rejection-sampling kernels (csrc/verify.hip through
the C ABI) with oracle/decoder_ops.verify_batch on the same inputs and the same
Philox noise: accepted length, per-candidate mask and bonus token must be equal
(both sides evaluate the same fp32 formulas; their reduction orders differ, so
a decision could flip only at a tie within fp32 rounding, which these seeded
cases do not contain — the asserts are exact). Then the
reference's own rejection-sampling checks (tests/test_spec_decode.py:78-323 of
the reference) run on the device: cases A/B/C, losslessness by TV convergence,
logits-not-probabilities and candidate/row alignment.
"""
import numpy as np
import pytest
import torch

from oracle import decoder_ops as od
from specdec_nanovllm_amd import ops
from specdec_nanovllm_amd.spec_decode.verify import VerifyResult, verify_batch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def state(seed, offset=0):
    return torch.tensor([seed, offset], dtype=torch.int64, device=DEV)


def run(dl, tl, toks, temps=None, point_mass=False, seed=0, offset=0):
    r = verify_batch(dl.to(DEV), tl.to(DEV), toks.to(DEV),
                     None if temps is None else temps.to(DEV), point_mass, state(seed, offset))
    return r.accepted.cpu().numpy(), r.bonus.cpu().numpy(), r.accept_mask.cpu().numpy()


def oracle(dl, tl, toks, temps=None, point_mass=False, seed=0, offset=0):
    return od.verify_batch(dl.float().numpy(), tl.float().numpy(), toks.numpy(),
                           None if temps is None else temps.numpy(), point_mass, seed, offset)


@pytest.mark.parametrize("B,k,V,ddt,tdt", [(8, 6, 151936, torch.float32, torch.float32),
                                            (8, 6, 151936, torch.float32, torch.bfloat16),
                                            (3, 2, 1000, torch.bfloat16, torch.bfloat16),
                                            (5, 1, 7, torch.float32, torch.float16)])
def test_matches_oracle(B, k, V, ddt, tdt):
    g = torch.Generator().manual_seed(B * 100 + k)
    tl = (torch.randn((B, k + 1, V), generator=g) * 3).to(tdt)
    # a draft near the target, so acceptance actually varies
    dl = (tl[:, :k].float() + torch.randn((B, k, V), generator=g)).to(ddt)
    q = torch.softmax(dl.float(), -1)
    toks = torch.stack([torch.multinomial(q[b], 1, generator=g)[:, 0] for b in range(B)])
    temps = torch.linspace(0.6, 1.4, B)
    got = run(dl, tl, toks, temps, seed=77, offset=5)
    want = oracle(dl, tl, toks, temps, seed=77, offset=5)
    assert np.array_equal(got[0], want[0]), (got[0], want[0])
    assert np.array_equal(got[2], want[2])
    assert np.array_equal(got[1], want[1]), (got[1], want[1])


def test_point_mass_matches_oracle():
    B, k, V = 16, 3, 500
    g = torch.Generator().manual_seed(5)
    tl = torch.randn((B, k + 1, V), generator=g)
    toks = torch.randint(0, V, (B, k), generator=g)
    dq = torch.zeros((B, k, V))
    dq.scatter_(2, toks[:, :, None], 1.0)
    got = run(dq, tl, toks, point_mass=True, seed=3)
    want = oracle(dq, tl, toks, point_mass=True, seed=3)
    for a, b in zip(got, want):
        assert np.array_equal(a, b)


def test_result_type_and_default_noise_advances():
    g = torch.Generator().manual_seed(6)
    tl = torch.randn((4, 3, 50), generator=g).to(DEV)
    dl = torch.randn((4, 2, 50), generator=g).to(DEV)
    toks = torch.randint(0, 50, (4, 2), generator=g).to(DEV)
    r1 = verify_batch(dl, tl, toks)
    assert isinstance(r1, VerifyResult)
    assert r1.accepted.dtype == torch.int64 and r1.bonus.dtype == torch.int64
    assert r1.accept_mask.dtype == torch.bool and r1.n_proposed.tolist() == [2] * 4
    draws = {tuple(verify_batch(dl, tl, toks).bonus.tolist()) for _ in range(8)}
    assert len(draws) > 1  # the default state's offset moves between calls


def test_graph_replays_draw_fresh_noise():
    g = torch.Generator().manual_seed(8)
    tl = torch.zeros((64, 2, 30), device=DEV)
    dl = torch.zeros((64, 1, 30), device=DEV)
    toks = torch.randint(0, 30, (64, 1), generator=g).to(DEV)
    st = state(123, 0)
    out = {}

    def step():
        out["r"] = ops.verify_batch(dl, tl, toks, rng_state=st)
        st[1:].add_(1)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    seen = []
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        seen.append(out["r"][1].clone())
        # the eager warm-up used offset 0; capture runs nothing; replay r uses 1 + r
        want = od.verify_batch(dl.cpu().numpy(), tl.cpu().numpy(), toks.cpu().numpy(),
                               seed=123, offset=1 + rep)
        assert np.array_equal(out["r"][1].cpu().numpy(), want[1])
    assert not torch.equal(seen[0], seen[1])


# --------------------------------------------------- the reference's own checks
def test_reference_case_a_equal_distributions_accept_all():
    g = torch.Generator().manual_seed(0)
    dl = torch.randn((1, 3, 20), generator=g)
    tl = torch.cat([dl, torch.randn((1, 1, 20), generator=g)], 1)
    probs = torch.softmax(dl[0], -1)
    toks = torch.stack([torch.multinomial(probs[j], 1, generator=g)[0] for j in range(3)])[None]
    for seed in range(10):
        acc, _, mask = run(dl, tl, toks, seed=seed)
        assert acc.tolist() == [3] and mask.all()


def test_reference_case_b_sharp_target():
    dl = torch.zeros((1, 3, 20))
    dl[:, 0, 7] = 50.0
    tl = torch.full((1, 4, 20), -50.0)
    tl[:, :, 7] = 50.0
    for seed in range(10):
        acc, _, _ = run(dl, tl, torch.zeros((1, 3), dtype=torch.int64), seed=seed)
        assert acc[0] <= 1


def test_reference_case_c_bonus_on_target_mode():
    N, V = 4000, 20
    pc = torch.full((V,), 1e-6)
    pc[5] = 1.0
    tl = pc.log().view(1, 1, V).expand(N, 2, V).contiguous()
    toks = torch.full((N, 1), 3, dtype=torch.int64)
    dq = torch.zeros((N, 1, V))
    dq.scatter_(2, toks[:, :, None], 1.0)
    acc, bonus, _ = run(dq, tl, toks, point_mass=True, seed=2)
    assert (acc == 0).all() and np.bincount(bonus, minlength=V).argmax() == 5


def _tv(N, seed):
    probs = torch.tensor([0.5, 0.2, 0.15, 0.05, 0.05, 0.05])
    g = torch.Generator().manual_seed(seed)
    d = torch.multinomial(probs.expand(N, 6), 1, replacement=True, generator=g)
    dq = torch.zeros((N, 1, 6))
    dq.scatter_(2, d[:, :, None], 1.0)
    tl = probs.log().view(1, 1, 6).expand(N, 2, 6).contiguous()
    acc, bonus, _ = run(dq, tl, d, point_mass=True, seed=seed, offset=seed)
    final = np.where(acc == 1, d[:, 0].numpy(), bonus)
    h = np.bincount(final, minlength=6) / N
    return 0.5 * np.abs(h - probs.numpy()).sum()


def test_reference_lossless_tv_converges():
    small = np.mean([_tv(40_000, s) for s in range(5)])
    large = np.mean([_tv(400_000, s) for s in range(3)])
    assert small / large > 2.0 and large < 0.004, (small, large)


def test_reference_draft_side_must_be_logits():
    p5 = torch.tensor([0.5, 0.2, 0.15, 0.05, 0.05, 0.05])
    N = 200_000
    g = torch.Generator().manual_seed(0)
    cand = torch.multinomial(p5.expand(N, 6), 1, replacement=True, generator=g)
    tgt = p5.log().view(1, 1, 6).expand(N, 2, 6).contiguous()

    def acc_tv(side):
        acc, bonus, _ = run(side, tgt, cand, seed=4)
        h = np.bincount(np.where(acc == 1, cand[:, 0].numpy(), bonus), minlength=6) / N
        return (acc == 1).mean(), 0.5 * np.abs(h - p5.numpy()).sum()

    acc_lg, tv_lg = acc_tv(p5.log().view(1, 1, 6).expand(N, 1, 6).contiguous())
    acc_pr, tv_pr = acc_tv(p5.view(1, 1, 6).expand(N, 1, 6).contiguous())
    assert acc_lg > 0.999 and tv_lg < 0.01 and tv_pr > 5 * tv_lg


def test_reference_candidate_row_alignment():
    K, V = 3, 20
    tl = torch.full((1, K + 1, V), -30.0)
    for j in range(K + 1):
        tl[0, j, 10 + j] = 30.0
    acc, bonus, _ = run(tl[:, :K].clone(), tl, torch.tensor([[10, 11, 12]]), seed=1)
    assert acc[0] == K and bonus[0] == 10 + K
    dl7 = tl[:, :K].clone()
    dl7[0, 0, 10] = -30.0
    dl7[0, 0, 3] = 30.0
    acc, bonus, _ = run(dl7, tl, torch.tensor([[3, 11, 12]]), seed=1)
    assert acc[0] == 0 and bonus[0] == 10
