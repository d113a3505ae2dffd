"""Pins of oracle/decoder_ops.verify_batch (CPU): the reference's own checks of
rejection sampling (tests/test_spec_decode.py:78-323 of the reference —
cases A/B/C, losslessness by TV convergence, logits-not-probabilities,
candidate/row alignment), restated on the same synthetic inputs, plus a
chi-square test that the first emitted token follows the target law for a
real (not point-mass) draft distribution.
"""
import numpy as np
import torch

from oracle import decoder_ops as od


def softmax(x):
    e = np.exp(x - x.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def test_case_a_equal_distributions_accept_all():
    g = torch.Generator().manual_seed(0)
    dl = torch.randn((1, 3, 20), generator=g).numpy()
    tl = np.concatenate([dl, torch.randn((1, 1, 20), generator=g).numpy()], axis=1)
    probs = softmax(dl[0])
    rng = np.random.default_rng(0)
    toks = np.array([[rng.choice(20, p=probs[j] / probs[j].sum()) for j in range(3)]])
    acc, bonus, mask = od.verify_batch(dl, tl, toks, seed=11)
    assert acc.tolist() == [3] and mask.all()


def test_case_b_sharp_target_rejects_early():
    dl = np.zeros((1, 3, 20), np.float32)
    dl[:, 0, 7] = 50.0
    tl = np.full((1, 4, 20), -50.0, np.float32)
    tl[:, :, 7] = 50.0
    for seed in range(20):
        acc, _, _ = od.verify_batch(dl, tl, np.zeros((1, 3), np.int64), seed=seed)
        assert acc[0] <= 1


def test_case_c_point_mass_rejected_bonus_on_target_mode():
    N, V = 4000, 20
    pc = np.full(V, 1e-6, np.float32)
    pc[5] = 1.0
    tl = np.broadcast_to(np.log(pc)[None, None, :], (N, 2, V)).copy()
    dq = np.zeros((N, 1, V), np.float32)
    dq[:, 0, 3] = 1.0
    acc, bonus, _ = od.verify_batch(dq, tl, np.full((N, 1), 3), point_mass=True, seed=3)
    assert (acc == 0).all()
    assert np.bincount(bonus, minlength=V).argmax() == 5


def _tv_point_mass(N, seed):
    probs = np.array([0.5, 0.2, 0.15, 0.05, 0.05, 0.05], np.float32)
    rng = np.random.default_rng(seed)
    d = rng.choice(6, size=N, p=probs)
    dq = np.zeros((N, 1, 6), np.float32)
    dq[np.arange(N), 0, d] = 1.0
    tl = np.broadcast_to(np.log(probs)[None, None, :], (N, 2, 6)).copy()
    acc, bonus, _ = od.verify_batch(dq, tl, d[:, None], point_mass=True, seed=seed, offset=seed)
    final = np.where(acc == 1, d, bonus)
    h = np.bincount(final, minlength=6) / N
    return 0.5 * np.abs(h - probs).sum()


def test_lossless_tv_converges():
    small = np.mean([_tv_point_mass(40_000, s) for s in range(5)])
    large = np.mean([_tv_point_mass(400_000, s) for s in range(3)])
    assert small / large > 2.0 and large < 0.004, (small, large)


def test_draft_side_must_be_logits():
    p5 = np.array([0.5, 0.2, 0.15, 0.05, 0.05, 0.05], np.float32)
    N = 200_000
    cand = np.random.default_rng(0).choice(6, size=(N, 1), p=p5)
    tgt = np.broadcast_to(np.log(p5)[None, None, :], (N, 2, 6)).copy()

    def acc_tv(draft_side):
        acc, bonus, _ = od.verify_batch(draft_side, tgt, cand, seed=9)
        final = np.where(acc == 1, cand[:, 0], bonus)
        h = np.bincount(final, minlength=6) / N
        return (acc == 1).mean(), 0.5 * np.abs(h - p5).sum()

    acc_lg, tv_lg = acc_tv(np.broadcast_to(np.log(p5)[None, None, :], (N, 1, 6)).copy())
    acc_pr, tv_pr = acc_tv(np.broadcast_to(p5[None, None, :], (N, 1, 6)).copy())
    assert acc_lg > 0.999 and tv_lg < 0.01
    assert tv_pr > 5 * tv_lg


def test_candidate_row_alignment():
    K, V = 3, 20
    tl = np.full((1, K + 1, V), -30.0, np.float32)
    for j in range(K + 1):
        tl[0, j, 10 + j] = 30.0
    dl = tl[:, :K].copy()
    acc, bonus, _ = od.verify_batch(dl, tl, np.array([[10, 11, 12]]), seed=1)
    assert acc[0] == K and bonus[0] == 10 + K
    dl7 = dl.copy()
    dl7[0, 0, 10] = -30.0
    dl7[0, 0, 3] = 30.0
    acc, bonus, _ = od.verify_batch(dl7, tl, np.array([[3, 11, 12]]), seed=1)
    assert acc[0] == 0 and bonus[0] == 10


def test_first_token_follows_target_law_chi_square():
    # a real draft distribution q != p: the first emitted token (the candidate
    # if accepted, else the bonus) must still be distributed as p
    N, V = 200_000, 7
    rng = np.random.default_rng(4)
    tl_row = rng.standard_normal(V).astype(np.float32)
    dl_row = (tl_row + rng.standard_normal(V)).astype(np.float32)
    p, q = softmax(tl_row), softmax(dl_row)
    cand = rng.choice(V, size=(N, 1), p=q / q.sum())
    dl = np.broadcast_to(dl_row[None, None, :], (N, 1, V)).copy()
    tl = np.broadcast_to(tl_row[None, None, :], (N, 2, V)).copy()
    acc, bonus, _ = od.verify_batch(dl, tl, cand, seed=21)
    final = np.where(acc == 1, cand[:, 0], bonus)
    counts = np.bincount(final, minlength=V)
    chi2 = (((counts - N * p) ** 2) / (N * p)).sum()
    assert chi2 < 22.5  # 6 degrees of freedom, p ~ 1e-3
    # and the acceptance rate is sum_x min(p, q)
    assert abs((acc == 1).mean() - np.minimum(p, q).sum()) < 0.005
