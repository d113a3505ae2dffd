"""GPU parity of paged decode / verify attention against the numpy oracle.

Tolerance (the stated bound for this path): |o - ref| <= 2e-3 + 1e-2 |ref| elementwise,
ref = float64 attention of the same bf16/fp16 inputs. Covers the C1/C2/C3
configurations, edge lengths around the 32/64/256-token tiles and pages,
padding rows, split counts, page sizes, head-major pages, GQA ratios, fp16,
ragged verify rows, scores whose row maximum rises, spikes or falls along the
keys (the running maximum re-based inside a walk), placement/width invariance,
determinism and HIP-graph replay, plus the reference-mirror entry points and their error behaviour.
"""
import math

import numpy as np
import pytest
import torch

from conftest import assert_close_attn, to_np
from oracle import kvcache as okv
from oracle import paged_attention as opa
from specdec_nanovllm_amd import ops, workloads
from specdec_nanovllm_amd.flash_attn_compat import flash_attn_varlen_func, flash_attn_with_kvcache
from specdec_nanovllm_amd.kernels.paged_decode_attn import paged_decode_attention
from specdec_nanovllm_amd.kernels.paged_decode_attn_cuda import paged_decode_attention_cuda
from specdec_nanovllm_amd.layers.attention import Attention
from specdec_nanovllm_amd.utils.context import reset_context, set_context

pytestmark = pytest.mark.gpu
DEV = "cuda"


def compact(k_cache, v_cache, bt):
    """Copy only the pages a table uses to the host (as float32) and remap the
    table onto them, so the oracle never touches the whole pool."""
    bt = bt.cpu()
    used = sorted(set(int(x) for x in bt.flatten().tolist() if x >= 0))
    remap = {p: i for i, p in enumerate(used)}
    idx = torch.tensor(used if used else [0], dtype=torch.long, device=k_cache.device)
    kc = to_np(k_cache[idx]).astype(np.float32)
    vc = to_np(v_cache[idx]).astype(np.float32)
    bt2 = np.array([[remap.get(int(x), -1) for x in row] for row in bt.tolist()],
                   dtype=np.int64).reshape(bt.shape)
    return kc, vc, bt2


def oracle(q, k_cache, v_cache, bt, lens, scale, cu_q=None):
    kc, vc, bt2 = compact(k_cache, v_cache, bt)
    cu = None if cu_q is None else cu_q.cpu().numpy()
    return opa.paged_attention(to_np(q), kc, vc, bt2, lens.cpu().numpy(), scale, cu)


def random_case(lens, *, hq=32, hkv=8, d=128, bs=256, width=None, dtype=torch.bfloat16,
                seed=0, spare=3):
    lens = torch.tensor(lens, dtype=torch.int32)
    need = sum(max(math.ceil(int(L) / bs), 0) for L in lens)
    nblk = need + spare
    g = torch.Generator().manual_seed(seed)
    w = width or max(max(math.ceil(int(L) / bs) for L in lens), 1)
    bt = workloads.block_tables_for(lens.tolist(), bs, nblk, g, w)[0]
    dg = workloads.device_generator(DEV, seed + 1)
    kc = torch.randn((nblk, bs, hkv, d), generator=dg, device=DEV).to(dtype)
    vc = torch.randn((nblk, bs, hkv, d), generator=dg, device=DEV).to(dtype)
    q = torch.randn((len(lens), hq, d), generator=dg, device=DEV).to(dtype)
    return q, kc, vc, bt, lens


def run_decode(q, kc, vc, bt, lens, **kw):
    return ops.paged_attention(q, kc, vc, bt.to(DEV), q.shape[-1] ** -0.5,
                               context_lens=lens.to(DEV), **kw)


# ----------------------------------------------------- benchmark configurations
@pytest.mark.parametrize("batch", [1, 8, 32])
def test_c2_decode_step(batch):
    case = workloads.decode_case(batch, seed=100 + batch)
    bt, lens, slots = case["tables"][0], case["lens"], case["slots"][0]
    kc, vc = case["k_cache"], case["v_cache"]
    ops.store_kvcache(case["k_new"], case["v_new"], kc, vc, slots.to(DEV))
    out = run_decode(case["q"], kc, vc, bt, lens)
    torch.cuda.synchronize()
    # the new rows are in the cache (read back through the table) ...
    for b in range(batch):
        p = int(lens[b]) - 1
        page = int(bt[b, p // 256])
        assert torch.equal(kc[page, p % 256], case["k_new"][b])
        assert torch.equal(vc[page, p % 256], case["v_new"][b])
    # ... and attention over them matches the oracle
    ref = oracle(case["q"], kc, vc, bt, lens, case["scale"])
    assert_close_attn(to_np(out), ref, what=f"C2 B={batch}")


def test_c1_geometry_bf16():
    # Qwen3-0.6B attention: 16q/8kv/128, B=1, L=1000, 64-block pool, 4 permuted pages
    rng = np.random.default_rng(0)
    bt = torch.from_numpy(rng.permutation(64)[:4].astype(np.int32)).view(1, 4)
    dg = workloads.device_generator(DEV, 1)
    kc = torch.randn((64, 256, 8, 128), generator=dg, device=DEV).to(torch.bfloat16)
    vc = torch.randn((64, 256, 8, 128), generator=dg, device=DEV).to(torch.bfloat16)
    q = torch.randn((1, 16, 128), generator=dg, device=DEV).to(torch.bfloat16)
    lens = torch.tensor([1000], dtype=torch.int32)
    out = run_decode(q, kc, vc, bt, lens)
    assert_close_attn(to_np(out), oracle(q, kc, vc, bt, lens, 128 ** -0.5), what="C1")


def test_c3_verify():
    case = workloads.verify_case(seed=5)
    assert case["crosses_page"], "C3 must include rows that straddle a 256-token page"
    kc, vc = case["k_cache"], case["v_cache"]
    ops.store_kvcache(case["k_new"], case["v_new"], kc, vc, case["slots"].to(DEV))
    out = ops.paged_attention(case["q"], kc, vc, case["table"].to(DEV), case["scale"],
                              cu_seqlens_k=case["cu_k"].to(DEV),
                              cu_seqlens_q=case["cu_q"].to(DEV), max_seqlen_q=case["k"] + 1)
    torch.cuda.synchronize()
    ref = oracle(case["q"], kc, vc, case["table"], case["keys"], case["scale"], case["cu_q"])
    assert_close_attn(to_np(out), ref, what="C3 verify")


# -------------------------------------------------------------------- edge cases
@pytest.mark.parametrize("L", [1, 2, 7, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257,
                               300, 511, 512, 513, 1000, 1024, 2049, 4095, 4096])
def test_edge_lengths(L):
    q, kc, vc, bt, lens = random_case([L, L // 2 + 1], seed=L)
    out = run_decode(q, kc, vc, bt, lens)
    assert_close_attn(to_np(out), oracle(q, kc, vc, bt, lens, 128 ** -0.5), what=f"L={L}")


def test_zero_length_padding_rows():
    # graph padding rows: ctx 0 and block-table row 0 (graph_pad.py PAD_ROW_BLOCK / PAD_CTX_LEN)
    q, kc, vc, bt, lens = random_case([0, 5, 0, 300, 1], seed=9)
    bt[0, :] = 0
    bt[2, :] = -1
    out = run_decode(q, kc, vc, bt, lens)
    got = to_np(out)
    assert np.all(got[0] == 0) and np.all(got[2] == 0)
    assert_close_attn(got, oracle(q, kc, vc, bt, lens, 128 ** -0.5), what="padding rows")


@pytest.mark.parametrize("splits", [1, 2, 3, 5, 16])
def test_split_count_invariance(splits):
    q, kc, vc, bt, lens = random_case([4096, 1700, 256, 3000], seed=21)
    base = run_decode(q, kc, vc, bt, lens)
    out = run_decode(q, kc, vc, bt, lens, num_splits=splits)
    ref = oracle(q, kc, vc, bt, lens, 128 ** -0.5)
    assert_close_attn(to_np(out), ref, what=f"splits={splits}")
    # only the fp32 summation order differs: within one bf16 unit of the default plan
    diff = np.abs(to_np(out) - to_np(base))
    assert np.all(diff <= 2.0 ** -7 * np.abs(to_np(base)) + 1e-5)


@pytest.mark.parametrize("bs", [16, 32, 64, 128, 512])
def test_page_sizes(bs):
    q, kc, vc, bt, lens = random_case([1, 100, 777, 2050], bs=bs, seed=bs)
    out = run_decode(q, kc, vc, bt, lens)
    assert_close_attn(to_np(out), oracle(q, kc, vc, bt, lens, 128 ** -0.5), what=f"bs={bs}")


def test_head_major_pages():
    q, kc, vc, bt, lens = random_case([513, 1500], seed=31)
    kh = kc.transpose(1, 2).contiguous()  # (blocks, Hkv, bs, D)
    vh = vc.transpose(1, 2).contiguous()
    out = ops.paged_attention(q, kh, vh, bt.to(DEV), 128 ** -0.5, context_lens=lens.to(DEV),
                              layout="head_major")
    assert_close_attn(to_np(out), oracle(q, kc, vc, bt, lens, 128 ** -0.5), what="head_major")


@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 8), (32, 4), (8, 8), (64, 8), (32, 1)])
def test_gqa_ratios(hq, hkv):
    q, kc, vc, bt, lens = random_case([700, 2000, 33], hq=hq, hkv=hkv, seed=hq * 100 + hkv)
    out = run_decode(q, kc, vc, bt, lens)
    assert_close_attn(to_np(out), oracle(q, kc, vc, bt, lens, 128 ** -0.5),
                      what=f"hq={hq} hkv={hkv}")


@pytest.mark.parametrize("batch", [33, 40, 64])
def test_mha_decode_between_33_and_64_sequences(batch):
    # one query row per kv head (G = 1): the merge kernel's workgroup is one whole
    # wave, whose 64 lanes each scan one sequence's length; plain and fused store
    rng = np.random.default_rng(batch)
    keys = rng.integers(1, 600, size=batch).tolist()
    q, kc, vc, bt, lens = random_case(keys, hq=8, hkv=8, seed=900 + batch)
    out = run_decode(q, kc, vc, bt, lens)
    assert_close_attn(to_np(out), oracle(q, kc, vc, bt, lens, 128 ** -0.5),
                      what=f"MHA decode B={batch}")
    dg = workloads.device_generator(DEV, 950 + batch)
    knew = torch.randn((batch, 8, 128), generator=dg, device=DEV).to(torch.bfloat16)
    vnew = torch.randn((batch, 8, 128), generator=dg, device=DEV).to(torch.bfloat16)
    slots = workloads.slots_for(bt, [[L - 1] for L in keys], 256).to(DEV)
    o, kc2, vc2 = _fused_vs_separate(q, kc, vc, bt.to(DEV), knew, vnew, slots, 128 ** -0.5,
                                     context_lens=lens.to(DEV))
    assert_close_attn(to_np(o), oracle(q, kc2, vc2, bt, lens, 128 ** -0.5),
                      what=f"MHA fused decode B={batch}")


def test_fp16():
    q, kc, vc, bt, lens = random_case([1234, 4000], dtype=torch.float16, seed=41)
    out = run_decode(q, kc, vc, bt, lens)
    assert_close_attn(to_np(out), oracle(q, kc, vc, bt, lens, 128 ** -0.5), what="fp16")


@pytest.mark.parametrize("hq,hkv", [(32, 8), (16, 8), (12, 3)])
def test_verify_ragged_rows(hq, hkv):
    # rows per sequence 1..7; one sequence has fewer keys than rows. 32/8 puts the
    # two row tiles on two waves; 12/3 (odd kv heads) keeps both tiles on one wave
    nq = [1, 7, 3, 5, 7, 4]
    keys = [900, 2600, 3, 257, 1, 40]
    lens = torch.tensor(keys, dtype=torch.int32)
    g = torch.Generator().manual_seed(77)
    bt = workloads.block_tables_for(keys, 256, 40, g, 12)[0]
    dg = workloads.device_generator(DEV, 78)
    kc = torch.randn((40, 256, hkv, 128), generator=dg, device=DEV).to(torch.bfloat16)
    vc = torch.randn((40, 256, hkv, 128), generator=dg, device=DEV).to(torch.bfloat16)
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(nq)]), dtype=torch.int32)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(keys)]), dtype=torch.int32)
    q = torch.randn((int(cu_q[-1]), hq, 128), generator=dg, device=DEV).to(torch.bfloat16)
    out = ops.paged_attention(q, kc, vc, bt.to(DEV), 128 ** -0.5, cu_seqlens_k=cu_k.to(DEV),
                              cu_seqlens_q=cu_q.to(DEV), max_seqlen_q=max(nq))
    ref = oracle(q, kc, vc, bt, lens, 128 ** -0.5, cu_q)
    assert_close_attn(to_np(out), ref, what="ragged verify")


def _steer_scores(q, kc, bt, lens, profile, bs=256):
    """Add c(t) u to key t of every sequence and 10 u to every query (u a unit
    vector), so each score gains about 10 c(t) / sqrt(D) nats on top of the
    N(0, 1) noise: "rising" grows the row maximum steadily along the walk
    (about 50 log2 units end to end, so the running maximum is re-based many
    times inside one split), "spike" puts one late key about 75 log2 units
    above the rest, "falling" keeps the maximum in the first keys."""
    d = q.shape[-1]
    u = torch.ones(d, device=DEV) / math.sqrt(d)
    for b, n in enumerate(lens.tolist()):
        t = torch.arange(n, dtype=torch.float32)
        if profile == "rising":
            c = 40.0 * t / max(n - 1, 1)
        elif profile == "spike":
            c = torch.where(t == max(n - 5, 0), 60.0, 0.0)
        else:
            c = 40.0 * (1.0 - t / max(n - 1, 1))
        ti = torch.arange(n)
        pages = bt[b, ti // bs].long().to(DEV)
        offs = (ti % bs).to(DEV)
        kc[pages, offs] = (kc[pages, offs].float() + c.to(DEV)[:, None, None] * u).to(kc.dtype)
    return (q.float() + 10.0 * u).to(q.dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("profile", ["rising", "spike", "falling"])
def test_running_maximum_moves_along_the_walk(profile, dtype):
    q, kc, vc, bt, lens = random_case([3000, 1500, 77, 300], dtype=dtype, seed=23)
    q = _steer_scores(q, kc, bt, lens, profile)
    ref = oracle(q, kc, vc, bt, lens, 128 ** -0.5)
    for splits in (None, 1, 5):
        kw = {} if splits is None else {"num_splits": splits}
        out = run_decode(q, kc, vc, bt, lens, **kw)
        assert_close_attn(to_np(out), ref, what=f"{profile} splits={splits}")


@pytest.mark.parametrize("profile", ["rising", "spike"])
def test_running_maximum_moves_verify_rows(profile):
    nq = [6, 1, 4]
    keys = [2600, 700, 260]
    lens = torch.tensor(keys, dtype=torch.int32)
    g = torch.Generator().manual_seed(79)
    bt = workloads.block_tables_for(keys, 256, 20, g, 12)[0]
    dg = workloads.device_generator(DEV, 80)
    kc = torch.randn((20, 256, 8, 128), generator=dg, device=DEV).to(torch.bfloat16)
    vc = torch.randn((20, 256, 8, 128), generator=dg, device=DEV).to(torch.bfloat16)
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(nq)]), dtype=torch.int32)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(keys)]), dtype=torch.int32)
    q = torch.randn((int(cu_q[-1]), 32, 128), generator=dg, device=DEV).to(torch.bfloat16)
    q = _steer_scores(q, kc, bt, lens, profile)
    out = ops.paged_attention(q, kc, vc, bt.to(DEV), 128 ** -0.5, cu_seqlens_k=cu_k.to(DEV),
                              cu_seqlens_q=cu_q.to(DEV), max_seqlen_q=max(nq))
    ref = oracle(q, kc, vc, bt, lens, 128 ** -0.5, cu_q)
    assert_close_attn(to_np(out), ref, what=f"{profile} verify")


def test_placement_and_width_invariance_bitwise():
    # same sequence data at different pages, with a wider -1 padded table
    q, kc, vc, bt, lens = random_case([1500, 700], seed=51, spare=20)
    out1 = run_decode(q, kc, vc, bt, lens)
    used = sorted(set(int(x) for x in bt.flatten().tolist() if x >= 0))
    free = [p for p in range(kc.shape[0]) if p not in used]
    move = {p: free[i] for i, p in enumerate(used)}
    kc2, vc2 = kc.clone(), vc.clone()
    for p, n in move.items():
        kc2[n] = kc[p]
        vc2[n] = vc[p]
    bt2 = torch.full((bt.shape[0], bt.shape[1] + 9), -1, dtype=torch.int32)
    for b in range(bt.shape[0]):
        for j in range(bt.shape[1]):
            if int(bt[b, j]) >= 0:
                bt2[b, j] = move[int(bt[b, j])]
    out2 = run_decode(q, kc2, vc2, bt2, lens)
    assert torch.equal(out1, out2)


def test_repeat_is_bitwise_deterministic():
    # 100 eager repeats of decode at the C2 B = 32 shape and of C3 verify with
    # its fused store (every repeat writes the same rows): bitwise equal outputs
    case = workloads.decode_case(32, seed=61)
    bt, lens = case["tables"][0].to(DEV), case["lens"].to(DEV)
    a = ops.paged_attention(case["q"], case["k_cache"], case["v_cache"], bt, case["scale"],
                            context_lens=lens)
    out = torch.empty_like(a)
    for i in range(100):
        ops.paged_attention(case["q"], case["k_cache"], case["v_cache"], bt, case["scale"],
                            context_lens=lens, out=out)
        assert torch.equal(a, out), f"decode repeat {i}"
    del case
    v = workloads.verify_case(seed=61)
    kw = dict(cu_seqlens_k=v["cu_k"].to(DEV), cu_seqlens_q=v["cu_q"].to(DEV),
              max_seqlen_q=v["k"] + 1, key=v["k_new"], value=v["v_new"],
              slot_mapping=v["slots"].to(DEV))
    vt = v["table"].to(DEV)
    a = ops.paged_attention(v["q"], v["k_cache"], v["v_cache"], vt, v["scale"], **kw)
    out = torch.empty_like(a)
    for i in range(100):
        ops.paged_attention(v["q"], v["k_cache"], v["v_cache"], vt, v["scale"], out=out, **kw)
        assert torch.equal(a, out), f"verify repeat {i}"


def test_graph_replays_are_bitwise_deterministic():
    # 100 replays of one HIP graph holding the C3 verify call with its fused
    # store, with eager work and a synchronisation between replays: every
    # replay equals the eager call bit for bit
    v = workloads.verify_case(seed=62)
    kw = dict(cu_seqlens_k=v["cu_k"].to(DEV), cu_seqlens_q=v["cu_q"].to(DEV),
              max_seqlen_q=v["k"] + 1, key=v["k_new"], value=v["v_new"],
              slot_mapping=v["slots"].to(DEV))
    vt = v["table"].to(DEV)
    out = torch.empty_like(v["q"])
    eager = ops.paged_attention(v["q"], v["k_cache"], v["v_cache"], vt, v["scale"], **kw)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.paged_attention(v["q"], v["k_cache"], v["v_cache"], vt, v["scale"], out=out, **kw)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.paged_attention(v["q"], v["k_cache"], v["v_cache"], vt, v["scale"], out=out, **kw)
    for i in range(100):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"


def test_hip_graph_replay_matches_eager():
    case = workloads.decode_case(8, seed=71, num_blocks=256, sets=2)
    kc, vc = case["k_cache"], case["v_cache"]
    q = case["q"].clone()
    knew, vnew = case["k_new"].clone(), case["v_new"].clone()
    bt = case["tables"][0].to(DEV)
    lens = case["lens"].to(DEV)
    slots = case["slots"][0].to(DEV)
    out = torch.empty_like(q)
    # warm up on a side stream, then capture store + attention
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.store_kvcache(knew, vnew, kc, vc, slots)
        ops.paged_attention(q, kc, vc, bt, case["scale"], context_lens=lens, out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ops.store_kvcache(knew, vnew, kc, vc, slots)
        ops.paged_attention(q, kc, vc, bt, case["scale"], context_lens=lens, out=out)
    for rep, tbl in enumerate([case["tables"][0], case["tables"][1], case["tables"][0]]):
        dg = workloads.device_generator(DEV, 1000 + rep)
        q.copy_(torch.randn(q.shape, generator=dg, device=DEV).to(q.dtype))
        knew.copy_(torch.randn(knew.shape, generator=dg, device=DEV).to(knew.dtype))
        bt.copy_(tbl.to(DEV))
        slots.copy_(workloads.slots_for(tbl, [[int(L) - 1] for L in case["lens"]], 256).to(DEV))
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        torch.cuda.synchronize()
        eager = ops.paged_attention(q, kc, vc, bt, case["scale"], context_lens=lens)
        torch.cuda.synchronize()
        assert torch.equal(got, eager), f"replay {rep} differs from eager"
        assert_close_attn(to_np(got), oracle(q, kc, vc, tbl, case["lens"], case["scale"]),
                          what=f"graph replay {rep}")


# ------------------------------------------------------------------ fused store
def _fused_vs_separate(q, kc, vc, bt, knew, vnew, slots, scale, **kw):
    kc1, vc1, kc2, vc2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    ops.store_kvcache(knew, vnew, kc1, vc1, slots)
    o1 = ops.paged_attention(q, kc1, vc1, bt, scale, **kw)
    o2 = ops.paged_attention(q, kc2, vc2, bt, scale, key=knew, value=vnew, slot_mapping=slots,
                             **kw)
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2), "fused store differs"
    # the fused launch adds the new keys in fp32 in its merge, the separate one
    # takes them through the main loop: equal up to rounding, both near float64
    assert_close_attn(to_np(o2), to_np(o1), what="fused vs store-then-attend")
    return o2, kc2, vc2


@pytest.mark.parametrize("batch", [1, 8, 32])
def test_fused_store_decode_is_store_then_attend(batch):
    case = workloads.decode_case(batch, seed=300 + batch, num_blocks=512)
    bt, lens, slots = case["tables"][0].to(DEV), case["lens"], case["slots"][0].to(DEV)
    o, kc, vc = _fused_vs_separate(case["q"], case["k_cache"], case["v_cache"], bt,
                                   case["k_new"], case["v_new"], slots, case["scale"],
                                   context_lens=lens.to(DEV))
    assert_close_attn(to_np(o), oracle(case["q"], kc, vc, case["tables"][0], lens, case["scale"]),
                      what=f"fused decode B={batch}")


def test_fused_store_verify_is_store_then_attend():
    case = workloads.verify_case(seed=5, num_blocks=256)
    o, kc, vc = _fused_vs_separate(case["q"], case["k_cache"], case["v_cache"],
                                   case["table"].to(DEV), case["k_new"], case["v_new"],
                                   case["slots"].to(DEV), case["scale"],
                                   cu_seqlens_k=case["cu_k"].to(DEV),
                                   cu_seqlens_q=case["cu_q"].to(DEV),
                                   max_seqlen_q=case["k"] + 1)
    ref = oracle(case["q"], kc, vc, case["table"], case["keys"], case["scale"], case["cu_q"])
    assert_close_attn(to_np(o), ref, what="fused verify")


def test_fused_store_pad_slots_and_small_pages():
    # slot -1 rows (graph padding / rows not to write) keep the cache row as the key;
    # 16-token pages take the per-lane page lookup path
    for bs in (256, 16):
        q, kc, vc, bt, lens = random_case([300, 1, 513, 40], bs=bs, seed=400 + bs)
        g = torch.Generator().manual_seed(bs)
        knew = torch.randn((4, 8, 128), generator=g).to(torch.bfloat16).to(DEV)
        vnew = torch.randn((4, 8, 128), generator=g).to(torch.bfloat16).to(DEV)
        slots = workloads.slots_for(bt, [[int(L) - 1] for L in lens], bs)
        slots[1] = -1
        slots[3] = -1
        o, kc2, vc2 = _fused_vs_separate(q, kc, vc, bt.to(DEV), knew, vnew, slots.to(DEV),
                                         128 ** -0.5, context_lens=lens.to(DEV))
        assert_close_attn(to_np(o), oracle(q, kc2, vc2, bt, lens, 128 ** -0.5),
                          what=f"pad slots bs={bs}")


@pytest.mark.parametrize("bs", [256, 16])
def test_fused_store_verify_short_sequences_and_pad_slots(bs):
    # 7 new rows per sequence: one sequence has no cached key (all its keys are
    # new), one has two; two rows of the long one are not stored (slot -1: the
    # cache row stays their key)
    n = 7
    keys = torch.tensor([7, 9, 600], dtype=torch.int32)
    _, kc, vc, bt, _ = random_case(keys.tolist(), bs=bs, seed=500 + bs)
    g = torch.Generator().manual_seed(bs + 1)
    N = n * len(keys)
    q = torch.randn((N, 32, 128), generator=g).to(torch.bfloat16).to(DEV)
    knew = torch.randn((N, 8, 128), generator=g).to(torch.bfloat16).to(DEV)
    vnew = torch.randn((N, 8, 128), generator=g).to(torch.bfloat16).to(DEV)
    slots = workloads.slots_for(bt, [list(range(int(L) - n, int(L))) for L in keys], bs)
    slots[2 * n + 3] = -1
    slots[2 * n + 6] = -1
    cu_q = torch.arange(0, N + 1, n, dtype=torch.int32)
    cu_k = torch.zeros(len(keys) + 1, dtype=torch.int32)
    cu_k[1:] = torch.cumsum(keys, 0)
    o, kc2, vc2 = _fused_vs_separate(q, kc, vc, bt.to(DEV), knew, vnew, slots.to(DEV),
                                     128 ** -0.5, cu_seqlens_k=cu_k.to(DEV),
                                     cu_seqlens_q=cu_q.to(DEV), max_seqlen_q=n)
    assert_close_attn(to_np(o), oracle(q, kc2, vc2, bt, keys, 128 ** -0.5, cu_q),
                      what=f"fused verify short bs={bs}")


def test_fused_store_more_rows_than_combine_threads():
    # rows outside every sequence's query range (engine pad tokens with real
    # slots) are still stored; 600 rows x 8 heads x 32 pieces is many times the
    # combine grid, so the grid-stride copy loop runs
    q, kc, vc, bt, lens = random_case([300, 700], hq=8, hkv=8, bs=16, seed=91, spare=40)
    N = 600
    g = torch.Generator().manual_seed(91)
    q = torch.randn((N, 8, 128), generator=g).to(torch.bfloat16).to(DEV)
    knew = torch.randn((N, 8, 128), generator=g).to(torch.bfloat16).to(DEV)
    vnew = torch.randn((N, 8, 128), generator=g).to(torch.bfloat16).to(DEV)
    slots = workloads.slots_for(bt, [[int(L) - 1] for L in lens], 16).tolist()
    unused = sorted(set(range(kc.shape[0])) - set(int(x) for x in bt.flatten().tolist()))
    slots += [blk * 16 + o for blk in unused for o in range(16)][:N - 2]
    slots = torch.tensor(slots, dtype=torch.int32, device=DEV)
    cu_q = torch.tensor([0, 1, 2], dtype=torch.int32, device=DEV)
    cu_k = torch.tensor([0, 300, 1000], dtype=torch.int32, device=DEV)
    kc1, vc1, kc2, vc2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    o1, o2 = torch.zeros_like(q), torch.zeros_like(q)
    kw = dict(cu_seqlens_k=cu_k, cu_seqlens_q=cu_q, max_seqlen_q=1)
    ops.store_kvcache(knew, vnew, kc1, vc1, slots)
    ops.paged_attention(q, kc1, vc1, bt.to(DEV), 128 ** -0.5, out=o1, **kw)
    ops.paged_attention(q, kc2, vc2, bt.to(DEV), 128 ** -0.5, out=o2, key=knew, value=vnew,
                        slot_mapping=slots, **kw)
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    assert_close_attn(to_np(o2), to_np(o1), what="fused, many rows")


def test_fused_store_without_sequences_only_stores():
    kc = torch.zeros((4, 16, 8, 128), dtype=torch.bfloat16, device=DEV)
    vc = torch.zeros_like(kc)
    g = torch.Generator().manual_seed(5)
    knew = torch.randn((5, 8, 128), generator=g).to(torch.bfloat16).to(DEV)
    vnew = torch.randn((5, 8, 128), generator=g).to(torch.bfloat16).to(DEV)
    slots = torch.tensor([3, -1, 17, 63, 40], dtype=torch.int32, device=DEV)
    kc1, vc1 = kc.clone(), vc.clone()
    ops.store_kvcache(knew, vnew, kc1, vc1, slots)
    ops.paged_attention(knew.clone(), kc, vc, torch.zeros((0, 1), dtype=torch.int32, device=DEV),
                        128 ** -0.5, cu_seqlens_k=torch.zeros(1, dtype=torch.int32, device=DEV),
                        cu_seqlens_q=torch.zeros(1, dtype=torch.int32, device=DEV),
                        max_seqlen_q=1, key=knew, value=vnew, slot_mapping=slots)
    torch.cuda.synchronize()
    assert torch.equal(kc, kc1) and torch.equal(vc, vc1) and kc.abs().sum() > 0


def test_fused_store_graph_replay():
    case = workloads.decode_case(8, seed=77, num_blocks=256)
    bt, lens, slots = case["tables"][0].to(DEV), case["lens"].to(DEV), case["slots"][0].to(DEV)
    kc, vc, q = case["k_cache"], case["v_cache"], case["q"]
    knew, vnew = case["k_new"], case["v_new"]
    out = torch.empty_like(q)

    def step():
        ops.paged_attention(q, kc, vc, bt, case["scale"], context_lens=lens, out=out,
                            key=knew, value=vnew, slot_mapping=slots)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    torch.cuda.synchronize()
    eager = out.clone()
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


# ------------------------------------------------------------- mirror entry points
def test_mirror_entry_points_agree():
    q, kc, vc, bt, lens = random_case([1000, 2500, 1], seed=81)
    btd, ld = bt.to(DEV), lens.to(DEV)
    base = run_decode(q, kc, vc, bt, lens)
    for version in (1, 2, 3):
        assert torch.equal(paged_decode_attention(q, kc, vc, btd, ld, 128 ** -0.5,
                                                  version=version), base)
    assert torch.equal(paged_decode_attention_cuda(q, kc, vc, btd, ld, 128 ** -0.5), base)
    fa = flash_attn_with_kvcache(q.unsqueeze(1), kc, vc, cache_seqlens=ld, block_table=btd,
                                 softmax_scale=128 ** -0.5, causal=True)
    assert fa.shape == (3, 1, 32, 128) and torch.equal(fa[:, 0], base)
    # Attention module, decode branch (store then attend)
    attn = Attention(32, 128, 128 ** -0.5, 8)
    attn.k_cache, attn.v_cache = kc, vc
    kc0 = kc.clone()
    knew = torch.randn((3, 8, 128), device=DEV).to(torch.bfloat16)
    slots = torch.full((3,), -1, dtype=torch.int32, device=DEV)  # no write: compare to base
    set_context(False, slot_mapping=slots, context_lens=ld, block_tables=btd)
    try:
        o = attn(q, knew, knew)
    finally:
        reset_context()
    # the fused store scores the last key in the merge launch: equal up to rounding
    assert o.shape == (3, 1, 32, 128)
    assert_close_attn(to_np(o[:, 0]), to_np(base), what="Attention decode (fused store)")
    assert torch.equal(kc, kc0)


def test_attention_module_verify_branch():
    case = workloads.verify_case(seed=91, num_blocks=256)
    kc, vc = case["k_cache"], case["v_cache"]
    attn = Attention(32, 128, case["scale"], 8)
    attn.k_cache, attn.v_cache = kc, vc
    set_context(True, case["cu_q"].to(DEV), case["cu_k"].to(DEV), case["k"] + 1,
                int(case["keys"].max()), case["slots"].to(DEV), None, case["table"].to(DEV),
                is_spec_verify=True)
    try:
        o = attn(case["q"], case["k_new"], case["v_new"])
    finally:
        reset_context()
    torch.cuda.synchronize()
    ref = oracle(case["q"], kc, vc, case["table"], case["keys"], case["scale"], case["cu_q"])
    assert_close_attn(to_np(o), ref, what="Attention verify")
    o2 = flash_attn_varlen_func(case["q"], kc, vc, case["cu_q"].to(DEV), case["cu_k"].to(DEV),
                                case["k"] + 1, int(case["keys"].max()),
                                softmax_scale=case["scale"], causal=True,
                                block_table=case["table"].to(DEV))
    assert_close_attn(to_np(o2), ref, what="varlen on the stored cache")


def test_errors_match_reference_kinds():
    q, kc, vc, bt, lens = random_case([10], seed=3)
    btd, ld = bt.to(DEV), lens.to(DEV)
    with pytest.raises(ValueError):  # paged_decode_attn.py:467-468
        paged_decode_attention(q, kc, vc, btd, ld, 0.1, version=4)
    with pytest.raises(AssertionError):  # GQA divisibility, paged_decode_attn.py:384
        paged_decode_attention(q[:, :30], kc, vc, btd, ld, 0.1)
    with pytest.raises(RuntimeError):  # unsupported head_dim (TORCH_CHECK kind)
        q64, k64, v64, bt64, l64 = random_case([10], d=64, seed=4)
        run_decode(q64, k64, v64, bt64, l64)
    with pytest.raises(RuntimeError):  # CPU tensors: no fallback
        ops.paged_attention(q.cpu(), kc.cpu(), vc.cpu(), bt, 0.1, context_lens=lens)


# -------------------------------------------------------------- measurement twins
@pytest.mark.parametrize("bs", [256, 16])
def test_twins_main_then_combine_is_the_full_call(bs):
    """The main-only and combine-only twins over one workspace give the full
    call's output bit for bit; the read-only floor leaves ``out`` untouched."""
    q, kc, vc, bt, lens = random_case([700, 1, 2049, 4096, 0, 333, 1800, 64], bs=bs, seed=21)
    print(f"twins: decode 8 seqs, page {bs}", flush=True)
    full = run_decode(q, kc, vc, bt, lens)
    nbytes = ops.paged_attention_workspace_bytes(len(lens), 1, q.shape[1], kc.shape[2],
                                                 bt.shape[1] * bs, device=DEV)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    out = torch.full_like(q, float("nan"))
    run_decode(q, kc, vc, bt, lens, twin="main", workspace=ws, out=out)
    run_decode(q, kc, vc, bt, lens, twin="combine", workspace=ws, out=out)
    assert torch.equal(out.view(torch.int16), full.view(torch.int16))
    untouched = torch.full_like(q, float("nan"))
    run_decode(q, kc, vc, bt, lens, twin="floor", workspace=ws, out=untouched)
    torch.cuda.synchronize()
    assert bool(torch.isnan(untouched.float()).all())


def test_twins_verify_rows():
    c = workloads.verify_case(8, 6, seed=5)
    print(f"twins: C3 verify seed {c['seed_used']}", flush=True)
    kw = dict(cu_seqlens_k=c["cu_k"].to(DEV), cu_seqlens_q=c["cu_q"].to(DEV), max_seqlen_q=7)
    bt = c["table"].to(DEV)
    full = ops.paged_attention(c["q"], c["k_cache"], c["v_cache"], bt, c["scale"], **kw)
    nbytes = ops.paged_attention_workspace_bytes(8, 7, 32, 8, bt.shape[1] * 256, device=DEV)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    out = torch.full_like(c["q"], float("nan"))
    for twin in ("main", "combine"):
        ops.paged_attention(c["q"], c["k_cache"], c["v_cache"], bt, c["scale"], twin=twin,
                            workspace=ws, out=out, **kw)
    assert torch.equal(out.view(torch.int16), full.view(torch.int16))
    ops.paged_attention(c["q"], c["k_cache"], c["v_cache"], bt, c["scale"], twin="floor",
                        workspace=ws, out=full, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), full.view(torch.int16))  # floor wrote nothing
