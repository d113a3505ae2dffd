"""The reference-named modules composed the way the engine drives them.

A 2-layer Qwen3-style decoder built only from this package's mirrors of the
reference modules — ``ReplicatedLinear`` quantized in place by
``apply_int8_quant`` (so ``LinearBase._apply`` dispatches to the W8A16 kernel),
``RMSNorm``, ``get_rope``, ``Attention``, ``SiluAndMul``, ``Sampler`` — and
driven only through ``set_context`` with the metadata the engine's
``prepare_decode`` / ``prepare_verify`` produce
(nanovllm/engine/model_runner.py:466-584), captured in a HIP graph on static
buffers padded to a batch bucket with the engine's pad rows (slot -1, context
length 0, block-table row 0, token / position 0: nanovllm/spec_decode/graph_pad.py:33-180,
model_runner.py:1218-1310).

Checks:
  * logits of the real rows within ``2e-2 * max|ref|`` of a float32 torch
    restatement of the same decoder (dequantized weights, softmax attention
    over the gathered pages, bottom-right causal rows for verify);
  * the graph replay bit for bit equal to the eager forward, logits and caches;
  * pad rows write no cache byte; the sampler's greedy tokens are the argmax;
  * two independent decode steps issued on two streams at once (default
    priority, as the reference's concurrent mixed mode does with its second
    stream, nanovllm/engine/mixed_batch.py:99-162) equal the serial run bit for bit.
"""
import math

import pytest
import torch
from torch import nn

from specdec_nanovllm_amd.layers.activation import SiluAndMul
from specdec_nanovllm_amd.layers.attention import Attention
from specdec_nanovllm_amd.layers.layernorm import RMSNorm
from specdec_nanovllm_amd.layers.linear import ReplicatedLinear
from specdec_nanovllm_amd.layers.quant import apply_int8_quant, dequantize_weight
from specdec_nanovllm_amd.layers.rotary_embedding import get_rope
from specdec_nanovllm_amd.layers.sampler import Sampler
from specdec_nanovllm_amd.utils.context import reset_context, set_context

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF = torch.bfloat16
HID, HQ, HKV, D, INTER, VOCAB, NL = 512, 8, 4, 128, 1024, 4096, 2
BS, MAX_POS, THETA, EPS = 256, 8192, 1e6, 1e-6
PAD_SLOT, PAD_ROW_BLOCK, PAD_CTX_LEN, PAD_TOKEN = -1, 0, 0, 0  # graph_pad.py constants


class Layer(nn.Module):
    def __init__(self):
        super().__init__()
        self.input_norm, self.post_norm = RMSNorm(HID, EPS), RMSNorm(HID, EPS)
        self.q_norm, self.k_norm = RMSNorm(D, EPS), RMSNorm(D, EPS)
        self.qkv = ReplicatedLinear(HID, (HQ + 2 * HKV) * D)
        self.o = ReplicatedLinear(HQ * D, HID)
        self.gate_up = ReplicatedLinear(HID, 2 * INTER)
        self.down = ReplicatedLinear(INTER, HID)
        self.attn = Attention(HQ, D, D ** -0.5, HKV)


class TinyQwen3(nn.Module):
    """Qwen3 decoder structure (nanovllm/models/qwen3.py:14-216) on the mirrors."""

    def __init__(self, seed=0):
        super().__init__()
        self.layers = nn.ModuleList(Layer() for _ in range(NL))
        self.final_norm = RMSNorm(HID, EPS)
        self.lm_head = ReplicatedLinear(HID, VOCAB)
        self.rotary = get_rope(D, D, MAX_POS, THETA)
        self.act = SiluAndMul()
        g = torch.Generator().manual_seed(seed)
        self.embed = (torch.randn((VOCAB, HID), generator=g) * 0.5).to(BF)
        for name, p in self.named_parameters():
            if "norm" in name:
                p.data = (1 + 0.1 * torch.randn(p.shape, generator=g)).to(BF)
            else:
                p.data = (torch.randn(p.shape, generator=g) * 0.03).to(BF)
        self.to(DEV)
        self.embed = self.embed.to(DEV)
        self.rotary.to(DEV)
        names = [f"layers.{i}.{m}" for i in range(NL) for m in ("qkv", "o", "gate_up", "down")]
        apply_int8_quant(self, names + ["lm_head"])

    def forward(self, input_ids, positions):
        h = self.embed[input_ids]
        residual = None
        for L in self.layers:
            if residual is None:
                residual, x = h, L.input_norm(h)
            else:
                x, residual = L.input_norm(h, residual)
            q, k, v = L.qkv(x).split([HQ * D, HKV * D, HKV * D], dim=-1)
            q = L.q_norm(q.reshape(-1, HQ, D))
            k = L.k_norm(k.reshape(-1, HKV, D))
            q, k = self.rotary(positions, q, k)
            o = L.attn(q, k, v.reshape(-1, HKV, D))
            h = L.o(o.reshape(-1, HQ * D))
            x, residual = L.post_norm(h, residual)
            h = L.down(self.act(L.gate_up(x)))
        x, _ = self.final_norm(h, residual)
        return self.lm_head(x)

    def set_caches(self, caches):
        for L, (kc, vc) in zip(self.layers, caches):
            L.attn.k_cache, L.attn.v_cache = kc, vc


def new_caches(num_blocks, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return [tuple(torch.randn((num_blocks, BS, HKV, D), generator=g, device=DEV).to(BF)
                  for _ in range(2)) for _ in range(NL)]


def clone_caches(caches):
    return [(k.clone(), v.clone()) for k, v in caches]


# ---------------------------------------------------------------- float32 reference
def ref_forward(model, caches, input_ids, positions, seqs):
    """float32 restatement for the real rows. ``seqs``: per sequence (rows, keys,
    table): its query rows (indices into input_ids), its key count after the
    new rows, its block table; new row j of a sequence sits at position
    keys - len(rows) + j and sees keys [0, keys - len(rows) + j]. Writes the
    new K/V rows into ``caches``."""
    bf = BF

    def lin(x, mod):
        return (x.float() @ dequantize_weight(mod.weight, mod.weight_scale).T).to(bf)

    def rms(x, w):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS)).to(bf) * w

    def add_rms(x, r, w):
        xf = x.float() + r.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + EPS)).to(bf) * w, xf.to(bf)

    cs = model.rotary.cos_sin_cache[positions].reshape(len(positions), -1)
    cos, sin = cs[:, None, :D // 2], cs[:, None, D // 2:]

    def rope(x):
        x1, x2 = x.float().chunk(2, dim=-1)
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(bf)

    h = model.embed[input_ids]
    res = None
    for li, L in enumerate(model.layers):
        if res is None:
            res, x = h, rms(h, L.input_norm.weight)
        else:
            x, res = add_rms(h, res, L.input_norm.weight)
        q, k, v = lin(x, L.qkv).split([HQ * D, HKV * D, HKV * D], dim=-1)
        q = rope(rms(q.reshape(-1, HQ, D), L.q_norm.weight))
        k = rope(rms(k.reshape(-1, HKV, D), L.k_norm.weight))
        v = v.reshape(-1, HKV, D)
        kc, vc = caches[li]
        o = torch.zeros((len(input_ids), HQ, D), dtype=bf, device=DEV)
        for rows, keys, table in seqs:
            n = len(rows)
            for j, r in enumerate(rows):  # the new rows go to their slots first
                p = keys - n + j
                blk, off = int(table[p // BS]), p % BS
                kc[blk, off], vc[blk, off] = k[r], v[r]
            pages = table[:math.ceil(keys / BS)].long()
            K = kc[pages].reshape(-1, HKV, D)[:keys].float()
            V = vc[pages].reshape(-1, HKV, D)[:keys].float()
            for j, r in enumerate(rows):
                vis = keys - n + j + 1
                qq = q[r].float().view(HKV, HQ // HKV, D)
                s = (qq @ K[:vis].permute(1, 2, 0).contiguous()) * (D ** -0.5)
                o[r] = (torch.softmax(s, -1) @ V[:vis].permute(1, 0, 2).contiguous()) \
                    .reshape(HQ, D).to(bf)
        h = lin(o.reshape(-1, HQ * D), L.o)
        x, res = add_rms(h, res, L.post_norm.weight)
        gate, up = lin(x, L.gate_up).chunk(2, dim=-1)
        h = lin(torch.nn.functional.silu(gate.float()).to(bf) * up, L.down)
    x, _ = add_rms(h, res, model.final_norm.weight)
    return x.float() @ dequantize_weight(model.lm_head.weight, model.lm_head.weight_scale).T


# -------------------------------------------------------------------------- helpers
def graph_of(fn):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


def decode_meta(lens, num_blocks, width, seed):
    """prepare_decode for sequences of ``lens`` tokens (the last one new):
    input ids, positions len-1, slots of position len-1, context_lens len,
    block tables over a shuffle of blocks 1.. (block 0 stays for pad rows)."""
    g = torch.Generator().manual_seed(seed)
    perm = (torch.randperm(num_blocks - 1, generator=g) + 1).tolist()
    tables, used = [], 0
    for L in lens:
        n = math.ceil(L / BS)
        tables.append(perm[used:used + n] + [-1] * (width - n))
        used += n
    ids = torch.randint(0, VOCAB, (len(lens),), generator=g)
    pos = torch.tensor([L - 1 for L in lens])
    slots = torch.tensor([tables[b][(L - 1) // BS] * BS + (L - 1) % BS for b, L in enumerate(lens)],
                         dtype=torch.int32)
    return ids, pos, slots, torch.tensor(lens, dtype=torch.int32), \
        torch.tensor(tables, dtype=torch.int32)


# ---------------------------------------------------------------------------- tests
def test_decode_bucket_graph_with_pad_rows():
    torch.manual_seed(0)
    model = TinyQwen3(seed=1)
    nblk, width, bucket = 24, 16, 4
    lens = [300, 1, 777]  # three real sequences, graph bucket 4: one pad row
    B = len(lens)
    print(f"engine compose: decode B={B} in bucket {bucket}", flush=True)
    ids, pos, slots, ctx, bt = decode_meta(lens, nblk, width, seed=2)
    caches = new_caches(nblk, seed=3)
    before = clone_caches(caches)
    model.set_caches(caches)
    # static graph buffers, filled as the engine fills them before a replay
    gv = dict(input_ids=torch.zeros(bucket, dtype=torch.int64, device=DEV),
              positions=torch.zeros(bucket, dtype=torch.int64, device=DEV),
              slot_mapping=torch.zeros(bucket, dtype=torch.int32, device=DEV),
              context_lens=torch.zeros(bucket, dtype=torch.int32, device=DEV),
              block_tables=torch.zeros((bucket, width), dtype=torch.int32, device=DEV))
    gv["input_ids"].fill_(PAD_TOKEN)
    gv["input_ids"][:B] = ids.to(DEV)
    gv["positions"].fill_(PAD_TOKEN)
    gv["positions"][:B] = pos.to(DEV)
    gv["slot_mapping"].fill_(PAD_SLOT)
    gv["slot_mapping"][:B] = slots.to(DEV)
    gv["context_lens"].fill_(PAD_CTX_LEN)
    gv["context_lens"][:B] = ctx.to(DEV)
    gv["block_tables"].fill_(PAD_ROW_BLOCK)
    gv["block_tables"][:B] = bt.to(DEV)
    temps = torch.zeros(bucket, device=DEV)  # greedy
    sampler = Sampler()
    out = {}

    def step():
        set_context(False, slot_mapping=gv["slot_mapping"], context_lens=gv["context_lens"],
                    block_tables=gv["block_tables"])
        out["logits"] = model(gv["input_ids"], gv["positions"])
        out["tokens"] = sampler(out["logits"], temps)
        reset_context()

    step()
    torch.cuda.synchronize()
    eager_logits, eager_tokens = out["logits"].clone(), out["tokens"].clone()
    eager_caches = clone_caches(caches)
    # pad rows wrote nothing: every cache byte outside the real slots is unchanged
    for (k0, v0), (k1, v1) in zip(before, caches):
        for c0, c1 in ((k0, k1), (v0, v1)):
            flat0, flat1 = c0.view(-1, HKV * D).clone(), c1.view(-1, HKV * D).clone()
            flat0[slots.long()] = 0
            flat1[slots.long()] = 0
            assert torch.equal(flat0.view(torch.int16), flat1.view(torch.int16))
    ref = ref_forward(model, clone_caches(before), ids.to(DEV), pos.to(DEV),
                      [([b], lens[b], bt[b]) for b in range(B)])
    got = eager_logits[:B].float()
    assert (got - ref).abs().max().item() <= 2e-2 * ref.abs().max().item()
    assert torch.equal(eager_tokens[:B], eager_logits[:B].float().argmax(-1))
    # the pad row sees no keys: its attention output is zero and nothing breaks
    assert torch.isfinite(eager_logits.float()).all()

    g = graph_of(step)
    for _ in range(3):
        for (kc, vc), (k0, v0) in zip(caches, before):
            kc.copy_(k0)
            vc.copy_(v0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out["logits"].view(torch.int16), eager_logits.view(torch.int16))
        assert torch.equal(out["tokens"], eager_tokens)
        for (k1, v1), (k2, v2) in zip(caches, eager_caches):
            assert torch.equal(k1.view(torch.int16), k2.view(torch.int16))
            assert torch.equal(v1.view(torch.int16), v2.view(torch.int16))


def test_verify_bucket_graph_with_pad_rows():
    model = TinyQwen3(seed=4)
    nblk, width, k = 24, 16, 3
    n = k + 1
    lens = [600, 255]  # confirmed lengths; rows at len-1 .. len+k-1 (the second crosses a page)
    B, bucket = len(lens), 3
    print(f"engine compose: verify B={B}, k={k}, bucket {bucket}", flush=True)
    g = torch.Generator().manual_seed(5)
    perm = (torch.randperm(nblk - 1, generator=g) + 1).tolist()
    tables, used = [], 0
    for L in lens:
        m = math.ceil((L + k) / BS)
        tables.append(perm[used:used + m] + [-1] * (width - m))
        used += m
    bt = torch.tensor(tables, dtype=torch.int32)
    ids = torch.randint(0, VOCAB, (B * n,), generator=g)
    pos = torch.tensor([p for L in lens for p in range(L - 1, L - 1 + n)])
    slots = torch.tensor([tables[b][p // BS] * BS + p % BS
                          for b, L in enumerate(lens) for p in range(L - 1, L - 1 + n)],
                         dtype=torch.int32)
    cu_q = [0]
    cu_k = [0]
    for L in lens:
        cu_q.append(cu_q[-1] + n)
        cu_k.append(cu_k[-1] + L + k)  # model_runner.py:531
    pad = bucket - B  # pad rows: n queries each, 0 keys (pad_cu_seqlens)
    for _ in range(pad):
        cu_q.append(cu_q[-1] + n)
        cu_k.append(cu_k[-1] + PAD_CTX_LEN)
    Q = bucket * n
    gv = dict(input_ids=torch.full((Q,), PAD_TOKEN, dtype=torch.int64, device=DEV),
              positions=torch.full((Q,), PAD_TOKEN, dtype=torch.int64, device=DEV),
              slot_mapping=torch.full((Q,), PAD_SLOT, dtype=torch.int32, device=DEV),
              cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32, device=DEV),
              cu_seqlens_k=torch.tensor(cu_k, dtype=torch.int32, device=DEV),
              block_tables=torch.full((bucket, width), PAD_ROW_BLOCK, dtype=torch.int32,
                                      device=DEV))
    gv["input_ids"][:B * n] = ids.to(DEV)
    gv["positions"][:B * n] = pos.to(DEV)
    gv["slot_mapping"][:B * n] = slots.to(DEV)
    gv["block_tables"][:B] = bt.to(DEV)
    caches = new_caches(nblk, seed=6)
    before = clone_caches(caches)
    model.set_caches(caches)
    out = {}

    def step():
        set_context(True, gv["cu_seqlens_q"], gv["cu_seqlens_k"], n, MAX_POS,
                    gv["slot_mapping"], None, gv["block_tables"], is_spec_verify=True)
        out["logits"] = model(gv["input_ids"], gv["positions"])
        reset_context()

    step()
    torch.cuda.synchronize()
    eager = out["logits"].clone()
    eager_caches = clone_caches(caches)
    ref = ref_forward(model, clone_caches(before), ids.to(DEV), pos.to(DEV),
                      [(list(range(b * n, (b + 1) * n)), lens[b] + k, bt[b]) for b in range(B)])
    got = eager[:B * n].float()
    assert (got - ref).abs().max().item() <= 2e-2 * ref.abs().max().item()
    for (k0, v0), (k1, v1) in zip(before, caches):  # pad rows wrote nothing
        for c0, c1 in ((k0, k1), (v0, v1)):
            flat0, flat1 = c0.view(-1, HKV * D).clone(), c1.view(-1, HKV * D).clone()
            flat0[slots.long()] = 0
            flat1[slots.long()] = 0
            assert torch.equal(flat0.view(torch.int16), flat1.view(torch.int16))
    g_ = graph_of(step)
    for _ in range(3):
        for (kc, vc), (k0, v0) in zip(caches, before):
            kc.copy_(k0)
            vc.copy_(v0)
        torch.cuda.synchronize()
        g_.replay()
        torch.cuda.synchronize()
        assert torch.equal(out["logits"].view(torch.int16), eager.view(torch.int16))
        for (k1, v1), (k2, v2) in zip(caches, eager_caches):
            assert torch.equal(k1.view(torch.int16), k2.view(torch.int16))
            assert torch.equal(v1.view(torch.int16), v2.view(torch.int16))


def test_two_streams_at_once_equal_serial():
    """Two independent decode steps (own caches, own metadata) issued on two
    default-priority streams without a sync between them give the serial run's
    logits bit for bit: calls share no workspace or library state."""
    model = TinyQwen3(seed=7)
    nblk, width = 48, 16
    runs = []
    for r, lens in enumerate(([1500, 33, 2048, 700], [4096, 1, 257, 1024, 3000])):
        ids, pos, slots, ctx, bt = decode_meta(lens, nblk, width, seed=10 + r)
        runs.append(dict(ids=ids.to(DEV), pos=pos.to(DEV), slots=slots.to(DEV),
                         ctx=ctx.to(DEV), bt=bt.to(DEV), caches=new_caches(nblk, seed=20 + r)))
    init = [clone_caches(x["caches"]) for x in runs]

    def forward(x):
        model.set_caches(x["caches"])
        set_context(False, slot_mapping=x["slots"], context_lens=x["ctx"], block_tables=x["bt"])
        y = model(x["ids"], x["pos"])
        reset_context()
        return y

    print("engine compose: two decode steps, serial then on two streams", flush=True)
    serial = [forward(x) for x in runs]
    torch.cuda.synchronize()
    serial = [y.clone() for y in serial]
    serial_caches = [clone_caches(x["caches"]) for x in runs]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for _ in range(3):
        for x, c0 in zip(runs, init):
            for (kc, vc), (k0, v0) in zip(x["caches"], c0):
                kc.copy_(k0)
                vc.copy_(v0)
        cur = torch.cuda.current_stream()
        outs = [None, None]
        for i, (x, s) in enumerate(zip(runs, streams)):
            s.wait_stream(cur)
            with torch.cuda.stream(s):
                outs[i] = forward(x)
        for s in streams:
            cur.wait_stream(s)
        torch.cuda.synchronize()
        for y, want in zip(outs, serial):
            assert torch.equal(y.view(torch.int16), want.view(torch.int16))
        for x, want in zip(runs, serial_caches):
            for (k1, v1), (k2, v2) in zip(x["caches"], want):
                assert torch.equal(k1.view(torch.int16), k2.view(torch.int16))
                assert torch.equal(v1.view(torch.int16), v2.view(torch.int16))
