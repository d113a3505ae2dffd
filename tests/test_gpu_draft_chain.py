"""GPU parity of the C5 draft chain (draft_chain.DraftChain) against a plain
torch float32 restatement of the same decoder step: dequantized weights
(``q * scale``), softmax attention over the gathered paged rows, the same bf16
rounding points between ops. Floating point: logits must agree to
``max|got - ref| <= 2e-2 * max|ref|`` (bf16 activations between ops), and the
HIP-graph replay of the chain must reproduce the eager chain bit for bit.
Both forms of the step are covered: eager-torch neighbours and this library's
fused neighbour kernels — on a small stack (every step checked), and at the C5
configuration itself (28 layers, hidden 1024, 16 q / 8 kv heads, intermediate
3072, vocab 151936, a 2048-token context prefilled from uniform random token
ids, k = 6 steps, batch 1 and 16: the first and the last step checked against
the reference, every drafted token against the argmax of its logits, the graph
replay bitwise).
"""
import pytest
import torch

from specdec_nanovllm_amd.draft_chain import DraftChain
from specdec_nanovllm_amd.layers.quant import dequantize_weight

pytestmark = pytest.mark.gpu

SMALL = dict(ctx_len=300, k=3, layers=2, hidden=256, heads=4, kv_heads=2, head_dim=128,
             inter=512, vocab=1000, seed=3)


def ref_step(ch: DraftChain, kv: torch.Tensor, tokens: torch.Tensor, s: int) -> torch.Tensor:
    """Float32 torch forward of draft step s (writes the new K/V rows into kv)."""
    B, Hq, Hkv, D, bs = ch.B, ch.Hq, ch.Hkv, ch.D, ch.bs
    bf = torch.bfloat16

    def lin(x, qw):
        return (x.float() @ dequantize_weight(*qw).T).to(bf)

    def rms(x, w):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + ch.eps)).to(bf) * w

    def add_rms(x, r, w):
        xf = x.float() + r.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + ch.eps)).to(bf) * w, xf.to(bf)

    def rope(x, pos):
        c, sn = ch.cos[pos][:, None, :], ch.sin[pos][:, None, :]
        x1, x2 = x.float().chunk(2, dim=-1)
        return torch.cat((x1 * c - x2 * sn, x2 * c + x1 * sn), dim=-1).to(bf)

    pos = ch.positions[s]
    h = ch.embed[tokens]
    res = None
    for li, lw in enumerate(ch.layers):
        if res is None:
            res, x = h, rms(h, lw["in_norm"])
        else:
            x, res = add_rms(h, res, lw["in_norm"])
        qkv = lin(x, lw["qkv"])
        q, k, v = qkv.split([Hq * D, Hkv * D, Hkv * D], dim=-1)
        q = rope(rms(q.reshape(B, Hq, D), lw["q_norm"]), pos)
        k = rope(rms(k.reshape(B, Hkv, D), lw["k_norm"]), pos)
        v = v.reshape(B, Hkv, D)
        flat_k = kv[0, li].view(-1, Hkv, D)
        flat_v = kv[1, li].view(-1, Hkv, D)
        flat_k[ch.slots[s].long()] = k
        flat_v[ch.slots[s].long()] = v
        o = torch.empty((B, Hq, D), dtype=bf, device=q.device)
        for b in range(B):
            L = int(ch.ctx[s, b])
            pages = ch.block_table[b, :(L + bs - 1) // bs].long()
            K = kv[0, li][pages].reshape(-1, Hkv, D)[:L].float()
            V = kv[1, li][pages].reshape(-1, Hkv, D)[:L].float()
            G = Hq // Hkv
            qq = q[b].float().view(Hkv, G, D)
            att = torch.softmax((qq @ K.permute(1, 2, 0).contiguous()) * ch.scale, dim=-1)
            o[b] = (att @ V.permute(1, 0, 2).contiguous()).reshape(Hq, D).to(bf)
        h = lin(o.reshape(B, Hq * D), lw["o"])
        x, res = add_rms(h, res, lw["post_norm"])
        gu = lin(x, lw["gate_up"])
        gate, up = gu.chunk(2, dim=-1)
        h = lin(torch.nn.functional.silu(gate) * up, lw["down"])
    x, _ = add_rms(h, res, ch.final_norm)
    return (x.float() @ dequantize_weight(*ch.lm_head).T)


@pytest.mark.parametrize("fused", [False, True])
def test_draft_chain_matches_float32_reference(fused):
    ch = DraftChain(3, fused=fused, **SMALL)
    kv_ref = ch.kv.clone()
    logits = []
    for s in range(ch.k):
        logits.append(ch.step(s).float())
    tokens = ch.tokens.clone()
    torch.cuda.synchronize()
    for s in range(ch.k):
        ref = ref_step(ch, kv_ref, ch.tokens[s], s)
        err = (logits[s] - ref).abs().max().item()
        assert err <= 2e-2 * ref.abs().max().item(), f"step {s}: max err {err:.4g}"
        # the drafted token is the argmax of the step's own logits
        assert torch.equal(tokens[s + 1], logits[s].argmax(dim=-1))
    # the new K/V rows landed where the reference put them
    assert torch.equal(ch.kv, kv_ref) or (ch.kv.float() - kv_ref.float()).abs().max() < 5e-2


@pytest.mark.parametrize("fused", [False, True])
def test_draft_chain_graph_replay_is_bitwise_eager(fused):
    ch = DraftChain(2, fused=fused, **SMALL)
    kv0, tok0 = ch.kv.clone(), ch.tokens.clone()
    ch.chain()
    torch.cuda.synchronize()
    eager = ch.tokens.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ch.kv.copy_(kv0)
        ch.tokens.copy_(tok0)
        ch.chain()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ch.chain()
    for _ in range(3):
        ch.kv.copy_(kv0)
        ch.tokens.copy_(tok0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ch.tokens, eager)


# ------------------------------------------------------------ the C5 configuration
@pytest.fixture(scope="module", params=[1, 16], ids=["B1", "B16"])
def c5_chain(request):
    B = request.param
    print(f"C5 chain: building B={B}, 28 layers, ctx 2048 (prefill of random ids)", flush=True)
    ch = DraftChain(B, ctx_len=2048, k=6, seed=B)
    torch.cuda.synchronize()
    yield ch
    del ch
    torch.cuda.empty_cache()


@pytest.mark.parametrize("fused", [False, True], ids=["eager", "fused"])
def test_c5_configuration(c5_chain, fused):
    ch = c5_chain
    ch.fused = fused
    print(f"C5 chain B={ch.B} fused={fused}: eager steps", flush=True)
    kv0, tok0 = ch.kv.clone(), ch.tokens.clone()
    logits = [ch.step(s).float() for s in range(ch.k)]
    torch.cuda.synchronize()
    eager_tok, eager_kv = ch.tokens.clone(), ch.kv.clone()
    for s in range(ch.k):  # the greedy draft: each token is the argmax of its own logits
        assert torch.equal(eager_tok[s + 1], logits[s].argmax(dim=-1)), f"step {s}"
    print(f"C5 chain B={ch.B} fused={fused}: float32 reference of step 0", flush=True)
    kv_ref = kv0.clone()
    ref = ref_step(ch, kv_ref, tok0[0], 0)
    err = (logits[0] - ref).abs().max().item()
    assert err <= 2e-2 * ref.abs().max().item(), f"step 0: max err {err:.4g}"
    # the last draft step (s = k - 1) against the reference too, over the cache
    # the chain's own steps 0 .. k - 2 left (their rows are in eager_kv; the
    # reference rewrites step k - 1's rows itself)
    last = ch.k - 1
    print(f"C5 chain B={ch.B} fused={fused}: float32 reference of step {last}", flush=True)
    kv_ref = eager_kv.clone()
    ref = ref_step(ch, kv_ref, eager_tok[last], last)
    err = (logits[last] - ref).abs().max().item()
    assert err <= 2e-2 * ref.abs().max().item(), f"step {last}: max err {err:.4g}"
    del kv_ref, ref, logits
    print(f"C5 chain B={ch.B} fused={fused}: HIP graph of the 6 steps", flush=True)
    ch.kv.copy_(kv0)
    ch.tokens.copy_(tok0)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        ch.chain()
    torch.cuda.current_stream().wait_stream(st)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ch.chain()
    for _ in range(2):
        ch.kv.copy_(kv0)
        ch.tokens.copy_(tok0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ch.tokens, eager_tok)
        assert torch.equal(ch.kv.view(torch.int16), eager_kv.view(torch.int16))
    ch.kv.copy_(kv0)  # the fixture's initial state for the next form
    ch.tokens.copy_(tok0)
    del g, kv0, eager_kv
