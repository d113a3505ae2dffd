"""GPU parity of the int8 quantize kernel (csrc/quantize.hip, through the C
ABI) and of the on-disk format converter / loader.

Integer output: q must equal the oracle's (oracle/w8a16.quantize_weight, the
fp32 formula of nanovllm/layers/quant.py:123-148) bit for bit, and the bf16
scale bits too — including exact round-half-even ties and all-zero rows.
"""
import json
import os

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from conftest import bits16
from oracle import w8a16 as ow8
from specdec_nanovllm_amd import ops
from specdec_nanovllm_amd.layers.quant import quantize_weight
from specdec_nanovllm_amd.utils import int8_checkpoint as ic

pytestmark = pytest.mark.gpu
DEV = "cuda"


def oracle_q(w, granularity="per_channel", group_size=128):
    q, s = ow8.quantize_weight(w.float().cpu().numpy(), granularity, group_size)
    return q, torch.from_numpy(np.ascontiguousarray(s, dtype=np.float32)).to(torch.bfloat16)


@pytest.mark.parametrize("N,K,dtype,gran,gs", [(64, 1024, torch.bfloat16, "per_channel", 0),
                                               (37, 3072, torch.float16, "per_channel", 0),
                                               (5, 256, torch.float32, "per_channel", 0),
                                               (48, 1024, torch.bfloat16, "per_group", 128),
                                               (9, 512, torch.float32, "per_group", 64)])
def test_quantize_matches_oracle_bitwise(N, K, dtype, gran, gs):
    g = torch.Generator().manual_seed(N * K)
    w = (torch.randn((N, K), generator=g) * torch.rand((N, 1), generator=g) * 0.1).to(dtype)
    q, s = quantize_weight(w.to(DEV), gran, gs or 128)
    rq, rs = oracle_q(w, gran, gs or 128)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(bits16(s.reshape(rs.shape)), bits16(rs))


def test_round_half_even_ties_and_zero_rows():
    # scale = amax / 127 = 2^-4 exactly; w = (k + 1/2) 2^-4 sits on the ties
    K = 256
    w = torch.zeros((3, K), dtype=torch.float32)
    w[0, 0] = 127 * 2.0 ** -4
    w[0, 1:9] = torch.tensor([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5]) * 2.0 ** -4
    w[2] = torch.linspace(-1, 1, K)  # row 1 stays all zero: scale 1e-8, q 0
    q, s = ops.quantize_int8(w.to(DEV))
    assert q[0, 1:9].tolist() == [0, 2, 2, 0, -2, -2, 126, -126]
    assert q[1].abs().sum().item() == 0
    rq, rs = oracle_q(w)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(bits16(s.view(-1)), bits16(rs))


def _tiny_qwen3_checkpoint(d, layers=2, hidden=256, heads=4, kv=2, hd=64, inter=512, vocab=300):
    g = torch.Generator().manual_seed(1)
    t = {}

    def r(*shape):
        return (torch.randn(shape, generator=g) * 0.05).to(torch.bfloat16)
    t["model.embed_tokens.weight"] = r(vocab, hidden)
    for i in range(layers):
        p = f"model.layers.{i}."
        t[p + "self_attn.q_proj.weight"] = r(heads * hd, hidden)
        t[p + "self_attn.k_proj.weight"] = r(kv * hd, hidden)
        t[p + "self_attn.v_proj.weight"] = r(kv * hd, hidden)
        t[p + "self_attn.o_proj.weight"] = r(hidden, heads * hd)
        t[p + "self_attn.q_norm.weight"] = r(hd)
        t[p + "self_attn.k_norm.weight"] = r(hd)
        t[p + "mlp.gate_proj.weight"] = r(inter, hidden)
        t[p + "mlp.up_proj.weight"] = r(inter, hidden)
        t[p + "mlp.down_proj.weight"] = r(hidden, inter)
        t[p + "input_layernorm.weight"] = r(hidden)
        t[p + "post_attention_layernorm.weight"] = r(hidden)
    t["model.norm.weight"] = r(hidden)
    t["lm_head.weight"] = r(vocab, hidden)
    save_file(t, os.path.join(d, "model.safetensors"))
    with open(os.path.join(d, "config.json"), "w") as fh:
        json.dump({"model_type": "qwen3", "tie_word_embeddings": False}, fh)
    return t


@pytest.mark.parametrize("gran", ["per_channel", "per_group"])
def test_converter_round_trip(tmp_path, gran):
    src, dst = tmp_path / "bf16", tmp_path / "int8"
    src.mkdir()
    t = _tiny_qwen3_checkpoint(str(src))
    cfg = ic.quantize_checkpoint(str(src), str(dst), gran, 64)
    assert sorted(os.listdir(dst)) == ["config.json", "model_int8.safetensors", "quant_config.json"]
    assert cfg["quant_method"] == "int8_w8a16" and cfg["granularity"] == gran
    assert cfg["n_quantized"] == 14 and cfg["n_kept"] == len(t) - 14
    with safe_open(str(dst / "model_int8.safetensors"), "pt", "cpu") as f:
        keys = set(f.keys())
        for k, w in t.items():
            if ic.wants_quant(k):
                q, s = f.get_tensor(k), f.get_tensor(k + "_scale")
                N, K = w.shape
                assert q.dtype == torch.int8 and s.dtype == torch.bfloat16
                assert s.shape == ((N, 1) if gran == "per_channel" else (N, K // 64, 1))
                rq, rs = oracle_q(w, gran, 64)
                assert np.array_equal(q.numpy(), rq)
                assert np.array_equal(bits16(s.reshape(rs.shape)), bits16(rs))
            else:
                assert k + "_scale" not in keys and torch.equal(f.get_tensor(k), w)
    kind, g2, _, mods, qc = ic.read_quant_config(str(dst))
    assert kind == "int8" and g2 == gran and len(mods) == 8  # 2 layers x (qkv, o, gate_up, down)
    if gran == "per_channel":
        loaded = ic.load_int8_modules(str(dst), device=DEV)
        q, s = loaded["model.layers.1.self_attn.qkv_proj"]
        parts = [quantize_weight(t[f"model.layers.1.self_attn.{n}_proj.weight"].to(DEV))
                 for n in ("q", "k", "v")]
        assert torch.equal(q, torch.cat([p[0] for p in parts]))
        assert torch.equal(s, torch.cat([p[1] for p in parts]))
        q, s = loaded["model.layers.0.mlp.gate_up_proj"]
        assert q.shape == (1024, 256) and s.shape == (1024,)
    else:
        with pytest.raises(ValueError):
            ic.load_int8_modules(str(dst), device=DEV)
