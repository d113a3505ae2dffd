"""CPU checks of the W8A16 on-disk format's host logic: which checkpoint
tensors are quantized (scripts/quantize_int8.py:35-46 of the reference),
the HF-name -> engine-module mapping with its completeness rule
(nanovllm/layers/quant.py:31-63) and the quant_config detection
(nanovllm/config.py:214-230)."""
import json

import pytest

from specdec_nanovllm_amd.layers.quant import hf_names_to_modules
from specdec_nanovllm_amd.utils import int8_checkpoint as ic


def test_selection_and_presets():
    L = "model.layers.3."
    assert ic.wants_quant(L + "self_attn.q_proj.weight")
    assert ic.wants_quant(L + "mlp.down_proj.weight")
    for k in ("model.embed_tokens.weight", "lm_head.weight", L + "input_layernorm.weight",
              L + "self_attn.q_norm.weight", L + "self_attn.q_proj.bias", "model.norm.weight"):
        assert not ic.wants_quant(k), k
    assert ic.wants_quant(L + "mlp.up_proj.weight", "ffn")
    assert not ic.wants_quant(L + "self_attn.o_proj.weight", "ffn")
    assert ic.wants_quant(L + "self_attn.o_proj.weight", "attn")
    assert not ic.wants_quant(L + "mlp.down_proj.weight", "ffn_no_down")


def test_hf_names_to_modules_complete_groups_only():
    L = "model.layers.0."
    full = [L + f"self_attn.{n}_proj.weight" for n in "qkv"] + \
           [L + "mlp.gate_proj.weight", L + "mlp.up_proj.weight", L + "mlp.down_proj.weight",
            L + "self_attn.o_proj.weight"]
    assert hf_names_to_modules(full) == sorted([L + "self_attn.qkv_proj", L + "mlp.gate_up_proj",
                                                L + "mlp.down_proj", L + "self_attn.o_proj"])
    with pytest.raises(ValueError):
        hf_names_to_modules([L + "self_attn.q_proj.weight", L + "self_attn.k_proj.weight"])
    with pytest.raises(ValueError):
        hf_names_to_modules([L + "mlp.gate_proj.weight"])
    with pytest.raises(ValueError):
        hf_names_to_modules(["model.embed_tokens.weight"])


def test_read_quant_config(tmp_path):
    assert ic.read_quant_config(str(tmp_path))[0] is None
    with pytest.raises(ValueError):
        ic.read_quant_config(str(tmp_path), kind="int8")
    L = "model.layers.0."
    (tmp_path / "quant_config.json").write_text(json.dumps({
        "quant_method": "int8_w8a16", "granularity": "per_group", "group_size": 64,
        "quantized_layers": [L + "mlp.down_proj.weight"]}))
    kind, gran, gs, mods, qc = ic.read_quant_config(str(tmp_path))
    assert (kind, gran, gs, mods) == ("int8", "per_group", 64, (L + "mlp.down_proj",))
    (tmp_path / "quant_config.json").write_text(json.dumps({"quant_method": "gptq"}))
    with pytest.raises(ValueError):
        ic.read_quant_config(str(tmp_path))
