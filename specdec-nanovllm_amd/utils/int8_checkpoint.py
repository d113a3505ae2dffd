"""The W8A16 on-disk format: converter, config reader and direct loader.

Mirrors the reference's three pieces of the format:
  * ``quantize_checkpoint`` — scripts/quantize_int8.py:48-166: a bf16 HF
    checkpoint becomes ``model_int8.safetensors`` (each quantized weight under
    its own key as int8, plus ``<key>_scale`` bf16 of shape [N, 1] per channel
    or [N, K // G, 1] per group; every other tensor bf16) and
    ``quant_config.json`` (quant_method "int8_w8a16", granularity, group_size,
    qmax, the quantized layer names, per-layer statistics); other files are
    copied. Only the block linears q/k/v/o/gate/up/down are quantized
    (embed_tokens, lm_head, norms and biases stay bf16), optionally narrowed by
    a preset. The quantization runs on the GPU (``ops.quantize_int8``), one
    tensor at a time.
  * ``read_quant_config`` — config.py:214-230 (`_resolve_quant`): a model
    directory with quant_config.json selects int8 and the modules to quantize.
  * ``load_int8_modules`` — utils/loader.py:147-176 (the load_int8_values path
    of `build_model_int8`): the int8 shards and scales of a converted
    checkpoint, concatenated into the engine's packed modules (q, k, v ->
    qkv_proj; gate, up -> gate_up_proj) in the engine's row order, per channel.
"""
from __future__ import annotations

import json
import os
import re
import shutil
from glob import glob

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from .. import ops
from ..layers.quant import QMAX, hf_names_to_modules

# Which tensors are quantized (scripts/quantize_int8.py:35-46): the block
# linears, by HF key; the format's consumers rely on exactly this selection.
QUANT_RE = re.compile(r"\.(q_proj|k_proj|v_proj|o_proj|gate_proj|up_proj|down_proj)\.weight$")
PRESETS = {
    "all": None,
    "ffn": re.compile(r"\.(gate_proj|up_proj|down_proj)\.weight$"),
    "attn": re.compile(r"\.(q_proj|k_proj|v_proj|o_proj)\.weight$"),
    "ffn_no_down": re.compile(r"\.(gate_proj|up_proj)\.weight$"),
}
SKIP_RE = re.compile(r"(embed_tokens|lm_head|norm|bias)")
INT8_FILE = "model_int8.safetensors"

# Qwen3's packed modules (models/qwen3.py packed_modules_mapping) and the row
# order of their shards (utils/loader.py:18).
QWEN3_PACKED = {"q_proj": ("qkv_proj", "q"), "k_proj": ("qkv_proj", "k"),
                "v_proj": ("qkv_proj", "v"), "gate_proj": ("gate_up_proj", 0),
                "up_proj": ("gate_up_proj", 1)}
_SHARD_ORDER = {"q": 0, "k": 1, "v": 2, 0: 0, 1: 1}


def wants_quant(key: str, preset: str = "all") -> bool:
    """Is checkpoint tensor ``key`` quantized under ``preset``?"""
    want = bool(QUANT_RE.search(key)) and not SKIP_RE.search(key)
    if want and PRESETS[preset] is not None:
        want = bool(PRESETS[preset].search(key))
    return want


def quantize_checkpoint(model_dir: str, out_dir: str, granularity: str = "per_channel",
                        group_size: int = 128, preset: str = "all",
                        device: str | torch.device = "cuda") -> dict:
    """Convert a bf16 checkpoint directory; returns the quant_config written."""
    if granularity not in ("per_channel", "per_group"):
        raise ValueError(granularity)
    src, dst = os.path.abspath(model_dir), os.path.abspath(out_dir)
    os.makedirs(dst, exist_ok=True)
    files = sorted(glob(os.path.join(src, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no safetensors under {src}")
    out, stats = {}, []
    n_quant = n_keep = bytes_q = bytes_k = 0
    gs = group_size if granularity == "per_group" else 0
    for fi in files:
        with safe_open(fi, "pt", "cpu") as f:
            for key in f.keys():
                t = f.get_tensor(key)
                if t.dtype not in (torch.bfloat16, torch.float16, torch.float32):
                    t = t.to(torch.bfloat16)
                if wants_quant(key, preset):
                    assert t.dim() == 2, f"{key}: only 2-D weights are quantized"
                    N, K = t.shape
                    if gs:
                        assert K % gs == 0, f"{key}: group size {gs} does not divide K={K}"
                    wd = t.to(device)
                    q, s = ops.quantize_int8(wd, gs)
                    G = gs or K
                    wf = wd.float().view(N, K // G, G)
                    amax = wf.abs().amax(dim=2)
                    deq = q.float().view(N, K // G, G) * s.float().view(N, K // G, 1)
                    err = ((wf - deq).norm() / wf.norm().clamp_min(1e-12)).item()
                    sat = (q.abs() == QMAX).float().mean().item()
                    scale_shape = (N, 1) if not gs else (N, K // G, 1)
                    out[key] = q.cpu()
                    out[key + "_scale"] = s.view(scale_shape).cpu()
                    n_quant += 1
                    bytes_q += q.numel() + s.numel() * 2
                    sf = s.float()
                    stats.append({
                        "name": key, "shape": [N, K],
                        "amax_mean": float(amax.mean()), "amax_max": float(amax.max()),
                        "scale_mean": float(sf.mean()), "scale_min": float(sf.min()),
                        "scale_max": float(sf.max()), "rel_err": err, "saturate_frac": sat,
                        "bytes_bf16": N * K * 2, "bytes_int8": q.numel() + s.numel() * 2})
                    del wd, wf, deq, q, s
                else:
                    out[key] = t.to(torch.bfloat16)
                    n_keep += 1
                    bytes_k += t.numel() * 2
    save_file(out, os.path.join(dst, INT8_FILE), metadata={"format": "pt"})
    del out
    for name in os.listdir(src):
        path = os.path.join(src, name)
        if os.path.isfile(path) and not name.endswith(".safetensors"):
            shutil.copy2(path, os.path.join(dst, name))
    cfg = {
        "quant_method": "int8_w8a16",
        "granularity": granularity,
        "group_size": group_size if granularity == "per_group" else None,
        "qmax": QMAX, "symmetric": True,
        "quantized_layers": [s["name"] for s in stats],
        "kept_bf16_layers": [],
        "preset": preset,
        "source_model": src,
        "n_quantized": n_quant, "n_kept": n_keep,
        "bytes_bf16_total": sum(s["bytes_bf16"] for s in stats) + bytes_k,
        "bytes_int8_total": bytes_q + bytes_k,
        "note": "quantized = block linears (q/k/v/o/gate/up/down); "
                "embed_tokens / lm_head / norm / bias stay bf16",
        "per_layer": stats,
    }
    with open(os.path.join(dst, "quant_config.json"), "w") as fh:
        json.dump(cfg, fh, indent=2, ensure_ascii=False)
    return cfg


def read_quant_config(model_dir: str, kind: str | None = None,
                      granularity: str = "per_channel", group_size: int = 128):
    """config.py:214-230: (kind, granularity, group_size, modules, config).
    Without quant_config.json: (None, granularity, group_size, (), None), or
    ValueError when int8 was asked for."""
    path = os.path.join(model_dir, "quant_config.json")
    if not os.path.isfile(path):
        if kind == "int8":
            raise ValueError(f"quant_weights='int8' but {model_dir} has no quant_config.json")
        return None, granularity, group_size, (), None
    with open(path) as fh:
        qc = json.load(fh)
    if qc.get("quant_method") != "int8_w8a16":
        raise ValueError(f"unsupported quantization format: {qc.get('quant_method')}")
    mods = tuple(hf_names_to_modules(qc["quantized_layers"]))
    return "int8", qc.get("granularity", granularity), qc.get("group_size") or group_size, mods, qc


def load_int8_modules(model_dir: str, packed_modules_mapping=None,
                      device: str | torch.device = "cuda") -> dict:
    """utils/loader.py:147-176 (int8 values read from the checkpoint): the
    quantized weights of a converted directory as {engine module name:
    (q int8 [N, K], scale bf16 [N])}, packed shards concatenated along the
    output rows in the engine's order. Per channel only, as the reference."""
    packed = QWEN3_PACKED if packed_modules_mapping is None else packed_modules_mapping
    fp = os.path.join(model_dir, INT8_FILE)
    if not os.path.isfile(fp):
        files = sorted(glob(os.path.join(model_dir, "*.safetensors")))
        if not files:
            raise FileNotFoundError(f"no safetensors under {model_dir}")
        fp = files[0]
    shards: dict = {}
    with safe_open(fp, "pt", "cpu") as f:
        keys = set(f.keys())
        for wk in sorted(keys):
            if wk.endswith("_scale") or wk + "_scale" not in keys:
                continue
            w = f.get_tensor(wk)
            s = f.get_tensor(wk + "_scale")
            if w.dtype != torch.int8 or s.dtype != torch.bfloat16:
                raise ValueError(f"{wk}: expected int8 weight and bf16 scale, got {w.dtype} / {s.dtype}")
            if s.numel() != w.shape[0]:
                raise ValueError(f"{wk}: per-group scales are not direct-loadable (as the reference)")
            name, sid = wk, None
            for k, (v, shard) in packed.items():
                if k in wk:
                    name, sid = wk.replace(k, v), shard
                    break
            shards.setdefault(name[: -len(".weight")], {})[sid] = (w, s)
    out = {}
    for mod, sh in shards.items():
        order = list(sh) if len(sh) == 1 else sorted(sh, key=lambda x: _SHARD_ORDER[x])
        q = torch.cat([sh[x][0] for x in order], dim=0).contiguous()
        sc = torch.cat([sh[x][1].reshape(-1) for x in order], dim=0).contiguous()
        out[mod] = (q.to(device), sc.to(device))
    return out
