"""The draft step's neighbour ops restated in numpy (bf16 activations).

Test infrastructure only (see oracle/__init__.py). Values are float32 arrays
holding bf16 numbers; ``bf16.round_f32`` is every conversion back to bf16.

  rmsnorm / add_rmsnorm   nanovllm/layers/layernorm.py:16-47
  rope                    nanovllm/layers/rotary_embedding.py:6-48
  qk_norm_rope            nanovllm/models/qwen3.py:80-88 (q/k norm, then RoPE)
  silu_mul                nanovllm/layers/activation.py:6-11
  philox4x32_10, sample   nanovllm/layers/sampler.py:6-12 (exponential race),
                          with this build's counter-based noise
  verify_batch            nanovllm/spec_decode/verify.py:39-183 (rejection
                          sampling), with the same noise
"""
import numpy as np

from . import bf16

_R = bf16.round_f32


def _f16(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def rounder(dtype: str):
    """The activation dtype's rounding of float32 values: "bf16" or "f16"."""
    return {"bf16": bf16.round_f32, "f16": _f16}[dtype]


def rmsnorm(x, w, eps, dtype="bf16"):
    """layernorm.py:16-26: fp32 x * rsqrt(mean(x^2) + eps), to the dtype, times w,
    to the dtype."""
    R = rounder(dtype)
    x = np.asarray(x, dtype=np.float32)
    var = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    r = (np.float32(1.0) / np.sqrt(var + np.float32(eps))).astype(np.float32)
    return R(R(x * r) * np.asarray(w, dtype=np.float32))


def add_rmsnorm(x, residual, w, eps, dtype="bf16"):
    """layernorm.py:28-40: s = x + residual in fp32; residual_out = s in the
    dtype; the norm of s (not of the rounded residual). Returns (out, residual_out)."""
    s = np.asarray(x, dtype=np.float32) + np.asarray(residual, dtype=np.float32)
    return rmsnorm(s, w, eps, dtype), rounder(dtype)(s)


def rope(x, positions, cos_sin, dtype="bf16"):
    """rotary_embedding.py:6-16 on (T, H, D): x1, x2 = halves; y1 = x1 cos - x2 sin,
    y2 = x2 cos + x1 sin in fp32 (separately rounded products), then bf16."""
    x = np.asarray(x, dtype=np.float32)
    half = x.shape[-1] // 2
    cs = np.asarray(cos_sin, dtype=np.float32)[np.asarray(positions)]  # (T, D)
    c, s = cs[:, None, :half], cs[:, None, half:2 * half]
    x1, x2 = x[..., :half], x[..., half:]
    y1 = (x1 * c).astype(np.float32) - (x2 * s).astype(np.float32)
    y2 = (x2 * c).astype(np.float32) + (x1 * s).astype(np.float32)
    return rounder(dtype)(np.concatenate([y1, y2], axis=-1))


def rope_cache(max_position, head_dim, base):
    """rotary_embedding.py:29-36: (max_position, head_dim) fp32 rows [cos | sin]."""
    inv_freq = 1.0 / (np.float32(base) ** (np.arange(0, head_dim, 2, dtype=np.float32) / head_dim))
    t = np.arange(max_position, dtype=np.float32)
    freqs = np.outer(t, inv_freq.astype(np.float32)).astype(np.float32)
    return np.concatenate([np.cos(freqs), np.sin(freqs)], axis=-1).astype(np.float32)


def qk_norm_rope(q, k, positions, cos_sin, q_w=None, k_w=None, eps=1e-6, dtype="bf16"):
    """qwen3.py:80-88: per-head RMSNorm of q and k (when weights are given),
    then RoPE of both."""
    if q_w is not None:
        q = rmsnorm(q, q_w, eps, dtype)
        k = rmsnorm(k, k_w, eps, dtype)
    return rope(q, positions, cos_sin, dtype), rope(k, positions, cos_sin, dtype)


def silu_mul(x, dtype="bf16"):
    """activation.py:6-11 with eager rounding: R(R(silu(g)) * u), R the dtype."""
    R = rounder(dtype)
    x = np.asarray(x, dtype=np.float32)
    half = x.shape[-1] // 2
    g, u = x[..., :half], x[..., half:]
    s = R((g / (np.float32(1) + np.exp(-g, dtype=np.float32))).astype(np.float32))
    return R(s * u)


def argmax_first(logits):
    """torch.argmax semantics: index of the first maximum of each row."""
    return np.argmax(np.asarray(logits, dtype=np.float32), axis=-1).astype(np.int64)


_M0, _M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
_W0, _W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)


def philox4x32_10(c0, c1, c2, c3, k0, k1):
    """Philox4x32-10 (Salmon et al., SC 2011) on uint32 arrays; returns 4 arrays."""
    c = [np.asarray(v, dtype=np.uint32).copy() for v in (c0, c1, c2, c3)]
    k0 = np.asarray(k0, dtype=np.uint32).copy()
    k1 = np.asarray(k1, dtype=np.uint32).copy()
    mask = np.uint64(0xFFFFFFFF)
    with np.errstate(over="ignore"):
        for _ in range(10):
            p0 = _M0 * c[0].astype(np.uint64)
            p1 = _M1 * c[2].astype(np.uint64)
            n0 = (p1 >> np.uint64(32)).astype(np.uint32) ^ c[1] ^ k0
            n1 = (p1 & mask).astype(np.uint32)
            n2 = (p0 >> np.uint64(32)).astype(np.uint32) ^ c[3] ^ k1
            n3 = (p0 & mask).astype(np.uint32)
            c = [n0, n1, n2, n3]
            k0 = k0 + _W0
            k1 = k1 + _W1
    return c


def element_words(idx, c1, c2, c3, seed):
    """The 32-bit noise word of element idx: word idx % 4 of the Philox block
    with counter (idx // 4, c1, c2, c3) (four elements per Philox call)."""
    idx = np.asarray(idx, dtype=np.uint32)
    r = philox4x32_10(idx >> np.uint32(2), c1, c2, c3, np.uint32(seed & 0xFFFFFFFF),
                      np.uint32((seed >> 32) & 0xFFFFFFFF))
    return np.choose((idx & np.uint32(3)).astype(np.int64), r)


def sample_keys(logits, temperatures, seed, offset):
    """The per-element race keys: l / T - log(max(-log U, 1e-10)), U in (0, 1]
    from element_words of column i with counter (i // 4, row ^ offset_hi,
    offset_lo, 0). argmax of these is the draw of sampler.py:6-12
    (argmax(softmax(l / T) / E), E = -log U ~ Exp(1))."""
    logits = np.asarray(logits, dtype=np.float32)
    rows, V = logits.shape
    col = np.broadcast_to(np.arange(V, dtype=np.uint32)[None, :], (rows, V))
    row = np.broadcast_to(np.arange(rows, dtype=np.uint32)[:, None], (rows, V))
    off_lo, off_hi = np.uint32(offset & 0xFFFFFFFF), np.uint32((offset >> 32) & 0xFFFFFFFF)
    w = element_words(col, row ^ off_hi, np.full((rows, V), off_lo, np.uint32),
                      np.zeros((rows, V), np.uint32), seed)
    u = ((w >> np.uint32(8)).astype(np.float32) + np.float32(1)) * np.float32(1.0 / 16777216.0)
    e = np.maximum(-np.log(u), np.float32(1e-10)).astype(np.float32)
    t = np.asarray(temperatures, dtype=np.float32)[:, None]
    return (logits * (np.float32(1) / t) - np.log(e)).astype(np.float32)


def sample(logits, temperatures, seed, offset):
    """Tokens of sampler.py:6-12 with this noise; rows with T <= 0 are greedy."""
    temperatures = np.asarray(temperatures, dtype=np.float32)
    keys = sample_keys(logits, np.where(temperatures > 0, temperatures, 1), seed, offset)
    greedy = argmax_first(logits)
    return np.where(temperatures > 0, np.argmax(keys, axis=-1), greedy).astype(np.int64)


def _philox_word0(c0, c1, c2, c3, seed):
    return philox4x32_10(c0, c1, c2, c3, np.uint32(seed & 0xFFFFFFFF),
                         np.uint32((seed >> 32) & 0xFFFFFFFF))[0]


def _softmax_rows(x):
    x = np.asarray(x, dtype=np.float32)
    m = x.max(axis=-1, keepdims=True)
    e = np.exp((x - m).astype(np.float32), dtype=np.float32)
    return (e / e.sum(axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)


def verify_batch(draft, target, tokens, temperatures=None, point_mass=False, seed=0, offset=0):
    """spec_decode/verify.py:39-183 with this build's noise. Returns
    (accepted (B,), bonus (B,), accept_mask (B, k)).

    q = softmax(draft / T) (draft as given when point_mass), p = softmax(target / T);
    candidate j passes when u_j < min(1, p_j[x_j] / max(q_j[x_j], 1e-10)) (never
    when q_j[x_j] == 0), u_j = (Philox(j, b ^ off_hi, off_lo, 1).c0 >> 8) 2^-24;
    accepted = first failure (k if none); bonus = argmax(max(0, p_a - q_a) / E)
    with q_k = 0, or argmax(p_a / E) when that residual is all zero,
    E_i = max(-log U_i, 1e-10), U_i = ((W_i >> 8) + 1) 2^-24 with W_i = element_words of i with
    counter (i // 4, b ^ off_hi, off_lo, 2).
    """
    draft = np.asarray(draft, dtype=np.float32)
    target = np.asarray(target, dtype=np.float32)
    B, k, V = draft.shape
    T = np.ones(B, np.float32) if temperatures is None else np.asarray(temperatures, np.float32)
    T = np.where(T > 0, T, np.float32(1)).astype(np.float32)
    q = draft if point_mass else _softmax_rows(draft / T[:, None, None])
    p = _softmax_rows(target / T[:, None, None])
    off_lo = np.uint32(offset & 0xFFFFFFFF)
    off_hi = np.uint32((offset >> 32) & 0xFFFFFFFF)
    bb = np.arange(B, dtype=np.uint32) ^ off_hi                        # (B,)
    tok = np.asarray(tokens, dtype=np.int64).reshape(B, k)
    valid = (tok >= 0) & (tok < V)
    tc = np.where(valid, tok, 0)
    qt = np.where(valid, np.take_along_axis(q, tc[:, :, None], 2)[:, :, 0], np.float32(0))
    pt = np.where(valid, np.take_along_axis(p[:, :k], tc[:, :, None], 2)[:, :, 0], np.float32(0))
    ratio = np.where(qt > 0, np.minimum(pt / np.maximum(qt, np.float32(1e-10)), np.float32(1)),
                     np.float32(0)).astype(np.float32)
    jj = np.broadcast_to(np.arange(k, dtype=np.uint32)[None, :], (B, k))
    w = _philox_word0(jj, np.broadcast_to(bb[:, None], (B, k)), np.full((B, k), off_lo, np.uint32),
                      np.ones((B, k), np.uint32), seed)
    u = (w >> np.uint32(8)).astype(np.float32) * np.float32(1.0 / 16777216.0)
    mask = u < ratio
    fail = ~mask
    accepted = np.where(fail.any(axis=1), fail.argmax(axis=1), k).astype(np.int64)
    rows = np.arange(B)
    pa = p[rows, accepted]                                             # (B, V)
    qpad = np.concatenate([q, np.zeros((B, 1, V), np.float32)], axis=1)
    qa = qpad[rows, accepted]
    r = np.maximum(pa - qa, np.float32(0))
    cols = np.broadcast_to(np.arange(V, dtype=np.uint32)[None, :], (B, V))
    w2 = element_words(cols, np.broadcast_to(bb[:, None], (B, V)), np.full((B, V), off_lo, np.uint32),
                       np.full((B, V), 2, np.uint32), seed)
    U = ((w2 >> np.uint32(8)).astype(np.float32) + np.float32(1)) * np.float32(1.0 / 16777216.0)
    E = np.maximum(-np.log(U), np.float32(1e-10)).astype(np.float32)
    use_r = r.sum(axis=1, dtype=np.float32) > 0
    bonus = np.where(use_r, np.argmax(r / E, axis=1), np.argmax(pa / E, axis=1)).astype(np.int64)
    return accepted, bonus, mask
