// store_kvcache.hip — bit-exact KV-cache slot write for gfx950.
//
// Same contract as `store_kvcache_kernel` (nanovllm/layers/attention.py:10-30):
// token i with slot s != -1 copies its (num_kv_heads x head_dim) key and value
// rows to cache position (s / block_size, s % block_size). The reference runs
// one program per token and moves the whole row with one vector of D
// elements; here the row is cut into 16-byte pieces so every lane issues one
// 16-byte load and one 16-byte store, and a single grid-stride launch covers
// all tokens, heads and both tensors.
#include "sd_common.h"

namespace {

struct StoreParams {
  const char* key;
  const char* value;
  char* k_cache;
  char* v_cache;
  const int32_t* slots;
  int64_t key_stok, key_shead;      // bytes
  int64_t val_stok, val_shead;      // bytes
  int64_t c_sblk, c_spos, c_shead;  // bytes
  int64_t num_tokens;
  int64_t num_slots;
  int32_t num_heads;
  int32_t pieces;  // 16-byte pieces per head row
  int32_t block_size;
};

// One work item = one 16-byte piece of one head row of K or V.
__global__ __launch_bounds__(256) void store_kvcache_kernel(StoreParams p) {
  const int64_t per_tensor = p.num_tokens * p.num_heads * p.pieces;
  const int64_t total = 2 * per_tensor;
  for (int64_t it = blockIdx.x * 256ll + threadIdx.x; it < total; it += gridDim.x * 256ll) {
    const bool is_v = it >= per_tensor;
    int64_t r = is_v ? it - per_tensor : it;
    const int piece = static_cast<int>(r % p.pieces);
    r /= p.pieces;
    const int head = static_cast<int>(r % p.num_heads);
    const int64_t tok = r / p.num_heads;
    const int64_t slot = p.slots[tok];
    if (slot < 0 || slot >= p.num_slots) continue;  // -1 = padding row, never written
    const int64_t blk = slot / p.block_size;
    const int64_t off = slot - blk * p.block_size;
    const char* src = is_v ? p.value + tok * p.val_stok + head * p.val_shead
                           : p.key + tok * p.key_stok + head * p.key_shead;
    char* dst = (is_v ? p.v_cache : p.k_cache) + blk * p.c_sblk + off * p.c_spos +
                head * p.c_shead;
    sd::store16(dst + piece * 16, sd::load16(src + piece * 16));
  }
}

}  // namespace

extern "C" int sd_store_kvcache(const void* key, int64_t key_stride_tok, int64_t key_stride_head,
                                const void* value, int64_t value_stride_tok,
                                int64_t value_stride_head, void* k_cache, void* v_cache,
                                int64_t cache_stride_block, int64_t cache_stride_pos,
                                int64_t cache_stride_head, const int32_t* slot_mapping,
                                int64_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                                int32_t block_size, int64_t num_blocks, int32_t elem_bytes,
                                void* stream) {
  sd::clear_error();
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0 ||
      num_blocks <= 0) {
    sd::set_error("store_kvcache: invalid sizes (tokens=%lld heads=%d head_dim=%d bs=%d "
                  "blocks=%lld)",
                  (long long)num_tokens, num_kv_heads, head_dim, block_size,
                  (long long)num_blocks);
    return SD_ERR_VALUE;
  }
  if (num_tokens > (1ll << 31) || num_kv_heads > (1 << 16) || head_dim > (1 << 12) ||
      block_size > (1 << 20) || num_blocks > (1ll << 32)) {
    sd::set_error("store_kvcache: sizes too large (tokens=%lld heads=%d head_dim=%d bs=%d "
                  "blocks=%lld)", (long long)num_tokens, num_kv_heads, head_dim, block_size,
                  (long long)num_blocks);
    return SD_ERR_UNSUPPORTED;
  }
  if (!sd::strides_ok({key_stride_tok, key_stride_head, value_stride_tok, value_stride_head,
                       cache_stride_block, cache_stride_pos, cache_stride_head})) {
    sd::set_error("store_kvcache: strides must lie in [-2^40, 2^40] elements");
    return SD_ERR_VALUE;
  }
  if (num_tokens == 0) return SD_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping) {
    sd::set_error("store_kvcache: null pointer argument");
    return SD_ERR_VALUE;
  }
  if (elem_bytes != 2 && elem_bytes != 4) {
    sd::set_error("store_kvcache: elem_bytes must be 2 or 4, got %d", elem_bytes);
    return SD_ERR_UNSUPPORTED;
  }
  const int64_t row_bytes = static_cast<int64_t>(head_dim) * elem_bytes;
  const int64_t eb = elem_bytes;
  const bool ok16 = row_bytes % 16 == 0 && sd::aligned16(key) && sd::aligned16(value) &&
                    sd::aligned16(k_cache) && sd::aligned16(v_cache) &&
                    (key_stride_tok * eb) % 16 == 0 && (key_stride_head * eb) % 16 == 0 &&
                    (value_stride_tok * eb) % 16 == 0 && (value_stride_head * eb) % 16 == 0 &&
                    (cache_stride_block * eb) % 16 == 0 && (cache_stride_pos * eb) % 16 == 0 &&
                    (cache_stride_head * eb) % 16 == 0;
  if (!ok16) {
    sd::set_error("store_kvcache: rows, pointers and strides must be 16-byte aligned");
    return SD_ERR_UNSUPPORTED;
  }
  StoreParams p;
  p.key = static_cast<const char*>(key);
  p.value = static_cast<const char*>(value);
  p.k_cache = static_cast<char*>(k_cache);
  p.v_cache = static_cast<char*>(v_cache);
  p.slots = slot_mapping;
  p.key_stok = key_stride_tok * eb;
  p.key_shead = key_stride_head * eb;
  p.val_stok = value_stride_tok * eb;
  p.val_shead = value_stride_head * eb;
  p.c_sblk = cache_stride_block * eb;
  p.c_spos = cache_stride_pos * eb;
  p.c_shead = cache_stride_head * eb;
  p.num_tokens = num_tokens;
  p.num_slots = num_blocks * block_size;
  p.num_heads = num_kv_heads;
  p.pieces = static_cast<int32_t>(row_bytes / 16);
  p.block_size = block_size;
  const int64_t items = 2 * num_tokens * num_kv_heads * p.pieces;
  int64_t blocks = (items + 255) / 256;
  if (blocks > 2048) blocks = 2048;
  hipLaunchKernelGGL(store_kvcache_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), p);
  return sd::check_launch("store_kvcache");
}
