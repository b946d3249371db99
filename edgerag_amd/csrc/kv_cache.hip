// Slot-mapped KV append, history gather and whole-block copy over the head-major paged pool
// [n_kv_heads, num_blocks, block_size, head_dim].
//
// All three are pure data movement, bound by HBM bandwidth: each thread moves one 16-byte
// vector (8 fp16 / 4 fp32 elements), consecutive threads touch consecutive 16-byte chunks of one
// pool row, so every wave issues fully coalesced 1 KiB accesses. No LDS, no MFMA.
#include "common.h"

namespace edgerag {
namespace {

constexpr int kThreads = 256;

// ---- append ----------------------------------------------------------------------------------
// One thread per (token, head, VEC-element chunk); blockIdx.y selects key (0) or value (1).
// Src/Dst differ only when the caller appends e.g. fp32 activations into an fp16 pool; the
// conversion rounds to nearest-even like Tensor.to() (edgerag/cache/paged.py:206).
template <typename Src, typename Dst, int VEC>
__global__ __launch_bounds__(kThreads) void kv_append_kernel(
    const Src* __restrict__ key, const Src* __restrict__ value, int64_t s_tok, int64_t s_head,
    const int32_t* __restrict__ slots, int32_t num_tokens, Dst* __restrict__ kpool,
    Dst* __restrict__ vpool, int32_t n_heads, int32_t num_blocks, int32_t block_size,
    int32_t head_dim) {
  const Src* src = blockIdx.y == 0 ? key : value;
  Dst* pool = blockIdx.y == 0 ? kpool : vpool;
  if (src == nullptr) return;
  const int chunks = head_dim / VEC;
  const int64_t total = int64_t(num_tokens) * n_heads * chunks;
  const int64_t n_slots = int64_t(num_blocks) * block_size;
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * kThreads) {
    const int c = int(i % chunks);
    const int64_t th = i / chunks;
    const int h = int(th % n_heads);
    const int t = int(th / n_heads);
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= n_slots) continue;  // padding, or a slot outside the pool
    const int64_t blk = slot / block_size, off = slot % block_size;
    const Src* s = src + t * s_tok + h * s_head + c * VEC;
    Dst* d = pool + ((int64_t(h) * num_blocks + blk) * block_size + off) * head_dim + c * VEC;
    if constexpr (sizeof(Src) * VEC == 16 && sizeof(Dst) == sizeof(Src) &&
                  __is_same(Src, Dst)) {
      store16(d, load16(s));
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) d[e] = from_f32<Dst>(to_f32<Src>(s[e]));
    }
  }
}

// ---- gather ----------------------------------------------------------------------------------
template <typename T, int VEC>
__global__ __launch_bounds__(kThreads) void kv_gather_kernel(
    const T* __restrict__ pool, int32_t n_heads, int32_t num_blocks, int32_t block_size,
    int32_t head_dim, const int32_t* __restrict__ block_ids, int32_t seq_len, T* __restrict__ out) {
  const int chunks = head_dim / VEC;
  const int64_t total = int64_t(n_heads) * seq_len * chunks;
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * kThreads) {
    const int c = int(i % chunks);
    const int64_t hp = i / chunks;
    const int p = int(hp % seq_len);
    const int h = int(hp / seq_len);
    const int32_t blk = block_ids[p / block_size];
    T* d = out + (int64_t(h) * seq_len + p) * head_dim + c * VEC;
    if (blk < 0 || blk >= num_blocks) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) d[e] = from_f32<T>(0.f);
      continue;
    }
    const T* s = pool + ((int64_t(h) * num_blocks + blk) * block_size + p % block_size) * head_dim +
                 c * VEC;
    if constexpr (sizeof(T) * VEC == 16) {
      store16(d, load16(s));
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) d[e] = s[e];
    }
  }
}

// ---- block copy ------------------------------------------------------------------------------
// Moves raw 16-byte chunks (or bytes for odd-sized blocks): dtype-agnostic.
__global__ __launch_bounds__(kThreads) void kv_copy_blocks16(
    Vec16* __restrict__ pool, int32_t n_heads, int32_t num_blocks, int64_t block_chunks,
    const int32_t* __restrict__ src, const int32_t* __restrict__ dst, int32_t n_pairs) {
  const int64_t per_pair = int64_t(n_heads) * block_chunks;
  const int64_t total = per_pair * n_pairs;
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * kThreads) {
    const int pair = int(i / per_pair);
    const int64_t rem = i % per_pair;
    const int h = int(rem / block_chunks);
    const int64_t c = rem % block_chunks;
    const int32_t s = src[pair], d = dst[pair];
    if (s < 0 || s >= num_blocks || d < 0 || d >= num_blocks) continue;
    pool[(int64_t(h) * num_blocks + d) * block_chunks + c] =
        pool[(int64_t(h) * num_blocks + s) * block_chunks + c];
  }
}

__global__ __launch_bounds__(kThreads) void kv_copy_blocks1(
    uint8_t* __restrict__ pool, int32_t n_heads, int32_t num_blocks, int64_t block_bytes,
    const int32_t* __restrict__ src, const int32_t* __restrict__ dst, int32_t n_pairs) {
  const int64_t per_pair = int64_t(n_heads) * block_bytes;
  const int64_t total = per_pair * n_pairs;
  for (int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * kThreads) {
    const int pair = int(i / per_pair);
    const int64_t rem = i % per_pair;
    const int h = int(rem / block_bytes);
    const int64_t c = rem % block_bytes;
    const int32_t s = src[pair], d = dst[pair];
    if (s < 0 || s >= num_blocks || d < 0 || d >= num_blocks) continue;
    pool[(int64_t(h) * num_blocks + d) * block_bytes + c] =
        pool[(int64_t(h) * num_blocks + s) * block_bytes + c];
  }
}

int elem_size(int32_t dtype) {
  switch (dtype) {
    case EDGERAG_F32: return 4;
    case EDGERAG_F16: return 2;
    case EDGERAG_BF16: return 2;
    default: return 0;
  }
}

unsigned grid_for(int64_t work) {
  int64_t blocks = (work + kThreads - 1) / kThreads;
  if (blocks < 1) blocks = 1;
  if (blocks > 65535LL * 16) blocks = 65535LL * 16;  // grid-stride loops cover the rest
  return unsigned(blocks);
}

template <typename Src, typename Dst>
int launch_append(const void* key, const void* value, int64_t s_tok, int64_t s_head,
                  const int32_t* slots, int32_t T, void* kp, void* vp, int32_t H, int32_t NB,
                  int32_t BS, int32_t D, hipStream_t stream) {
  constexpr int kVec = 16 / (sizeof(Src) > sizeof(Dst) ? sizeof(Src) : sizeof(Dst));
  const bool vec_ok = D % kVec == 0 && (s_tok % kVec) == 0 && (s_head % kVec) == 0 &&
                      (key == nullptr || aligned16(key)) && (value == nullptr || aligned16(value)) &&
                      (kp == nullptr || aligned16(kp)) && (vp == nullptr || aligned16(vp));
  if (vec_ok) {
    const int64_t work = int64_t(T) * H * (D / kVec);
    hipLaunchKernelGGL((kv_append_kernel<Src, Dst, kVec>), dim3(grid_for(work), 2), dim3(kThreads),
                       0, stream, static_cast<const Src*>(key), static_cast<const Src*>(value),
                       s_tok, s_head, slots, T, static_cast<Dst*>(kp), static_cast<Dst*>(vp), H,
                       NB, BS, D);
  } else {
    const int64_t work = int64_t(T) * H * D;
    hipLaunchKernelGGL((kv_append_kernel<Src, Dst, 1>), dim3(grid_for(work), 2), dim3(kThreads), 0,
                       stream, static_cast<const Src*>(key), static_cast<const Src*>(value), s_tok,
                       s_head, slots, T, static_cast<Dst*>(kp), static_cast<Dst*>(vp), H, NB, BS,
                       D);
  }
  return check_launch("edgerag_kv_append");
}

template <typename Src>
int dispatch_append_dst(int32_t pool_dtype, const void* key, const void* value, int64_t s_tok,
                        int64_t s_head, const int32_t* slots, int32_t T, void* kp, void* vp,
                        int32_t H, int32_t NB, int32_t BS, int32_t D, hipStream_t stream) {
  switch (pool_dtype) {
    case EDGERAG_F32:
      return launch_append<Src, float>(key, value, s_tok, s_head, slots, T, kp, vp, H, NB, BS, D,
                                       stream);
    case EDGERAG_F16:
      return launch_append<Src, f16>(key, value, s_tok, s_head, slots, T, kp, vp, H, NB, BS, D,
                                     stream);
    case EDGERAG_BF16:
      return launch_append<Src, bf16>(key, value, s_tok, s_head, slots, T, kp, vp, H, NB, BS, D,
                                      stream);
  }
  return fail(EDGERAG_EINVAL, "edgerag_kv_append: unknown pool dtype %d", pool_dtype);
}

template <typename T>
int launch_gather(const void* pool, int32_t H, int32_t NB, int32_t BS, int32_t D,
                  const int32_t* ids, int32_t L, void* out, hipStream_t stream) {
  constexpr int kVec = 16 / sizeof(T);
  const int64_t total_elems = int64_t(H) * L * D;
  if (D % kVec == 0 && aligned16(pool) && aligned16(out)) {
    hipLaunchKernelGGL((kv_gather_kernel<T, kVec>), dim3(grid_for(total_elems / kVec)),
                       dim3(kThreads), 0, stream, static_cast<const T*>(pool), H, NB, BS, D, ids, L,
                       static_cast<T*>(out));
  } else {
    hipLaunchKernelGGL((kv_gather_kernel<T, 1>), dim3(grid_for(total_elems)), dim3(kThreads), 0,
                       stream, static_cast<const T*>(pool), H, NB, BS, D, ids, L,
                       static_cast<T*>(out));
  }
  return check_launch("edgerag_kv_gather");
}

int check_pool_shape(const char* fn, int32_t H, int32_t NB, int32_t BS, int32_t D) {
  if (H <= 0 || NB <= 0 || BS <= 0 || D <= 0) {
    return fail(EDGERAG_EINVAL, "%s: pool dims must be positive (H=%d NB=%d BS=%d D=%d)", fn, H, NB,
                BS, D);
  }
  return EDGERAG_OK;
}

}  // namespace
}  // namespace edgerag

using namespace edgerag;

extern "C" int edgerag_kv_append(const void* key, const void* value, int32_t src_dtype,
                                 int64_t src_stride_tok, int64_t src_stride_head,
                                 const int32_t* slot_mapping, int32_t num_tokens, void* key_pool,
                                 void* value_pool, int32_t pool_dtype, int32_t n_kv_heads,
                                 int32_t num_blocks, int32_t block_size, int32_t head_dim,
                                 void* stream) {
  clear_error();
  if (int rc = check_pool_shape("edgerag_kv_append", n_kv_heads, num_blocks, block_size, head_dim))
    return rc;
  if (num_tokens < 0) return fail(EDGERAG_EINVAL, "edgerag_kv_append: num_tokens < 0");
  if (num_tokens == 0) return EDGERAG_OK;
  if (slot_mapping == nullptr) return fail(EDGERAG_EINVAL, "edgerag_kv_append: slot_mapping is NULL");
  if ((key == nullptr) != (key_pool == nullptr) || (value == nullptr) != (value_pool == nullptr)) {
    return fail(EDGERAG_EINVAL, "edgerag_kv_append: each source needs its pool and vice versa");
  }
  if (key == nullptr && value == nullptr) return EDGERAG_OK;
  auto s = static_cast<hipStream_t>(stream);
  switch (src_dtype) {
    case EDGERAG_F32:
      return dispatch_append_dst<float>(pool_dtype, key, value, src_stride_tok, src_stride_head,
                                        slot_mapping, num_tokens, key_pool, value_pool, n_kv_heads,
                                        num_blocks, block_size, head_dim, s);
    case EDGERAG_F16:
      return dispatch_append_dst<f16>(pool_dtype, key, value, src_stride_tok, src_stride_head,
                                      slot_mapping, num_tokens, key_pool, value_pool, n_kv_heads,
                                      num_blocks, block_size, head_dim, s);
    case EDGERAG_BF16:
      return dispatch_append_dst<bf16>(pool_dtype, key, value, src_stride_tok, src_stride_head,
                                       slot_mapping, num_tokens, key_pool, value_pool, n_kv_heads,
                                       num_blocks, block_size, head_dim, s);
  }
  return fail(EDGERAG_EINVAL, "edgerag_kv_append: unknown src dtype %d", src_dtype);
}

extern "C" int edgerag_kv_gather(const void* pool, int32_t dtype, int32_t n_kv_heads,
                                 int32_t num_blocks, int32_t block_size, int32_t head_dim,
                                 const int32_t* block_ids, int32_t seq_len, void* out,
                                 void* stream) {
  clear_error();
  if (int rc = check_pool_shape("edgerag_kv_gather", n_kv_heads, num_blocks, block_size, head_dim))
    return rc;
  if (seq_len < 0) return fail(EDGERAG_EINVAL, "edgerag_kv_gather: seq_len < 0");
  if (seq_len == 0) return EDGERAG_OK;
  if (pool == nullptr || out == nullptr || block_ids == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_kv_gather: NULL pointer");
  auto s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case EDGERAG_F32:
      return launch_gather<float>(pool, n_kv_heads, num_blocks, block_size, head_dim, block_ids,
                                  seq_len, out, s);
    case EDGERAG_F16:
      return launch_gather<f16>(pool, n_kv_heads, num_blocks, block_size, head_dim, block_ids,
                                seq_len, out, s);
    case EDGERAG_BF16:
      return launch_gather<bf16>(pool, n_kv_heads, num_blocks, block_size, head_dim, block_ids,
                                 seq_len, out, s);
  }
  return fail(EDGERAG_EINVAL, "edgerag_kv_gather: unknown dtype %d", dtype);
}

extern "C" int edgerag_kv_copy_blocks(void* pool, int32_t dtype, int32_t n_kv_heads,
                                      int32_t num_blocks, int32_t block_size, int32_t head_dim,
                                      const int32_t* src_blocks, const int32_t* dst_blocks,
                                      int32_t n_pairs, void* stream) {
  clear_error();
  if (int rc =
          check_pool_shape("edgerag_kv_copy_blocks", n_kv_heads, num_blocks, block_size, head_dim))
    return rc;
  const int es = elem_size(dtype);
  if (es == 0) return fail(EDGERAG_EINVAL, "edgerag_kv_copy_blocks: unknown dtype %d", dtype);
  if (n_pairs < 0) return fail(EDGERAG_EINVAL, "edgerag_kv_copy_blocks: n_pairs < 0");
  if (n_pairs == 0) return EDGERAG_OK;
  if (pool == nullptr || src_blocks == nullptr || dst_blocks == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_kv_copy_blocks: NULL pointer");
  auto s = static_cast<hipStream_t>(stream);
  const int64_t block_bytes = int64_t(block_size) * head_dim * es;
  if (block_bytes % 16 == 0 && aligned16(pool)) {
    const int64_t chunks = block_bytes / 16;
    hipLaunchKernelGGL(kv_copy_blocks16, dim3(grid_for(chunks * n_kv_heads * n_pairs)),
                       dim3(kThreads), 0, s, static_cast<Vec16*>(pool), n_kv_heads, num_blocks,
                       chunks, src_blocks, dst_blocks, n_pairs);
  } else {
    hipLaunchKernelGGL(kv_copy_blocks1, dim3(grid_for(block_bytes * n_kv_heads * n_pairs)),
                       dim3(kThreads), 0, s, static_cast<uint8_t*>(pool), n_kv_heads, num_blocks,
                       block_bytes, src_blocks, dst_blocks, n_pairs);
  }
  return check_launch("edgerag_kv_copy_blocks");
}
