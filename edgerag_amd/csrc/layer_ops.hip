// Fused elementwise ops around the hot path of one decoder layer, on packed token-major rows.
//
// * rmsnorm_kernel: optional residual add, then RMSNorm, one workgroup per row:
//     h = x (+ delta), rounded to T once like the reference's `hidden + attn_out`
//     y = weight * T(h * rsqrt(mean(h^2) + eps))   (edgerag/core/layers.py:40-47: fp32 variance,
//                                                   cast back before the weight multiply)
// * rope_append_kernel: the fused q/k/v projection output -> RoPE on q and k (halves convention,
//   out = T(T(x * cos) + T(rotate_half(x) * sin)), layers.py:93-114), q written token-major for
//   the attention kernel, post-RoPE k and raw v scattered into the paged pools by slot
//   (layers.py:301-306 -> paged.py:186-206). Same roundings as the reference's fp16 tensor ops.
// * silu_mul_kernel: SwiGLU's act = T(T(silu(gate)) * up) on the fused [gate | up] projection
//   (layers.py:341).
// All three are memory-bound and small (a few MB per step); their point is the launch count.
#include "common.h"

namespace edgerag {
namespace {

constexpr int kNormThreads = 256;

template <typename T>
__device__ __forceinline__ T round_to(float v) {
  return from_f32<T>(v);
}

// One workgroup per row. Each thread holds up to kPer elements of the row in registers.
template <typename T, int kPer>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(
    const T* __restrict__ x, const T* __restrict__ delta, const T* __restrict__ weight,
    int64_t x_stride, int64_t d_stride, int32_t width, float eps, T* __restrict__ h_out,
    T* __restrict__ y, int64_t h_stride, int64_t y_stride) {
#pragma clang fp contract(off)
  const int64_t row = blockIdx.x;
  const T* xr = x + row * x_stride;
  const T* dr = delta != nullptr ? delta + row * d_stride : nullptr;
  float v[kPer];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    float hv = 0.f;
    if (c < width) {
      hv = to_f32<T>(xr[c]);
      if (dr != nullptr) hv = to_f32<T>(round_to<T>(hv + to_f32<T>(dr[c])));
    }
    v[j] = hv;
    ss = fmaf(hv, hv, ss);
  }
  ss = xor_sum<0, 6>(ss);
  __shared__ float part[kNormThreads / kWave];
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = ss;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / kWave; ++w) total += part[w];
  const float r = rsqrtf(total / float(width) + eps);
  T* hr = h_out != nullptr ? h_out + row * h_stride : nullptr;
  T* yr = y + row * y_stride;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int c = threadIdx.x + j * kNormThreads;
    if (c < width) {
      if (hr != nullptr) hr[c] = round_to<T>(v[j]);
      const float nv = to_f32<T>(round_to<T>(v[j] * r));
      yr[c] = round_to<T>(to_f32<T>(weight[c]) * nv);
    }
  }
}

// Vector form for rows of 16-byte-aligned chunks (E = 16 / sizeof(T) elements): thread t owns
// chunks t, t + 256, ... of the row. Every load of the row (x, delta and weight) is issued before
// any is used, so a row costs one memory round trip; chunks past the row re-read its last chunk
// and are masked.
// The rotary table rows at each token's position (what edgerag_rope_rows writes), gathered by the
// embedding launch of a step: positions == NULL for none.
struct RopeRowsArgs {
  const int32_t* positions;
  const void* cos_t;
  const void* sin_t;
  int32_t max_pos, head_dim;
  void* cos_out;
  void* sin_out;
};

// ids != NULL (embedding lookup + the first RMSNorm): row r of x is table row ids[r], copied to
// h_out; an id outside [0, n_table) has no row: its h and y are written as NaN. rr.positions !=
// NULL: the workgroup of row r also writes row r of the rotary rows (a position outside the
// table gets a NaN row).
template <typename T, int NV>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_vec_kernel(
    const T* __restrict__ x, const int32_t* __restrict__ ids, int32_t n_table,
    const T* __restrict__ delta, const T* __restrict__ weight, int64_t x_stride,
    int64_t d_stride, int32_t width, float eps, T* __restrict__ h_out, T* __restrict__ y,
    int64_t h_stride, int64_t y_stride, const RopeRowsArgs rr) {
#pragma clang fp contract(off)
  constexpr int E = 16 / sizeof(T);
  const int64_t row = blockIdx.x;
  const int nch = width / E;
  if (rr.positions != nullptr && int(threadIdx.x) < rr.head_dim) {  // wave-uniform pointer test
    const int pos = rr.positions[row];
    const int dd = threadIdx.x;
    const bool ok = pos >= 0 && pos < rr.max_pos;
    const int64_t src = int64_t(ok ? pos : 0) * rr.head_dim + dd;
    const T c = ok ? static_cast<const T*>(rr.cos_t)[src] : round_to<T>(__builtin_nanf(""));
    const T sn = ok ? static_cast<const T*>(rr.sin_t)[src] : round_to<T>(__builtin_nanf(""));
    static_cast<T*>(rr.cos_out)[row * rr.head_dim + dd] = c;
    static_cast<T*>(rr.sin_out)[row * rr.head_dim + dd] = sn;
  }
  int64_t src = row;
  bool bad = false;
  if (ids != nullptr) {
    const int32_t id = ids[row];
    bad = id < 0 || id >= n_table;
    src = bad ? 0 : id;
  }
  const T* xr = x + src * x_stride;
  const T* dr = delta != nullptr ? delta + row * d_stride : nullptr;
  Vec16 xv[NV], dv[NV], wv[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int ch = min(int(threadIdx.x) + j * kNormThreads, nch - 1);
    xv[j] = load16(xr + ch * E);
    dv[j] = dr != nullptr ? load16(dr + ch * E) : Vec16{};
    wv[j] = load16(weight + ch * E);
  }
  // Consuming the loaded words here keeps the compiler from moving any load below the reduction.
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      asm volatile("" : "+v"(xv[j].w[q]), "+v"(dv[j].w[q]), "+v"(wv[j].w[q]));
  float h[NV][E];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const bool in = int(threadIdx.x) + j * kNormThreads < nch;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      float hv = vec_elem<T>(xv[j], e);
      if (dr != nullptr) hv = to_f32<T>(round_to<T>(hv + vec_elem<T>(dv[j], e)));
      h[j][e] = in ? hv : 0.f;
      ss = fmaf(h[j][e], h[j][e], ss);
    }
  }
  ss = xor_sum<0, 6>(ss);
  __shared__ float part[kNormThreads / kWave];
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = ss;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / kWave; ++w) total += part[w];
  const float r = rsqrtf(total / float(width) + eps);
  T* hr = h_out != nullptr ? h_out + row * h_stride : nullptr;
  T* yr = y + row * y_stride;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int ch = int(threadIdx.x) + j * kNormThreads;
    if (ch >= nch) continue;
    T ho[E], yo[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
      ho[e] = round_to<T>(bad ? __builtin_nanf("") : h[j][e]);
      const float nv = to_f32<T>(round_to<T>(h[j][e] * r));
      yo[e] = round_to<T>(bad ? __builtin_nanf("") : vec_elem<T>(wv[j], e) * nv);
    }
    if (hr != nullptr) store16(hr + ch * E, *reinterpret_cast<const Vec16*>(ho));
    store16(yr + ch * E, *reinterpret_cast<const Vec16*>(yo));
  }
}

// out[p] = x1 cos[p] + (-x2) sin[p]; out[p + half] = x2 cos[p + half] + x1 sin[p + half].
// No contraction: each product is rounded before the add, like the reference's separate tensor
// ops, also on the fp32 path.
template <typename T>
__device__ __forceinline__ void rotate_pair(float x1, float x2, const T* __restrict__ cr,
                                            const T* __restrict__ sr, int p, int half, T& o1,
                                            T& o2) {
#pragma clang fp contract(off)
  const float a1 = to_f32<T>(round_to<T>(x1 * to_f32<T>(cr[p])));
  const float b1 = to_f32<T>(round_to<T>(-x2 * to_f32<T>(sr[p])));
  const float a2 = to_f32<T>(round_to<T>(x2 * to_f32<T>(cr[p + half])));
  const float b2 = to_f32<T>(round_to<T>(x1 * to_f32<T>(sr[p + half])));
  o1 = round_to<T>(a1 + b1);
  o2 = round_to<T>(a2 + b2);
}

// One thread per (token, head, pair i in [0, d/2)) of the q, k and v heads of the fused
// projection row [q heads | k heads | v heads].
template <typename T>
__global__ __launch_bounds__(256) void rope_append_kernel(
    const T* __restrict__ qkv, int64_t qkv_stride, const int32_t* __restrict__ positions,
    const T* __restrict__ cos_t, const T* __restrict__ sin_t, int32_t max_pos, int32_t n_tokens,
    int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim, T* __restrict__ q_out,
    int64_t q_stride_tok, const int32_t* __restrict__ slots, T* __restrict__ kpool,
    T* __restrict__ vpool, int32_t num_blocks, int32_t block_size) {
#pragma clang fp contract(off)
  const int half = head_dim / 2;
  const int heads = n_q_heads + 2 * n_kv_heads;
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= int64_t(n_tokens) * heads * half) return;
  const int p = int(i % half);
  const int64_t th = i / half;
  const int hd = int(th % heads);
  const int t = int(th / heads);
  const T* src = qkv + int64_t(t) * qkv_stride + int64_t(hd) * head_dim;
  const float x1 = to_f32<T>(src[p]), x2 = to_f32<T>(src[p + half]);
  if (hd >= n_q_heads + n_kv_heads) {  // v: copied as is
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= int64_t(num_blocks) * block_size) return;
    const int h = hd - n_q_heads - n_kv_heads;
    T* dst = vpool + ((int64_t(h) * num_blocks + slot / block_size) * block_size +
                      slot % block_size) * head_dim;
    dst[p] = src[p];
    dst[p + half] = src[p + half];
    return;
  }
  const int pos = positions[t];
  T o1, o2;
  if (pos < 0 || pos >= max_pos) {
    // No table row: the token's q and k become NaN, so a caller whose table is too short sees
    // it in the logits instead of getting another position's rotation.
    o1 = o2 = round_to<T>(__builtin_nanf(""));
  } else {
    rotate_pair<T>(x1, x2, cos_t + int64_t(pos) * head_dim, sin_t + int64_t(pos) * head_dim, p,
                   half, o1, o2);
  }
  if (hd < n_q_heads) {
    T* dst = q_out + int64_t(t) * q_stride_tok + int64_t(hd) * head_dim;
    dst[p] = o1;
    dst[p + half] = o2;
  } else {
    const int64_t slot = slots[t];
    if (slot < 0 || slot >= int64_t(num_blocks) * block_size) return;
    const int h = hd - n_q_heads;
    T* dst = kpool + ((int64_t(h) * num_blocks + slot / block_size) * block_size +
                      slot % block_size) * head_dim;
    dst[p] = o1;
    dst[p + half] = o2;
  }
}

template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(const T* __restrict__ gu, int64_t gu_stride,
                                                       int32_t n_tokens, int32_t inter,
                                                       T* __restrict__ out, int64_t out_stride) {
#pragma clang fp contract(off)
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= int64_t(n_tokens) * inter) return;
  const int64_t t = i / inter;
  const int c = int(i % inter);
  const float g = to_f32<T>(gu[t * gu_stride + c]);
  const float u = to_f32<T>(gu[t * gu_stride + inter + c]);
  const float s = to_f32<T>(round_to<T>(g / (1.f + expf(-g))));
  out[t * out_stride + c] = round_to<T>(s * u);
}

// Vector form: one thread per 16-byte chunk of the intermediate width (both halves loaded
// before either is used).
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_vec_kernel(const T* __restrict__ gu,
                                                           int64_t gu_stride, int32_t n_tokens,
                                                           int32_t inter, T* __restrict__ out,
                                                           int64_t out_stride) {
#pragma clang fp contract(off)
  constexpr int E = 16 / sizeof(T);
  const int nch = inter / E;
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= int64_t(n_tokens) * nch) return;
  const int64_t t = i / nch;
  const int c = int(i % nch) * E;
  const Vec16 gv = load16(gu + t * gu_stride + c);
  const Vec16 uv = load16(gu + t * gu_stride + inter + c);
  T o[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float g = vec_elem<T>(gv, e);
    const float sv = to_f32<T>(round_to<T>(g / (1.f + expf(-g))));
    o[e] = round_to<T>(sv * vec_elem<T>(uv, e));
  }
  store16(out + t * out_stride + c, *reinterpret_cast<const Vec16*>(o));
}

inline bool aligned_rows(const void* p, int64_t stride_elems, int elem_size) {
  return p == nullptr || (aligned16(p) && (stride_elems * elem_size) % 16 == 0);
}

template <typename T>
int launch_rmsnorm(const void* x, const void* delta, const void* weight, void* h_out, void* y,
                   int32_t rows, int32_t width, int64_t xs, int64_t ds, int64_t hs, int64_t ys,
                   float eps, hipStream_t s, const int32_t* ids = nullptr, int32_t n_table = 0,
                   const RopeRowsArgs& rr = RopeRowsArgs{}) {
  constexpr int E = 16 / sizeof(T);
  const int nch = width / E;
  if (width % E == 0 && aligned_rows(x, xs, sizeof(T)) && aligned_rows(delta, ds, sizeof(T)) &&
      aligned_rows(weight, 0, sizeof(T)) && aligned_rows(h_out, hs, sizeof(T)) &&
      aligned_rows(y, ys, sizeof(T)) && nch <= 8 * kNormThreads) {
    const int nv = (nch + kNormThreads - 1) / kNormThreads;
#define EDGERAG_NORMV(NV)                                                                       \
  hipLaunchKernelGGL((rmsnorm_vec_kernel<T, NV>), dim3(rows), dim3(kNormThreads), 0, s,         \
                     static_cast<const T*>(x), ids, n_table, static_cast<const T*>(delta),      \
                     static_cast<const T*>(weight), xs, ds, width, eps,                         \
                     static_cast<T*>(h_out), static_cast<T*>(y), hs, ys, rr)
    if (nv <= 1) EDGERAG_NORMV(1);
    else if (nv <= 2) EDGERAG_NORMV(2);
    else if (nv <= 4) EDGERAG_NORMV(4);
    else EDGERAG_NORMV(8);
#undef EDGERAG_NORMV
    return check_launch("edgerag_rmsnorm");
  }
  if (ids != nullptr || rr.positions != nullptr)
    return fail(EDGERAG_EUNSUPPORTED, "edgerag_embed_rmsnorm: rows of %d elements not in "
                "16-byte chunks (or above 8 x %d chunks)", width, kNormThreads);
  const int per = (width + kNormThreads - 1) / kNormThreads;
#define EDGERAG_NORM(P)                                                                         \
  hipLaunchKernelGGL((rmsnorm_kernel<T, P>), dim3(rows), dim3(kNormThreads), 0, s,              \
                     static_cast<const T*>(x), static_cast<const T*>(delta),                    \
                     static_cast<const T*>(weight), xs, ds, width, eps,                         \
                     static_cast<T*>(h_out), static_cast<T*>(y), hs, ys)
  if (per <= 4) EDGERAG_NORM(4);
  else if (per <= 8) EDGERAG_NORM(8);
  else if (per <= 16) EDGERAG_NORM(16);
  else if (per <= 32) EDGERAG_NORM(32);
  else return fail(EDGERAG_EUNSUPPORTED, "edgerag_rmsnorm: width %d above 8192", width);
#undef EDGERAG_NORM
  return check_launch("edgerag_rmsnorm");
}

// Greedy token choice: out[r] = argmax_j x[r][j], the first index of the maximum (torch.argmax's
// choice; a NaN counts as larger than every number, and the first NaN wins). One 1024-thread
// workgroup per row, 16-byte loads when the row allows them; lanes, then waves, reduce
// (value, index) pairs with the same rule.
__device__ __forceinline__ bool argmax_better(float v, int i, float bv, int bi) {
  if (v != v) return bv == bv || i < bi;  // NaN
  if (bv != bv) return false;
  return v > bv || (v == bv && i < bi);
}

template <typename T>
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const T* __restrict__ x, int64_t stride,
                                                           int32_t cols, bool vec,
                                                           int32_t* __restrict__ out) {
  constexpr int VEC = 16 / int(sizeof(T));
  const T* row = x + int64_t(blockIdx.x) * stride;
  float bv = -INFINITY;
  int bi = INT32_MAX;
  if (vec) {
    for (int j = int(threadIdx.x) * VEC; j < cols; j += 1024 * VEC) {
      const uint4 raw = *reinterpret_cast<const uint4*>(row + j);
      const T* e = reinterpret_cast<const T*>(&raw);
#pragma unroll
      for (int q = 0; q < VEC; ++q) {
        const float v = to_f32<T>(e[q]);
        if (argmax_better(v, j + q, bv, bi)) {
          bv = v;
          bi = j + q;
        }
      }
    }
  } else {
    for (int j = int(threadIdx.x); j < cols; j += 1024) {
      const float v = to_f32<T>(row[j]);
      if (argmax_better(v, j, bv, bi)) {
        bv = v;
        bi = j;
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) {
    const float ov = __shfl_xor(bv, off);
    const int oi = __shfl_xor(bi, off);
    if (argmax_better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __shared__ float wv[16];
  __shared__ int wi[16];
  const int wave = int(threadIdx.x) / kWave;
  if (threadIdx.x % kWave == 0) {
    wv[wave] = bv;
    wi[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; ++w)
      if (argmax_better(wv[w], wi[w], bv, bi)) {
        bv = wv[w];
        bi = wi[w];
      }
    out[blockIdx.x] = bi;
  }
}

}  // namespace
}  // namespace edgerag

using namespace edgerag;

extern "C" int edgerag_rmsnorm(const void* x, int64_t x_stride, const void* delta,
                               int64_t delta_stride, const void* weight, void* h_out,
                               int64_t h_stride, void* y, int64_t y_stride, int32_t rows,
                               int32_t width, float eps, int32_t dtype, void* stream) {
  clear_error();
  if (rows < 0 || width <= 0) return fail(EDGERAG_EINVAL, "edgerag_rmsnorm: rows %d width %d", rows, width);
  if (rows == 0) return EDGERAG_OK;
  if (x == nullptr || weight == nullptr || y == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_rmsnorm: NULL pointer");
  if (delta != nullptr && h_out == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_rmsnorm: a residual add needs h_out");
  auto s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case EDGERAG_F32: return launch_rmsnorm<float>(x, delta, weight, h_out, y, rows, width, x_stride, delta_stride, h_stride, y_stride, eps, s);
    case EDGERAG_F16: return launch_rmsnorm<f16>(x, delta, weight, h_out, y, rows, width, x_stride, delta_stride, h_stride, y_stride, eps, s);
    case EDGERAG_BF16: return launch_rmsnorm<bf16>(x, delta, weight, h_out, y, rows, width, x_stride, delta_stride, h_stride, y_stride, eps, s);
  }
  return fail(EDGERAG_EINVAL, "edgerag_rmsnorm: dtype %d", dtype);
}

extern "C" int edgerag_embed_rmsnorm(const int32_t* ids, int32_t rows, const void* table,
                                     int64_t table_stride, int32_t vocab, const void* weight,
                                     void* h_out, int64_t h_stride, void* y, int64_t y_stride,
                                     int32_t width, float eps, const int32_t* positions,
                                     const void* cos_table, const void* sin_table,
                                     int32_t max_pos, int32_t head_dim, void* cos_out,
                                     void* sin_out, int32_t dtype, void* stream) {
  clear_error();
  if (rows < 0 || width <= 0 || vocab <= 0)
    return fail(EDGERAG_EINVAL, "edgerag_embed_rmsnorm: rows %d width %d vocab %d", rows, width,
                vocab);
  if (rows == 0) return EDGERAG_OK;
  if (ids == nullptr || table == nullptr || weight == nullptr || h_out == nullptr || y == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_embed_rmsnorm: NULL pointer");
  const RopeRowsArgs rr{positions, cos_table, sin_table, max_pos, head_dim, cos_out, sin_out};
  if (positions != nullptr &&
      (cos_table == nullptr || sin_table == nullptr || cos_out == nullptr || sin_out == nullptr ||
       max_pos <= 0 || head_dim <= 0 || head_dim > kNormThreads))
    return fail(EDGERAG_EINVAL, "edgerag_embed_rmsnorm: rotary rows need both tables, both "
                "outputs, max_pos > 0 and 0 < head_dim <= %d", kNormThreads);
  auto s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case EDGERAG_F32: return launch_rmsnorm<float>(table, nullptr, weight, h_out, y, rows, width, table_stride, 0, h_stride, y_stride, eps, s, ids, vocab, rr);
    case EDGERAG_F16: return launch_rmsnorm<f16>(table, nullptr, weight, h_out, y, rows, width, table_stride, 0, h_stride, y_stride, eps, s, ids, vocab, rr);
    case EDGERAG_BF16: return launch_rmsnorm<bf16>(table, nullptr, weight, h_out, y, rows, width, table_stride, 0, h_stride, y_stride, eps, s, ids, vocab, rr);
  }
  return fail(EDGERAG_EINVAL, "edgerag_embed_rmsnorm: dtype %d", dtype);
}

extern "C" int edgerag_rope_append(const void* qkv, int64_t qkv_stride, const int32_t* positions,
                                   const void* cos_table, const void* sin_table, int32_t max_pos,
                                   int32_t n_tokens, int32_t n_q_heads, int32_t n_kv_heads,
                                   int32_t head_dim, void* q_out, int64_t q_stride_tok,
                                   const int32_t* slots, void* key_pool, void* value_pool,
                                   int32_t num_blocks, int32_t block_size, int32_t dtype,
                                   void* stream) {
  clear_error();
  if (n_tokens < 0 || n_q_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim % 2 ||
      max_pos <= 0 || num_blocks <= 0 || block_size <= 0)
    return fail(EDGERAG_EINVAL, "edgerag_rope_append: bad shape");
  if (n_tokens == 0) return EDGERAG_OK;
  if (qkv == nullptr || positions == nullptr || cos_table == nullptr || sin_table == nullptr ||
      q_out == nullptr || slots == nullptr || key_pool == nullptr || value_pool == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_rope_append: NULL pointer");
  const int64_t total = int64_t(n_tokens) * (n_q_heads + 2 * n_kv_heads) * (head_dim / 2);
  const dim3 grid(unsigned((total + 255) / 256)), block(256);
  auto s = static_cast<hipStream_t>(stream);
#define EDGERAG_ROPE(TYPE)                                                                      \
  hipLaunchKernelGGL((rope_append_kernel<TYPE>), grid, block, 0, s,                             \
                     static_cast<const TYPE*>(qkv), qkv_stride, positions,                     \
                     static_cast<const TYPE*>(cos_table), static_cast<const TYPE*>(sin_table), \
                     max_pos, n_tokens, n_q_heads, n_kv_heads, head_dim,                       \
                     static_cast<TYPE*>(q_out), q_stride_tok, slots,                           \
                     static_cast<TYPE*>(key_pool), static_cast<TYPE*>(value_pool), num_blocks,  \
                     block_size)
  switch (dtype) {
    case EDGERAG_F32: EDGERAG_ROPE(float); break;
    case EDGERAG_F16: EDGERAG_ROPE(f16); break;
    case EDGERAG_BF16: EDGERAG_ROPE(bf16); break;
    default: return fail(EDGERAG_EINVAL, "edgerag_rope_append: dtype %d", dtype);
  }
#undef EDGERAG_ROPE
  return check_launch("edgerag_rope_append");
}

// One thread per (token, 2-byte element) of the per-token cos / sin rows: the table row at the
// token's position, or NaN where the position has no row.
template <typename T>
__global__ __launch_bounds__(256) void rope_rows_kernel(const int32_t* __restrict__ positions,
                                                        int32_t n_tokens,
                                                        const T* __restrict__ cos_t,
                                                        const T* __restrict__ sin_t,
                                                        int32_t max_pos, int32_t head_dim,
                                                        T* __restrict__ cos_out,
                                                        T* __restrict__ sin_out) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= int64_t(n_tokens) * head_dim) return;
  const int t = int(i / head_dim), d = int(i % head_dim);
  const int pos = positions[t];
  T c, s;
  if (pos < 0 || pos >= max_pos) {
    c = s = round_to<T>(__builtin_nanf(""));
  } else {
    c = cos_t[int64_t(pos) * head_dim + d];
    s = sin_t[int64_t(pos) * head_dim + d];
  }
  cos_out[i] = c;
  sin_out[i] = s;
}

extern "C" int edgerag_rope_rows(const int32_t* positions, int32_t n_tokens,
                                 const void* cos_table, const void* sin_table, int32_t max_pos,
                                 int32_t head_dim, int32_t dtype, void* cos_out, void* sin_out,
                                 void* stream) {
  clear_error();
  if (n_tokens < 0 || max_pos <= 0 || head_dim <= 0)
    return fail(EDGERAG_EINVAL, "edgerag_rope_rows: bad shape");
  if (n_tokens == 0) return EDGERAG_OK;
  if (positions == nullptr || cos_table == nullptr || sin_table == nullptr ||
      cos_out == nullptr || sin_out == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_rope_rows: NULL pointer");
  const int64_t total = int64_t(n_tokens) * head_dim;
  const dim3 grid(unsigned((total + 255) / 256)), block(256);
  auto s = static_cast<hipStream_t>(stream);
#define EDGERAG_ROPE_ROWS(TYPE)                                                                  \
  hipLaunchKernelGGL((rope_rows_kernel<TYPE>), grid, block, 0, s, positions, n_tokens,          \
                     static_cast<const TYPE*>(cos_table), static_cast<const TYPE*>(sin_table), \
                     max_pos, head_dim, static_cast<TYPE*>(cos_out), static_cast<TYPE*>(sin_out))
  switch (dtype) {
    case EDGERAG_F32: EDGERAG_ROPE_ROWS(float); break;
    case EDGERAG_F16: EDGERAG_ROPE_ROWS(f16); break;
    case EDGERAG_BF16: EDGERAG_ROPE_ROWS(bf16); break;
    default: return fail(EDGERAG_EINVAL, "edgerag_rope_rows: dtype %d", dtype);
  }
#undef EDGERAG_ROPE_ROWS
  return check_launch("edgerag_rope_rows");
}

extern "C" int edgerag_silu_mul(const void* gate_up, int64_t gate_up_stride, int32_t n_tokens,
                                int32_t intermediate, void* out, int64_t out_stride,
                                int32_t dtype, void* stream) {
  clear_error();
  if (n_tokens < 0 || intermediate <= 0)
    return fail(EDGERAG_EINVAL, "edgerag_silu_mul: bad shape");
  if (n_tokens == 0) return EDGERAG_OK;
  if (gate_up == nullptr || out == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_silu_mul: NULL pointer");
  const int es = dtype == EDGERAG_F32 ? 4 : 2;
  const bool vec = (intermediate * es) % 16 == 0 && aligned_rows(gate_up, gate_up_stride, es) &&
                   aligned_rows(out, out_stride, es);
  const int64_t total = int64_t(n_tokens) * (vec ? intermediate * es / 16 : intermediate);
  const dim3 grid(unsigned((total + 255) / 256)), block(256);
  auto s = static_cast<hipStream_t>(stream);
#define EDGERAG_SILU(TYPE)                                                                      \
  if (vec)                                                                                     \
    hipLaunchKernelGGL((silu_mul_vec_kernel<TYPE>), grid, block, 0, s,                          \
                       static_cast<const TYPE*>(gate_up), gate_up_stride, n_tokens,             \
                       intermediate, static_cast<TYPE*>(out), out_stride);                      \
  else                                                                                         \
    hipLaunchKernelGGL((silu_mul_kernel<TYPE>), grid, block, 0, s,                              \
                       static_cast<const TYPE*>(gate_up), gate_up_stride, n_tokens,             \
                       intermediate, static_cast<TYPE*>(out), out_stride)
  switch (dtype) {
    case EDGERAG_F32: EDGERAG_SILU(float); break;
    case EDGERAG_F16: EDGERAG_SILU(f16); break;
    case EDGERAG_BF16: EDGERAG_SILU(bf16); break;
    default: return fail(EDGERAG_EINVAL, "edgerag_silu_mul: dtype %d", dtype);
  }
#undef EDGERAG_SILU
  return check_launch("edgerag_silu_mul");
}

extern "C" int edgerag_argmax_rows(const void* x, int32_t dtype, int32_t rows, int32_t cols,
                                   int64_t row_stride, int32_t* out, void* stream) {
  clear_error();
  if (rows < 0 || cols <= 0 || row_stride < cols)
    return fail(EDGERAG_EINVAL, "edgerag_argmax_rows: bad shape (%d x %d, stride %lld)", rows, cols,
                (long long)row_stride);
  if (rows == 0) return EDGERAG_OK;
  if (x == nullptr || out == nullptr) return fail(EDGERAG_EINVAL, "edgerag_argmax_rows: NULL pointer");
  const int es = dtype == EDGERAG_F32 ? 4 : 2;
  const bool vec = (cols * es) % 16 == 0 && aligned_rows(x, row_stride, es);
  auto s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case EDGERAG_F32:
      hipLaunchKernelGGL((argmax_rows_kernel<float>), dim3(unsigned(rows)), dim3(1024), 0, s,
                         static_cast<const float*>(x), row_stride, cols, vec, out);
      break;
    case EDGERAG_F16:
      hipLaunchKernelGGL((argmax_rows_kernel<f16>), dim3(unsigned(rows)), dim3(1024), 0, s,
                         static_cast<const f16*>(x), row_stride, cols, vec, out);
      break;
    case EDGERAG_BF16:
      hipLaunchKernelGGL((argmax_rows_kernel<bf16>), dim3(unsigned(rows)), dim3(1024), 0, s,
                         static_cast<const bf16*>(x), row_stride, cols, vec, out);
      break;
    default: return fail(EDGERAG_EINVAL, "edgerag_argmax_rows: dtype %d", dtype);
  }
  return check_launch("edgerag_argmax_rows");
}
