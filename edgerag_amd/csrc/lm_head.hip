// The decoder's output head for the emitting rows of a step: logits = x . W^T with the fp16
// lm_head weight W [V, K] (no quantisation: the reference keeps lm_head fp16, linear.py:229-241),
// and each row's greedy token, argmax over the fp16 logits with torch.argmax's rule (first index
// of the maximum, a NaN counting as the maximum). Replaces F.linear(hidden, lm_head)
// (edgerag/core/model.py:150-152) and the executor's argmax (edgerag/serve/executor.py:136, :154).
//
// lm_head_kernel streams W once at HBM rate (201 MB for SmolLM2's 49152 x 2048):
// * a workgroup owns 16 consecutive vocabulary rows per wave, each wave over all of K;
// * the M <= 16 activation rows are staged in LDS once per workgroup (row stride 2K + 16 bytes,
//   so the 16-byte reads of 8 tokens hit distinct banks), not re-read from L2 per wave;
// * per 32-k step a lane loads 16 bytes of its weight row (4 lanes cover 64 contiguous bytes) and
//   feeds them straight to v_mfma_f32_16x16x32_f16 as the A operand, the activations from LDS as
//   B; U steps of loads are issued before any is consumed;
// * the epilogue rounds the fp32 sums to fp16 (the logits, as F.linear writes them), and reduces
//   the workgroup's candidates per token to one 64-bit key (ordered fp16 value << 32 | ~index),
//   written to a workspace slot of its own: no atomics, no cross-workgroup ordering.
// lm_head_pick_kernel takes the maximum key of each token's workgroup slots: its token id.
#include "common.h"

namespace edgerag {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kLmMaxM = 16;
// Launch shapes (waves per workgroup, 32-k steps of weight loads in flight per lane), measured on
// the 49152 x 2048 head: up to 8 rows, 4-wave workgroups (3 per CU) 16 steps deep; 9..16 rows
// stage twice the activations in LDS, and 12-wave workgroups (one per CU) 8 deep do better.
constexpr int kLmSmallWaves = 4, kLmSmallU = 16;
constexpr int kLmLargeWaves = 12, kLmLargeU = 8;
constexpr int kLmSmallM = 8;

__device__ __forceinline__ uint4 ldg16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// Order-preserving 16-bit key of an fp16 value: larger value -> larger key, -0 == +0, and every
// NaN above +inf (torch.argmax returns the first NaN).
__device__ __forceinline__ uint32_t ordered_key(uint16_t b) {
  if ((b & 0x7FFFu) > 0x7C00u) return 0xFFFFu;  // NaN
  if (b == 0x8000u) b = 0;                       // -0 -> +0
  return (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
}

__device__ __forceinline__ uint64_t key_max(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int mask) {
  const uint32_t lo = __shfl_xor(uint32_t(v), mask, kWave);
  const uint32_t hi = __shfl_xor(uint32_t(v >> 32), mask, kWave);
  return (uint64_t(hi) << 32) | lo;
}

template <int WAVES, int U, int R>
__global__ __launch_bounds__(WAVES * kWave) void lm_head_kernel(
    const f16* __restrict__ x, int64_t xs, int32_t m, int32_t k, const f16* __restrict__ w,
    int32_t v, f16* __restrict__ logits, int64_t ls, uint64_t* __restrict__ part) {
  extern __shared__ uint4 xt[];  // m rows of k fp16 each, row stride k / 8 + 1 uint4
  __shared__ uint64_t best[WAVES][kLmMaxM];
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int row0 = int(blockIdx.x) * (16 * WAVES) + wave * 16;
  const int row = min(row0 + li, v - 1);  // rows past V re-read the last one (never written)
  const int steps = k / 32;
  const int xrow = (k >> 3) + 1;  // uint4 per staged activation row

  // Weight row `row`, k chunk (step, lg): 16 bytes at element 32 step + 8 lg.
  const uint4* wp = reinterpret_cast<const uint4*>(w + int64_t(row) * k) + lg;
  // Staging the m x k/8 16-byte activation chunks. With R > 0 (at most R rows), thread c loads
  // chunk c of every row, then issues the first batch of weight loads, then stores the chunks to
  // LDS: the stores wait only for the activation loads (L2 hits, issued first) while the weight
  // loads stay in flight. Up to 8 rows this took the launch from 44.3 / 47.0 to 43.0-43.9 /
  // 44.8-44.9 us (1 / 8 rows), where a loop of load -> store per chunk waited out a round trip
  // per chunk, the first behind the weights. The 12-wave launch for 9..16 rows keeps that loop
  // (R = 0): staging 16 rows at once cost it its second workgroup per CU (108 VGPRs), and smaller
  // batches measured 48.9-49.9 against 47.7 us.
  const int chunks = k >> 3, nth = WAVES * kWave;
  uint4 wb[U];
  if constexpr (R == 0) {
#pragma unroll
    for (int u = 0; u < U; ++u) wb[u] = ldg16(wp + 4 * min(u, steps - 1));
    for (int i = threadIdx.x; i < m * chunks; i += nth)
      xt[(i / chunks) * xrow + i % chunks] = ldg16(x + int64_t(i / chunks) * xs + 8 * (i % chunks));
  } else {
    // Loads without branches: rows past m re-read row m - 1 and chunks past the row re-read its
    // last chunk (L2 hits); only the stores are guarded.
    const int c = threadIdx.x, cc = min(c, chunks - 1);
    uint4 xr[R];
#pragma unroll
    for (int t = 0; t < R; ++t) xr[t] = ldg16(x + int64_t(min(t, m - 1)) * xs + 8 * cc);
#pragma unroll
    for (int u = 0; u < U; ++u) wb[u] = ldg16(wp + 4 * min(u, steps - 1));
#pragma unroll
    for (int t = 0; t < R; ++t)
      if (t < m && c < chunks) xt[t * xrow + c] = xr[t];
    for (int i = c + nth; i < chunks; i += nth)  // K past 8 x threads
      for (int t = 0; t < m; ++t) xt[t * xrow + i] = ldg16(x + int64_t(t) * xs + 8 * i);
  }
  __syncthreads();

  const uint4* xp = xt + min(li, m - 1) * xrow + lg;  // token li (clamped), same k chunk
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < steps; s0 += U) {
    uint4 wn[U];
    const bool more = s0 + U < steps;
    if (more) {
#pragma unroll
      for (int u = 0; u < U; ++u) wn[u] = ldg16(wp + 4 * min(s0 + U + u, steps - 1));
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (s0 + u < steps) {
        const uint4 xa = xp[4 * (s0 + u)];
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, wb[u]),
                                                     __builtin_bit_cast(h8, xa), acc, 0, 0, 0);
      }
    }
    if (more) {
#pragma unroll
      for (int u = 0; u < U; ++u) wb[u] = wn[u];
    }
  }

  // D[r][j]: register i of lane l is vocabulary row row0 + 4 (l / 16) + i, token l % 16.
  const int tok = li;
  uint64_t key = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int vr = row0 + 4 * lg + i;
    const f16 h = __float2half_rn(acc[i]);
    if (tok < m && vr < v) {
      if (logits != nullptr) logits[int64_t(tok) * ls + vr] = h;
      const uint64_t kk = (uint64_t(ordered_key(__builtin_bit_cast(uint16_t, h))) << 32) |
                          uint64_t(0xFFFFFFFFu - uint32_t(vr));
      key = key_max(key, kk);
    }
  }
  key = key_max(key, shfl_xor_u64(key, 16));
  key = key_max(key, shfl_xor_u64(key, 32));
  if (lg == 0) best[wave][tok] = key;
  __syncthreads();
  if (threadIdx.x < unsigned(m)) {
    uint64_t b = best[0][threadIdx.x];
#pragma unroll
    for (int wv = 1; wv < WAVES; ++wv) b = key_max(b, best[wv][threadIdx.x]);
    part[int64_t(threadIdx.x) * gridDim.x + blockIdx.x] = b;
  }
}

__global__ __launch_bounds__(256) void lm_head_pick_kernel(const uint64_t* __restrict__ part,
                                                           int32_t n_part,
                                                           int32_t* __restrict__ tokens) {
  __shared__ uint64_t red[256 / kWave];
  const uint64_t* p = part + int64_t(blockIdx.x) * n_part;
  uint64_t b = 0;
  for (int i = threadIdx.x; i < n_part; i += 256) b = key_max(b, p[i]);
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) b = key_max(b, shfl_xor_u64(b, o));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = b;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 256 / kWave; ++i) b = key_max(b, red[i]);
    b = key_max(red[0], b);
    tokens[blockIdx.x] = int32_t(0xFFFFFFFFu - uint32_t(b & 0xFFFFFFFFu));
  }
}

int lm_head_workgroups(int32_t vocab, int waves) {
  return (vocab + 16 * waves - 1) / (16 * waves);
}

}  // namespace
}  // namespace edgerag

using namespace edgerag;

extern "C" int64_t edgerag_lm_head_workspace_bytes(int32_t m, int32_t vocab) {
  if (m < 1 || m > kLmMaxM || vocab < 1) return 0;
  // Sized for the launch shape with the most workgroups.
  return int64_t(m) * lm_head_workgroups(vocab, kLmSmallWaves) * int64_t(sizeof(uint64_t));
}

// Rows of k fp16 values staged in LDS, one 16-byte chunk of padding per row.
static size_t lm_head_stage_bytes(int32_t m, int32_t k) {
  return size_t(m) * (size_t(k / 8) + 1) * sizeof(uint4);
}
static constexpr size_t kLmStageMax = 128 * 1024;  // of the CU's 160 KiB

extern "C" int edgerag_lm_head_argmax_supported(int32_t m, int32_t k) {
  return m >= 1 && m <= kLmMaxM && k >= 32 && k % 32 == 0 &&
         lm_head_stage_bytes(m, k) <= kLmStageMax;
}

extern "C" int edgerag_lm_head_argmax(const void* x, int64_t x_stride, int32_t m, int32_t k,
                                      const void* weight, int32_t vocab, void* logits,
                                      int64_t logits_stride, int32_t* tokens, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
  clear_error();
  if (m < 1 || m > kLmMaxM)
    return fail(EDGERAG_EUNSUPPORTED, "edgerag_lm_head_argmax: %d rows (1..%d)", m, kLmMaxM);
  if (k < 32 || k % 32 != 0 || vocab < 1 || x_stride < k ||
      (logits != nullptr && logits_stride < vocab))
    return fail(EDGERAG_EINVAL, "edgerag_lm_head_argmax: bad shape (m %d, k %d, vocab %d)", m, k,
                vocab);
  if (x == nullptr || weight == nullptr || tokens == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_lm_head_argmax: NULL pointer");
  if (!aligned16(x) || !aligned16(weight) || (x_stride * 2) % 16 != 0)
    return fail(EDGERAG_EINVAL, "edgerag_lm_head_argmax: x rows and the weight must be 16-byte "
                                "aligned");
  const int64_t need = edgerag_lm_head_workspace_bytes(m, vocab);
  if (workspace == nullptr || workspace_bytes < need ||
      (reinterpret_cast<uintptr_t>(workspace) & 7u) != 0)
    return fail(EDGERAG_EWORKSPACE, "edgerag_lm_head_argmax: workspace %lld bytes, need %lld "
                                    "(8-byte aligned)",
                (long long)workspace_bytes, (long long)need);
  const size_t lds = lm_head_stage_bytes(m, k);
  if (lds > kLmStageMax)
    return fail(EDGERAG_EUNSUPPORTED, "edgerag_lm_head_argmax: %d rows of %d exceed the staging "
                                      "space", m, k);
  const bool small = m <= kLmSmallM;
  const int wgs = lm_head_workgroups(vocab, small ? kLmSmallWaves : kLmLargeWaves);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const f16* xh = static_cast<const f16*>(x);
  const f16* wh = static_cast<const f16*>(weight);
  f16* lh = static_cast<f16*>(logits);
  uint64_t* part = static_cast<uint64_t*>(workspace);
  if (small)
    hipLaunchKernelGGL((lm_head_kernel<kLmSmallWaves, kLmSmallU, kLmSmallM>), dim3(wgs),
                       dim3(kLmSmallWaves * kWave), lds, s, xh, x_stride, m, k, wh, vocab, lh,
                       logits_stride, part);
  else
    hipLaunchKernelGGL((lm_head_kernel<kLmLargeWaves, kLmLargeU, 0>), dim3(wgs),
                       dim3(kLmLargeWaves * kWave), lds, s, xh, x_stride, m, k, wh, vocab, lh,
                       logits_stride, part);
  hipLaunchKernelGGL(lm_head_pick_kernel, dim3(m), dim3(256), 0, s,
                     static_cast<const uint64_t*>(workspace), wgs, tokens);
  return check_launch("edgerag_lm_head_argmax");
}
