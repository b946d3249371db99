// Weight-only INT8 / INT4 linear layers on CDNA4 matrix cores (fp16 activations).
//
// Both kernels rebuild each weight exactly as the reference's dequantize_groupwise does
// (edgerag/core/quant.py:98-107): the code becomes an fp16 integer exactly (a byte or nibble is
// OR-ed into the mantissa of 1024.0 and the bias is subtracted, both exact), then one fp16
// multiply by the fp16 group scale rounds once, like `codes.half() * scales`. x . W^T then runs on
// v_mfma_f32_*_f16 with fp32 accumulation, as F.linear does on fp16 tensors
// (edgerag/core/linear.py:194-196). The fp16 weight matrix is never written to memory.
//
// * qlinear_skinny_kernel (M <= 64, the decode GEMVs): HBM-bound. A wave owns 16 or 32 output
//   rows and one K chunk; every lane streams 16 bytes of packed weights per load (4 lanes cover
//   64 contiguous bytes of a row), U loads deep, and feeds them to v_mfma_f32_16x16x32_f16 as the
//   A operand straight from registers (no LDS). The activations (B operand, up to 64 rows) come
//   from L2. The waves of a workgroup split K; their partial sums are added in LDS in a fixed order.
//   Only the lane-to-k assignment inside a k-step differs from textbook order, identically for
//   both operands: INT4 nibbles decode to the k order (0,4,1,5,2,6,3,7), so the activations are
//   permuted the same way in registers.
// * qlinear_gemm_kernel (M > 64, prefill slices): MFMA-bound. A 256-thread workgroup computes a
//   BN x BM tile of y^T through v_mfma_f32_32x32x16_f16; per 64-k step it stages the dequantised
//   weights and the activations in double-buffered, XOR-swizzled LDS, loading the next steps'
//   bytes from global memory while the current one is computed. With a workspace
//   (edgerag_quant_linear_ws) it also takes decode batches past the streaming GEMV's crossover,
//   and splits K over the workgroups when the 64x64 tiles alone would leave CUs idle
//   (qlinear_split_reduce_kernel adds the k ranges' partial tiles in order).
#include "quant_mfma.h"

#ifndef EDGERAG_SKINNY_MAX_M
#define EDGERAG_SKINNY_MAX_M 64
#endif
#ifndef EDGERAG_STREAM_MAX_M
#define EDGERAG_STREAM_MAX_M 64  // per-channel INT8 launches up to this M use the streaming kernel
#endif
#ifndef EDGERAG_STREAM_NARROW_F2
#define EDGERAG_STREAM_NARROW_F2 1  // 17..32 tokens on narrow N: two k-slices (see dispatch_stream)
#endif
#ifndef EDGERAG_STREAM_F2_TILES
#define EDGERAG_STREAM_F2_TILES 256  // 16-row tiles below which decode launches take two k-slices
#endif
#ifndef EDGERAG_STREAM_NT2_TILES
#define EDGERAG_STREAM_NT2_TILES 512  // 16-row tiles from which a workgroup takes two
#endif
#ifndef EDGERAG_GEMM_THREADS_128
#define EDGERAG_GEMM_THREADS_128 256  // threads of a 128x128 GEMM workgroup (256 or 512)
#endif
#ifndef EDGERAG_GEMM_MIN_WG
#define EDGERAG_GEMM_MIN_WG 1  // workgroups per CU the GEMM's register budget must allow
#endif
// Per tile shape: threads and register stages in flight of the GEMM workgroup (the 64x64 tiles,
// one workgroup per CU, need a deeper ring than the larger ones).
#ifndef EDGERAG_GEMM_STAGES_128
#define EDGERAG_GEMM_STAGES_128 2
#endif
#ifndef EDGERAG_GEMM_THREADS_128x64
#define EDGERAG_GEMM_THREADS_128x64 256
#endif
#ifndef EDGERAG_GEMM_STAGES_128x64
#define EDGERAG_GEMM_STAGES_128x64 2
#endif
#ifndef EDGERAG_GEMM_THREADS_64
#define EDGERAG_GEMM_THREADS_64 256
#endif
#ifndef EDGERAG_GEMM_STAGES_64
#define EDGERAG_GEMM_STAGES_64 4
#endif
#ifndef EDGERAG_GEMM_READ_AHEAD
#define EDGERAG_GEMM_READ_AHEAD 1  // 16-k steps whose LDS operands are read ahead of the MFMAs
#endif
#ifndef EDGERAG_SPLITK_MAX
#define EDGERAG_SPLITK_MAX 16  // most k splits
#endif
#ifndef EDGERAG_SPLITK_MIN_STEPS
#define EDGERAG_SPLITK_MIN_STEPS 2  // fewest 64-k steps per split
#endif
#ifndef EDGERAG_SPLITK_FIXED_STEPS
#define EDGERAG_SPLITK_FIXED_STEPS 12  // cost of a split launch's partials and second launch
#endif
#ifndef EDGERAG_GEMM_TARGET_WGS
#define EDGERAG_GEMM_TARGET_WGS 256  // the tile is the largest whose grid reaches this many
#endif

namespace edgerag {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x4 mfma16(h8 a, h8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x16 mfma32(h8 a, h8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ h2 as_h2(uint32_t v) { return __builtin_bit_cast(h2, v); }
__device__ __forceinline__ uint32_t as_u32(h2 v) { return __builtin_bit_cast(uint32_t, v); }

__device__ __forceinline__ h8 pack_h8(h2 a, h2 b, h2 c, h2 d) {
  return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// Four INT8 codes (two's complement bytes of `w`) times the scale, in k order: two fp16 pairs.
// Byte b becomes the fp16 1024 + (b ^ 0x80) via v_perm_b32; subtracting 1152 leaves the signed
// code exactly.
__device__ __forceinline__ void deq_i8_word(uint32_t w, h2 s2, h2& lo, h2& hi) {
  const uint32_t wx = w ^ 0x80808080u;
  const h2 bias = {_Float16(1152.f), _Float16(1152.f)};
  lo = (as_h2(__builtin_amdgcn_perm(0x64646464u, wx, 0x04010400u)) - bias) * s2;
  hi = (as_h2(__builtin_amdgcn_perm(0x64646464u, wx, 0x04030402u)) - bias) * s2;
}

// Eight INT4 codes of `w` (nibble i = k i, biased by 8) times the scale, as one MFMA operand in
// the k order (0,4,1,5,2,6,3,7): nibbles i and i + 4 sit 16 bits apart, so one mask per pair.
__device__ __forceinline__ h8 deq_i4_word_perm(uint32_t w, h2 s2) {
  const h2 bias = {_Float16(1032.f), _Float16(1032.f)};
  const h2 p0 = (as_h2((w & 0x000F000Fu) | 0x64006400u) - bias) * s2;
  const h2 p1 = (as_h2(((w >> 4) & 0x000F000Fu) | 0x64006400u) - bias) * s2;
  const h2 p2 = (as_h2(((w >> 8) & 0x000F000Fu) | 0x64006400u) - bias) * s2;
  const h2 p3 = (as_h2(((w >> 12) & 0x000F000Fu) | 0x64006400u) - bias) * s2;
  return pack_h8(p0, p1, p2, p3);
}

// Eight INT4 codes of `w` times the scale in natural k order (0..7), as four fp16 pairs.
__device__ __forceinline__ void deq_i4_word(uint32_t w, h2 s2, h2 (&p)[4]) {
  const h2 bias = {_Float16(1032.f), _Float16(1032.f)};
  const uint32_t lo = w & 0x0F0F0F0Fu;         // k 0, 2, 4, 6 in bytes 0..3
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;  // k 1, 3, 5, 7
  // byte 0 <- lo.b_i (k 2i), byte 2 <- hi.b_i (k 2i+1); bytes 1 and 3 <- 0 (selector 0x0c).
  p[0] = (as_h2(__builtin_amdgcn_perm(hi, lo, 0x0C040C00u) | 0x64006400u) - bias) * s2;
  p[1] = (as_h2(__builtin_amdgcn_perm(hi, lo, 0x0C050C01u) | 0x64006400u) - bias) * s2;
  p[2] = (as_h2(__builtin_amdgcn_perm(hi, lo, 0x0C060C02u) | 0x64006400u) - bias) * s2;
  p[3] = (as_h2(__builtin_amdgcn_perm(hi, lo, 0x0C070C03u) | 0x64006400u) - bias) * s2;
}

// Activations x0..x7 (16 bytes) reordered to (0,4,1,5,2,6,3,7), matching deq_i4_word_perm.
__device__ __forceinline__ h8 perm_x_i4(uint4 d) {
  const uint32_t e0 = __builtin_amdgcn_perm(d.z, d.x, 0x05040100u);
  const uint32_t e1 = __builtin_amdgcn_perm(d.z, d.x, 0x07060302u);
  const uint32_t e2 = __builtin_amdgcn_perm(d.w, d.y, 0x05040100u);
  const uint32_t e3 = __builtin_amdgcn_perm(d.w, d.y, 0x07060302u);
  return pack_h8(as_h2(e0), as_h2(e1), as_h2(e2), as_h2(e3));
}

__device__ __forceinline__ uint4 ldg16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// ---- skinny kernel (M <= 64) ----------------------------------------------------------------
constexpr int kMaxSkinnyWaves = 8;

template <int BITS>
struct SkinnyCfg {
  static constexpr int KB = BITS == 8 ? 64 : 128;  // k covered by one 16-byte load per lane
  static constexpr int STEPS = BITS == 8 ? 2 : 4;  // MFMA k-steps (8 k per lane) per load
};

template <int BITS, int NT, int MT, int U>
struct SkinnyBatch {
  uint4 w[U][NT];
  uint32_t s[U][NT];  // raw fp16 scale bits (a plain integer keeps it in a register)
  uint4 x[U][MT][SkinnyCfg<BITS>::STEPS];  // raw activations; masked and permuted when used
};

// Issue the loads of U consecutive 64-byte row chunks (one per lane group) for NT row tiles and
// the matching activations of MT 16-row tiles. Every load is unconditional (chunk indices are
// clamped into the row, activation rows into [0, M)) so that no value is selected right after its
// load, which would make the wave wait for it; the masks are applied in skinny_compute.
template <int BITS, int NT, int MT, int U, bool PG>
__device__ __forceinline__ void skinny_load(SkinnyBatch<BITS, NT, MT, U>& b, int kb, int nkb,
                                            const uint8_t* const (&wp)[NT],
                                            const f16* const (&sp)[NT], int g,
                                            const f16* const (&xp)[MT], const bool (&xv)[MT],
                                            int lg) {
  using C = SkinnyCfg<BITS>;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int kk = min(kb + u, nkb - 1);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      b.w[u][t] = ldg16(wp[t] + int64_t(kk) * 64);
      if constexpr (PG)
        b.s[u][t] = reinterpret_cast<const uint16_t*>(sp[t])[(kk * C::KB + lg * (C::KB / 4)) / g];
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      // Only lanes of real activation rows load (exec-masked); the others' registers are
      // ignored by skinny_compute.
      if (xv[mt]) {
        const f16* xk = xp[mt] + int64_t(kk) * C::KB;
#pragma unroll
        for (int st = 0; st < C::STEPS; ++st) b.x[u][mt][st] = ldg16(xk + 8 * st);
      }
    }
  }
}

// Chunks kb + u at or past kb_end (the end of this wave's K range) and activation rows past M
// contribute zero activations, so their MFMAs add exact zeros.
template <int BITS, int NT, int MT, int U, bool PG>
__device__ __forceinline__ void skinny_compute(const SkinnyBatch<BITS, NT, MT, U>& b, int kb,
                                               int kb_end, const bool (&xv)[MT],
                                               const uint32_t (&s_row)[NT],
                                               f32x4 (&acc)[NT][MT]) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const bool on = kb + u < kb_end;
    h8 xo[MT][SkinnyCfg<BITS>::STEPS];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int st = 0; st < SkinnyCfg<BITS>::STEPS; ++st) {
        const uint4 raw = (on && xv[mt]) ? b.x[u][mt][st] : uint4{0, 0, 0, 0};
        xo[mt][st] = BITS == 8 ? __builtin_bit_cast(h8, raw) : perm_x_i4(raw);
      }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      // The row scale is loop-invariant: passing it through an empty asm keeps its first use
      // (and so the wait for its load) inside the loop, after the batch's loads are issued.
      uint32_t sr = PG ? b.s[u][t] : s_row[t];
      if constexpr (!PG) asm volatile("" : "+v"(sr));
      const _Float16 s1 = __builtin_bit_cast(_Float16, uint16_t(sr));
      const h2 s2 = {s1, s1};
      const uint32_t words[4] = {b.w[u][t].x, b.w[u][t].y, b.w[u][t].z, b.w[u][t].w};
      if constexpr (BITS == 8) {
        h2 p[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) deq_i8_word(words[q], s2, p[2 * q], p[2 * q + 1]);
        const h8 a0 = pack_h8(p[0], p[1], p[2], p[3]);
        const h8 a1 = pack_h8(p[4], p[5], p[6], p[7]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc[t][mt] = mfma16(a0, xo[mt][0], acc[t][mt]);
          acc[t][mt] = mfma16(a1, xo[mt][1], acc[t][mt]);
        }
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const h8 a = deq_i4_word_perm(words[q], s2);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[t][mt] = mfma16(a, xo[mt][q], acc[t][mt]);
        }
      }
    }
  }
}

// One workgroup: 16*NT output rows, all M <= 16*MT activation rows, K split across its waves
// (blockDim.x / 64 of them). Lane l feeds row l % 16 of a tile (A operand) and activation row
// l % 16 of an m-tile (B operand); lane group l / 16 owns bytes [16 (l/16), +16) of every 64-byte
// row chunk.
// kw: the launch's waves per workgroup (blockDim.x / 64), passed among the leading arguments, which
// the library preloads into SGPRs, so the K split does not wait for a load of the workgroup size
// from the hidden kernel arguments.
template <int BITS, int NT, int MT, int U, int NB, bool PG, int KWMAX>
__global__ __launch_bounds__(KWMAX * kWave) void qlinear_skinny_kernel(
    const f16* __restrict__ x, int64_t xs, const uint8_t* __restrict__ packed,
    const f16* __restrict__ scales, int32_t m, int32_t k, int32_t n, int32_t g, int32_t kw,
    const f16* __restrict__ bias, f16* __restrict__ y, int64_t ys) {
  using C = SkinnyCfg<BITS>;
  __shared__ float red[KWMAX * NT * MT * 4 * kWave];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int nkb = k / C::KB;
  const int per = (nkb + kw - 1) / kw;
  const int kb0 = min(nkb, wave * per), kb1 = min(nkb, kb0 + per);
  const int64_t row_bytes = BITS == 8 ? k : k / 2;
  const int groups = k / g;
  const int n0 = blockIdx.x * 16 * NT;

  const uint8_t* wp[NT];
  const f16* sp[NT];
  uint32_t s_row[NT];  // raw bits of the row's only scale when PG is false (one group spans K)
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int row = min(n0 + 16 * t + li, n - 1);  // rows past N compute garbage, never stored
    wp[t] = packed + int64_t(row) * row_bytes + 16 * lg;
    sp[t] = scales + int64_t(row) * groups;
    s_row[t] = PG ? 0u : reinterpret_cast<const uint16_t*>(sp[t])[0];
  }
  const f16* xp[MT];
  bool xv[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int mrow = 16 * mt + li;
    xv[mt] = mrow < m;
    xp[mt] = x + int64_t(xv[mt] ? mrow : m - 1) * xs + lg * (C::KB / 4);
  }

  f32x4 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Super-batches of NB x U chunks: every load of a super-batch is issued before any of its
  // chunks is computed, so a wave pays one memory round trip per super-batch. The host sizes
  // the K split so that most waves need a single super-batch.
  for (int kb = kb0; kb < kb1; kb += NB * U) {
    SkinnyBatch<BITS, NT, MT, U> b[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i)
      skinny_load<BITS, NT, MT, U, PG>(b[i], kb + i * U, nkb, wp, sp, g, xp, xv, lg);
    issue_fence();
#pragma unroll
    for (int i = 0; i < NB; ++i)
      skinny_compute<BITS, NT, MT, U, PG>(b[i], kb + i * U, kb1, xv, s_row, acc);
  }

  // Sum the waves' partials in wave order (deterministic), then write y[m][n] (+ bias).
  constexpr int kVals = NT * MT * 4;
  constexpr int kElems = kVals * kWave;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        red[(wave * kVals + (t * MT + mt) * 4 + r) * kWave + lane] = acc[t][mt][r];
  __syncthreads();
  for (int e = threadIdx.x; e < kElems; e += blockDim.x) {
    const int l = e & 63, v = e >> 6;
    const int r = v & 3, mt = (v >> 2) % MT, t = (v >> 2) / MT;
    const int nrow = n0 + 16 * t + 4 * (l >> 4) + r;
    const int mrow = 16 * mt + (l & 15);
    if (nrow >= n || mrow >= m) continue;
    float sum = 0.f;
    for (int w = 0; w < kw; ++w) sum += red[w * kElems + e];
    const float bv = bias != nullptr ? __half2float(bias[nrow]) : 0.f;
    y[int64_t(mrow) * ys + nrow] = __float2half_rn(sum + bv);
  }
}

// ---- streaming kernel (INT8 per-channel, M <= 16) --------------------------------------------
// One workgroup owns NT tiles of R = 16 / F weight rows and all M <= MT R activation rows; its KW
// waves split K. The 16 A rows of v_mfma_f32_16x16x32_f16 are F k-slices x R weight rows and the
// 16 B columns of m-tile t are F k-slices x R activation rows (t R + [0, R)): lane row li = f R + r
// streams row r at 64-byte chunks c F + f, so each load instruction covers F x 64 contiguous bytes
// of R rows, and a workgroup needs only NT R rows (N / R workgroups fill the chip even for
// N = 2048). The NT row tiles of a wave share its activation registers.
// D[(f, r)][(f, j)] of tile (n-tile, t) is the slice-f partial of y[t R + j][r]; the off-diagonal
// blocks pair different k-slices and are never read.
// The dequantised weight is the exact integer code (no scale): the row's scale multiplies the fp32
// sum once, scale * sum(code * x), instead of rounding every code * scale to fp16 first.
//
// Epilogues (EPI):
// * kEpiPlain: y = the projection.
// * kEpiSwiglu (NT == 2): the weight is [gate; up] (N = 2 I rows) and row tile 1 is the up twin of
//   tile 0 (rows I + n0 + [0, R)), so every workgroup holds gate and up of the same R columns and
//   writes act[t][j] = fp16(fp16(silu(g)) * u) to y (T x I) instead of the projection.
// * kEpiRope (NT == 2, F == 1): the weight is the fused [q heads | k heads | v heads] projection
//   and the two row tiles are the two halves of one head (rows head D + tn D / 2 + j + [0, 16)),
//   so every rotate_half pair (d, d + D / 2) sits in one wave; q heads are rotated into q_out, k
//   heads rotated and v heads copied into the paged pools at the token's slot.
// * kEpiResidual: hidden[t][n] = fp16(hidden[t][n] + y[t][n]) in place (y itself is not written),
//   optionally xw[t][n] = fp16(w[n] * hidden[t][n]) with the next RMSNorm's weight w, plus one fp32
//   sum of squares of the new values per (token, workgroup): the partials a normed launch turns
//   into the RMSNorm factor, so that residual add + RMSNorm need no launch of their own and no
//   workgroup waits for another.
// The fp16 projection values the epilogues start from are the ones the plain launch of the same
// shape writes: the host gives the fused launches the same waves, batches and k-slices, so the
// summation order, and so the bits, are the same.
// NORM (with kEpiSwiglu / kEpiRope): the activation is a residual producer's xw = fp16(w * h) and
// the projection is of RMSNorm(h) = fp16(w * fp16(h * r)); computed as r * sum(code * xw) with r
// applied to the fp32 sum (one fp16 rounding moved, within the linear tolerance of the reference).
constexpr int kEpiPlain = 0, kEpiSwiglu = 1, kEpiRope = 2, kEpiResidual = 3;

// Sum of v over aligned groups of G lanes (G = 8, 16, 32 or 64), in the same order on every lane
// of a group (so every lane gets the same bits): DPP adds within a 16-lane row (mirror pairs, then
// the two lanes of each pair of quads), cross-row shuffles only above 16.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int G>
__device__ __forceinline__ float lane_group_sum(float v) {
  static_assert(G == 8 || G == 16 || G == 32 || G == 64, "lane group");
  if constexpr (G >= 16) v += dpp_f<0x140>(v);  // row_mirror: lane i + lane 15 - i
  v += dpp_f<0x141>(v);                          // row_half_mirror: i + 7 - i within 8
  v += dpp_f<0x4E>(v);                           // quad_perm [2, 3, 0, 1]
  v += dpp_f<0xB1>(v);                           // quad_perm [1, 0, 3, 2]
  if constexpr (G >= 32) v += __shfl_xor(v, 16, kWave);
  if constexpr (G >= 64) v += __shfl_xor(v, 32, kWave);
  return v;
}

// The reference's rotate_half RoPE on one element (fp16 ops, each product rounded before the add):
// first half: x1 cos - x2 sin; second half: x2 cos + x1 sin (x1 = element d, x2 = element d + D/2).
__device__ __forceinline__ f16 rope_elem(float own, float partner, bool second, float c, float sn) {
#pragma clang fp contract(off)
  const float a = __half2float(__float2half_rn(own * c));
  const float b = __half2float(__float2half_rn((second ? partner : -partner) * sn));
  return __float2half_rn(a + b);
}

// RH (kEpiRope): half the head dimension when known at compile time (0: ea.head_dim / 2). The
// weight rows of a RoPE workgroup follow from it, and ea is not among the leading kernel
// arguments preloaded into SGPRs: a run-time value makes the first loads wait for its fetch.
template <int F, int NT, int MT, int KW, int U, bool EXACT, int EPI, bool NORM, bool X1,
          int RH = 0>
__global__ __launch_bounds__(KW * kWave)
__attribute__((amdgpu_waves_per_eu(1, U * MT * NT >= 8 ? KW / 4 : 8))) void qlinear_stream_kernel(
    const f16* __restrict__ x, int64_t xs, int32_t m, int32_t k,
    const uint8_t* __restrict__ packed, const f16* __restrict__ scales,
    const f16* __restrict__ bias, int32_t n, f16* __restrict__ y, int64_t ys, const EpiArgs ea) {
  constexpr int R = 16 / F;
  constexpr int CB = 64 * F;               // bytes (= k) of one chunk step of a row
  constexpr int OUTS = NT * MT * R * R;    // outputs (token, row) of a workgroup
  constexpr int NO = (OUTS + KW * kWave - 1) / (KW * kWave);  // outputs per thread
  static_assert((KW * kWave) % (NT * R) == 0, "a thread's outputs share one weight row");
  static_assert(EPI == kEpiPlain || EPI == kEpiResidual || (NT == 2 && kWave % (NT * R) == 0) ||
                    (EPI == kEpiRope && NT == 1 && F == 2),
                "paired epilogues pair tile 0 with tile 1 inside one wave");
  static_assert(EPI != kEpiRope || (F == 1 && NT == 2) || (F == 2 && NT == 1),
                "RoPE pairs two 16-row tiles, or the rows of one 8-row tile");
  static_assert(EPI != kEpiResidual || kWave % (NT * R) == 0, "a token's rows share one wave");
  static_assert(!NORM || (EPI == kEpiSwiglu && F == 1) || EPI == kEpiRope, "normed inputs");
  // kEpiRope with one 8-row tile: lane row rr is element rr / 2 of the workgroup's run of a
  // head's first half (rr even) or its rotate_half partner in the second half (rr odd).
  constexpr bool ROPE8 = EPI == kEpiRope && NT == 1;
  constexpr int NPQ = kNormMaxParts / kWave;           // partials per lane and token
  constexpr int TOKW = NORM ? (MT * R + KW - 1) / KW : 1;  // tokens whose factor a wave sums
  __shared__ float red[KW * NT * MT * 4 * kWave];
  __shared__ float rnorm[NORM ? MT * R : 1];
  // X1 (one token): a wave loads the token's activations of a batch once, each lane a distinct
  // 16 bytes, and the lanes read their B operands from this LDS copy. Loading them straight
  // from global memory costs a 64-lane load instruction per operand and step although the lane
  // rows of one token all want the same bytes (the address unit's time goes by instructions,
  // not by distinct bytes: measured 0.8 us of a 6.2 us 8192->2048 launch).
  constexpr int XV = U * CB / 8;  // 16-byte chunks of one token's activations per batch
  __shared__ uint4 xlds[X1 ? KW : 1][X1 ? XV : 1];
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int lane = threadIdx.x & 63;
  const int li = lane & 15, lg = lane >> 4;
  const int f = li / R, r = li % R;
  // kEpiSwiglu: gate rows [0, half), up rows [half, n). kEpiRope: head_dim / 2.
  const int half = EPI == kEpiRope ? (RH > 0 ? RH : ea.head_dim >> 1) : n >> 1;
  constexpr int PAIRS = NT * R / 2;  // kEpiRope: rotate_half pairs of a workgroup
  const int per_head = half / PAIRS;  // kEpiRope: workgroups per head
  const int rope_head = EPI == kEpiRope ? int(blockIdx.x) / per_head : 0;
  const int rope_j = EPI == kEpiRope ? (int(blockIdx.x) % per_head) * PAIRS : 0;
  const int n0 = EPI == kEpiRope ? rope_head * 2 * half + rope_j
                                 : int(blockIdx.x) * (EPI == kEpiSwiglu ? R : NT * R);
  const int nc = k / CB;  // chunk steps: >= U, and a multiple of KW * U when EXACT
  const int per = (nc + KW - 1) / KW;
  const int c0 = min(nc, wave * per), c1 = min(nc, c0 + per);
  // Weight row of lane row rr in tile tn. Rows past N (past I in a SwiGLU half) re-read the last
  // row: they only feed D rows that are never read. (kEpiRope launches cover N exactly.)
  auto wrow = [&](int tn, int rr) {
    if constexpr (EPI == kEpiPlain || EPI == kEpiResidual) return min(n0 + tn * R + rr, n - 1);
    else if constexpr (EPI == kEpiSwiglu) return min(n0 + rr, half - 1) + tn * half;
    else if constexpr (ROPE8) return n0 + (rr & 1) * half + (rr >> 1);
    else return n0 + tn * half + rr;
  };

  // A lane of n-tile tn: weight row wrow(tn, r); B lane of m-tile t: activation row t R + r.
  // Rows past M re-read the last row: they only feed D columns that are never read.
  const uint8_t* wp[NT];
#pragma unroll
  for (int tn = 0; tn < NT; ++tn) wp[tn] = packed + int64_t(wrow(tn, r)) * k + f * 64 + 16 * lg;
  const f16* xp[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) xp[t] = x + int64_t(min(t * R + r, m - 1)) * xs + f * 64 + 16 * lg;

  // Output e (e = thread, thread + KW 64, ...) is lane row e % R of tile e % (NT R) / R, token
  // e / (NT R): all of a thread's outputs share one row, whose scale and bias are loaded now and
  // first waited for after the first batch is computed.
  // Whole aligned 32-bit words are loaded (nothing is computed on them before the pins), and the
  // bias word unconditionally -- from the scales when there is no bias -- so that no branch sits
  // between these loads and the batch loads (either would cost the batch its progressive waits).
  const int e_in = int(threadIdx.x) % (NT * R);
  const int e_row = wrow(e_in / R, e_in % R);
  const f16* b_src = bias != nullptr ? bias : scales;
  const int s_mis = int(reinterpret_cast<uintptr_t>(scales) >> 1) & 1;  // base at an odd half
  const int b_mis = int(reinterpret_cast<uintptr_t>(b_src) >> 1) & 1;
  const int s_idx = e_row + s_mis, b_idx = e_row + b_mis;
  uint32_t s_bits = reinterpret_cast<const uint32_t*>(scales - s_mis)[s_idx >> 1];
  uint32_t b_bits = reinterpret_cast<const uint32_t*>(b_src - b_mis)[b_idx >> 1];
  // kEpiRope: every output of this thread is element e_d of its head for token e / (NT R); the
  // token's cos / sin at e_d and its slot are loaded now as well (tokens past M re-read the last).
  const int e_d = ROPE8 ? (e_in & 1) * half + rope_j + (e_in >> 1)
                        : (e_in / R) * half + rope_j + e_in % R;
  // (Raw loads only, nothing computed on them before the pins, like the scale and bias words.)
  // These loads take their pointers from the epilogue arguments, which are not among the
  // leading kernel arguments preloaded into SGPRs: they are issued right after the first batch's
  // weight loads (epi_loads), so that the batch does not wait for the argument fetch.
  int32_t rope_slot[EPI == kEpiRope ? NO : 1];
  uint32_t rope_c[EPI == kEpiRope ? NO : 1], rope_s[EPI == kEpiRope ? NO : 1];
  uint32_t hid_pre[EPI == kEpiResidual ? NO : 1];
  uint32_t nw_pre = 0;  // kEpiResidual with xw: the next norm's weight at this thread's row
  float norm_pre[NORM ? TOKW * NPQ : 1];
  // The argument values pass through pin_s where they are used, so that no address computation
  // (and no wait for the argument fetch) is hoisted above the batch loads.
  auto epi_loads = [&]() {
    if constexpr (EPI == kEpiRope) {
      const auto* cos_u = as_global(reinterpret_cast<const uint16_t*>(pin_s(ea.cos_tok)));
      const auto* sin_u = as_global(reinterpret_cast<const uint16_t*>(pin_s(ea.sin_tok)));
      const auto* slots = as_global(pin_s(ea.slots));
      const int hd = pin_s(ea.head_dim);
#pragma unroll
      for (int o = 0; o < NO; ++o) {
        const int tok = min((int(threadIdx.x) + o * KW * kWave) / (NT * R), m - 1);
        rope_slot[o] = slots[tok];
        rope_c[o] = cos_u[int64_t(tok) * hd + e_d];
        rope_s[o] = sin_u[int64_t(tok) * hd + e_d];
      }
    }
    // kEpiResidual: the residual-stream value of each output. NORM: wave w sums the partials of
    // tokens w, w + KW, ..., lane l those with index l + 64 q (clamped; masked when summed).
    if constexpr (EPI == kEpiResidual) {
      const f16* hidden = pin_s(ea.hidden);
      const f16* next_w = pin_s(ea.next_w);
      const int64_t hid_st = pin_s(ea.hid_st);
      const auto* hid_u = as_global(reinterpret_cast<const uint16_t*>(hidden));
#pragma unroll
      for (int o = 0; o < NO; ++o) {
        const int tok = min((int(threadIdx.x) + o * KW * kWave) / (NT * R), m - 1);
        hid_pre[o] = hid_u[int64_t(tok) * hid_st + e_row];
      }
      // Loaded unconditionally (from the hidden row when there is no xw): no branch between
      // these loads.
      const auto* nw_u =
          as_global(reinterpret_cast<const uint16_t*>(next_w != nullptr ? next_w : hidden));
      nw_pre = nw_u[e_row];
    }
    if constexpr (NORM) {
      // Only the batch's tokens and the partials the producer wrote are loaded (wave-uniform
      // branches): at one token one wave of the workgroup loads its 256 sums, where every wave
      // loaded a clamped copy, 8 instructions per wave through the address unit (one token:
      // 2048->16384 gate/up 9.71 -> 9.58 us, q/k/v + RoPE 5.84 -> 5.64 us).
      const auto* norm_part = as_global(pin_s(ea.norm_part));
      const int parts = pin_s(ea.norm_parts);
#pragma unroll
      for (int j = 0; j < TOKW; ++j) {
        const int tok = wave + KW * j;
#pragma unroll
        for (int q = 0; q < NPQ; ++q) {
          norm_pre[j * NPQ + q] = 0.f;
          if (tok < m && kWave * q < parts)
            norm_pre[j * NPQ + q] =
                norm_part[int64_t(tok) * parts + min(lane + kWave * q, parts - 1)];
        }
      }
    }
  };

  f32x4 acc[NT][MT];
#pragma unroll
  for (int tn = 0; tn < NT; ++tn)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[tn][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const h2 bias2 = {_Float16(1152.f), _Float16(1152.f)};
  for (int cb = c0; cb < c1; cb += U) {
    // A batch of U steps starting no later than nc - U, so every load is in bounds and its
    // offsets are immediates. Unless EXACT (every wave owns whole batches), steps outside
    // [cb, c1) (already done, or another wave's) keep the accumulators unchanged.
    const int cs = min(cb, nc - U);
    uint4 w[U][NT], xa[U][MT], xc[U][MT];
    constexpr int XL = (XV + kWave - 1) / kWave;  // X1: activation loads per lane and batch
    uint4 xr[X1 ? XL : 1];
    if constexpr (X1) {  // issued first: the LDS copy waits for these, not for the weights
#pragma unroll
      for (int i = 0; i < XL; ++i)
        xr[i] = ldg16(x + int64_t(cs) * CB + int64_t(min(lane + kWave * i, XV - 1)) * 8);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {  // in step order, so step u waits only for its own loads
#pragma unroll
      for (int tn = 0; tn < NT; ++tn) w[u][tn] = ldg16(wp[tn] + int64_t(cs) * CB + u * CB);
      if constexpr (!X1) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const f16* xb = xp[t] + int64_t(cs) * CB + u * CB;
          xa[u][t] = ldg16(xb);
          xc[u][t] = ldg16(xb + 8);
        }
      }
    }
    if constexpr (EPI == kEpiRope || EPI == kEpiResidual || NORM) {
      if (cb == c0) {
        issue_fence();  // the batch's loads go out before the epilogue's wait for its arguments
        epi_loads();
      }
    }
    issue_fence();
    if constexpr (X1) {
      // The wave's own LDS rows: a wavefront barrier orders the writes before the reads (and
      // the reads of the previous batch before these writes).
#pragma unroll
      for (int i = 0; i < XL; ++i)
        if (lane + kWave * i < XV) xlds[wave][lane + kWave * i] = xr[i];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = (u * CB + f * 64 + 16 * lg) / 8;
        xa[u][0] = xlds[wave][c];
        xc[u][0] = xlds[wave][c + 1];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool on = EXACT || (cs + u >= cb && cs + u < c1);
#pragma unroll
      for (int tn = 0; tn < NT; ++tn) {
        const uint4 wq = w[u][tn];
        const uint32_t words[4] = {wq.x ^ 0x80808080u, wq.y ^ 0x80808080u, wq.z ^ 0x80808080u,
                                   wq.w ^ 0x80808080u};
        h2 p[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          // Byte b (offset binary after the xor) becomes the fp16 1024 + b; minus 1152 is the
          // code.
          p[2 * q] = as_h2(__builtin_amdgcn_perm(0x64646464u, words[q], 0x04010400u)) - bias2;
          p[2 * q + 1] = as_h2(__builtin_amdgcn_perm(0x64646464u, words[q], 0x04030402u)) - bias2;
        }
        const h8 a0 = pack_h8(p[0], p[1], p[2], p[3]), a1 = pack_h8(p[4], p[5], p[6], p[7]);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          f32x4 v = mfma16(a0, __builtin_bit_cast(h8, xa[u][t]), acc[tn][t]);
          v = mfma16(a1, __builtin_bit_cast(h8, xc[u][t]), v);
          acc[tn][t] = on ? v : acc[tn][t];
        }
      }
    }
    // The epilogue's scale and bias are waited for here, once the first batch is computed.
    if (cb == c0) {
      asm volatile("" : "+v"(s_bits), "+v"(b_bits));
      if constexpr (EPI == kEpiRope) {
#pragma unroll
        for (int o = 0; o < NO; ++o)
          asm volatile("" : "+v"(rope_slot[o]), "+v"(rope_c[o]), "+v"(rope_s[o]));
      }
      if constexpr (EPI == kEpiResidual) {
#pragma unroll
        for (int o = 0; o < NO; ++o) asm volatile("" : "+v"(hid_pre[o]));
        asm volatile("" : "+v"(nw_pre));
      }
      if constexpr (NORM) {
#pragma unroll
        for (int i = 0; i < TOKW * NPQ; ++i) asm volatile("" : "+v"(norm_pre[i]));
      }
    }
  }
  if (c0 >= c1) epi_loads();  // a wave with no K range still writes outputs (none for kEpiPlain,
                              // kEpiSwiglu without NORM: their epi_loads is empty)

  // Sum slices and waves in a fixed order, then y[m][n] = scale[n] * sum (+ bias[n]).
  // Accumulator register i of lane l holds D row 4 (l / 16) + i, column l % 16.
#pragma unroll
  for (int tn = 0; tn < NT; ++tn)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        red[(((wave * NT + tn) * MT + t) * 4 + i) * kWave + lane] = acc[tn][t][i];
  if constexpr (NORM) {
    // r_t = rsqrt(mean(h^2) + eps) from the producer's partials, summed in a fixed order (per
    // lane, then lane_group_sum), so every workgroup derives the same bits.
    float sq[TOKW];
#pragma unroll
    for (int j = 0; j < TOKW; ++j) {  // the tokens' reductions interleave
      sq[j] = 0.f;
#pragma unroll
      for (int q = 0; q < NPQ; ++q) {
        float v = norm_pre[j * NPQ + q];
        asm volatile("" : "+v"(v));
        sq[j] += lane + kWave * q < ea.norm_parts ? v : 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < TOKW; ++j) sq[j] = lane_group_sum<kWave>(sq[j]);
#pragma unroll
    for (int j = 0; j < TOKW; ++j) {
      const int tok = wave + KW * j;  // wave-uniform
      if (tok < MT * R && lane == 0) rnorm[tok] = rsqrtf(sq[j] / float(k) + ea.eps);
    }
  }
  __syncthreads();
  // (Consumed again here so that the conversions below are not hoisted above the main loop,
  // which would wait for the loads before the first batch is issued.)
  asm volatile("" : "+v"(s_bits), "+v"(b_bits));
  const int sh_s = (s_idx & 1) * 16, sh_b = (b_idx & 1) * 16;
  const float scale = float(__builtin_bit_cast(_Float16, uint16_t(s_bits >> sh_s)));
  const float bv =
      bias != nullptr ? float(__builtin_bit_cast(_Float16, uint16_t(b_bits >> sh_b))) : 0.f;
  auto out_sum = [&](int tok, int tn, int rr) {
    const int t = tok / R, jj = tok % R;
    float sum = 0.f;
#pragma unroll
    for (int fs = 0; fs < F; ++fs) {
      const int drow = fs * R + rr, dcol = fs * R + jj;
      const int l = 16 * (drow >> 2) + dcol, i = drow & 3;
      for (int wv = 0; wv < KW; ++wv)
        sum += red[(((wv * NT + tn) * MT + t) * 4 + i) * kWave + l];
    }
    const float sc = NORM ? scale * rnorm[tok] : scale;
    return __float2half_rn(__builtin_fmaf(sc, sum, bv));
  };
  if constexpr (EPI == kEpiPlain) {
    for (int e = threadIdx.x; e < OUTS; e += KW * kWave) {
      const int tok = e / (NT * R), row_in = e % (NT * R);
      const int nrow = n0 + row_in;
      if (tok >= m || nrow >= n) continue;
      y[int64_t(tok) * ys + nrow] = out_sum(tok, row_in / R, row_in % R);
    }
  } else if constexpr (EPI == kEpiResidual) {
    // h = fp16(hidden + y); the NT R lanes of one token (consecutive, aligned) then sum their h^2,
    // and the token's first lane writes the workgroup's partial.
#pragma unroll
    for (int o = 0; o < NO; ++o) {
      const int e = int(threadIdx.x) + o * KW * kWave;
      if (e >= OUTS) break;  // uniform per wave
      const int tok = e / (NT * R), row_in = e % (NT * R);
      const int nrow = n0 + row_in;
      const bool ok = tok < m && nrow < n;
      float sq = 0.f;
      if (ok) {
        const float hv = __half2float(__builtin_bit_cast(f16, uint16_t(hid_pre[o])));
        const f16 h = __float2half_rn(hv + __half2float(out_sum(tok, row_in / R, row_in % R)));
        ea.hidden[int64_t(tok) * ea.hid_st + nrow] = h;
        const float hf = __half2float(h);
        sq = hf * hf;
        if (ea.xw != nullptr)  // w * h is exact in fp32 (two fp16 factors): one rounding
          ea.xw[int64_t(tok) * ea.xw_st + nrow] =
              __float2half_rn(__half2float(__builtin_bit_cast(f16, uint16_t(nw_pre))) * hf);
      }
      sq = lane_group_sum<NT * R>(sq);
      if (row_in == 0 && tok < m) ea.part[int64_t(tok) * gridDim.x + blockIdx.x] = sq;
    }
  } else if constexpr (EPI == kEpiSwiglu) {
    // The up output of gate lane l sits in lane l + R of the same wave (same token, tile 1). OUTS
    // and the stride are multiples of 64, so whole waves run each iteration and the shuffle sees
    // every lane.
    for (int e = threadIdx.x; e < OUTS; e += KW * kWave) {
      const int tok = e / (NT * R), row_in = e % (NT * R);
      const int tn = row_in / R, rr = row_in % R;
      const float v = __half2float(out_sum(tok, tn, rr));
      const float u = __shfl_down(v, R, kWave);
      if (tn == 0 && tok < m && n0 + rr < half)
        y[int64_t(tok) * ys + n0 + rr] = __float2half_rn(silu_rounded_f16(v) * u);
    }
  } else {
    // Element d of a head sits in lane l and its rotate_half partner d +- D/2 in lane l ^ 16
    // (two 16-row tiles) or l ^ 1 (one 8-row tile).
    const int tn = e_in / R;
    const bool second = ROPE8 ? (e_in & 1) != 0 : tn == 1;
    const int nq = ea.n_q_heads, nkv = ea.n_kv_heads;
    const int64_t pool_rows = int64_t(ea.num_blocks) * ea.block_size;
#pragma unroll
    for (int o = 0; o < NO; ++o) {
      const int e = int(threadIdx.x) + o * KW * kWave;
      if (e >= OUTS) break;  // uniform per wave
      const int tok = e / (NT * R);
      const float v = __half2float(out_sum(tok, tn, e_in % R));
      const float partner = __shfl_xor(v, ROPE8 ? 1 : 16, kWave);
      if (tok >= m) continue;
      const float c = __half2float(__builtin_bit_cast(f16, uint16_t(rope_c[o])));
      const float sn = __half2float(__builtin_bit_cast(f16, uint16_t(rope_s[o])));
      const int head = rope_head;
      if (head < nq) {
        ea.q_out[int64_t(tok) * ea.q_st + int64_t(head) * ea.head_dim + e_d] =
            rope_elem(v, partner, second, c, sn);
        continue;
      }
      const int64_t slot = rope_slot[o];
      if (slot < 0 || slot >= pool_rows) continue;
      const int kvh = head < nq + nkv ? head - nq : head - nq - nkv;
      const int64_t off =
          ((int64_t(kvh) * ea.num_blocks + slot / ea.block_size) * ea.block_size +
           slot % ea.block_size) * ea.head_dim + e_d;
      if (head < nq + nkv)
        ea.kpool[off] = rope_elem(v, partner, second, c, sn);
      else
        ea.vpool[off] = __float2half_rn(v);
    }
  }
}

// ---- tiled GEMM (M > 64) --------------------------------------------------------------------
constexpr int kBK = 64;     // k per LDS stage
constexpr int kLdsRow = 64;  // halves per LDS row (one row of a 64-k stage)

// Halves offset of 16-byte chunk `c` (k 8c .. 8c + 7 of the stage) of LDS row `row`. The stage is
// stored in MFMA operand order: for each 32-row tile and 16-k step ks = c / 2, the 64 lanes'
// operands (lane = 32 (c & 1) + row % 32) fill one block of 64 16-byte slots, so every operand
// read is one 1 KiB ds_read_b128. Inside a block the lane's slot is XOR-ed with
// lds_swizzle(ks) (bits 1..3 only, so each aligned group of 8 or 16 lanes still covers every
// bank once): the stagers write 2 or 4 chunks of the same row from adjacent lanes, i.e. to
// blocks with different ks, and without the swizzle those writes would land on the same banks
// (slots 512 B apart). With it, any 8 or 16 adjacent stager lanes hit distinct banks for both
// stager shapes (4 lanes per row, ks = lane % 4; 2 lanes per row, ks / 2 = lane % 2).
__device__ __forceinline__ constexpr int lds_swizzle(int ks) {
  return ((ks & 2) << 2) | ((((ks >> 1) ^ ks) & 1) << 2) | ((ks & 1) << 1);
}
__device__ __forceinline__ int lds_off(int row, int c) {
  const int ks = c >> 1;
  const int lane = (c & 1) * 32 + (row & 31);
  return (((row >> 5) * 4 + ks) * 64 + (lane ^ lds_swizzle(ks))) * 8;
}

// A BN x BM tile computed by NTH threads: waves in a 2 x (NTH / 128) grid (N x M), each owning
// TN x TM 32x32 MFMA tiles. With 512 threads two waves share each SIMD, so one wave's memory
// and LDS waits overlap the other's matrix work.
template <int BITS_, int BN_, int BM_, int NTH_>
struct GemmCfg {
  static constexpr int BITS = BITS_, BN = BN_, BM = BM_, NTH = NTH_;
  static constexpr int NWN = 2, NWM = NTH / 128;                    // wave grid
  static constexpr int W_ROW_BYTES = BITS == 8 ? kBK : kBK / 2;    // packed bytes per row, per stage
  static constexpr int W_BPT = BN * W_ROW_BYTES / NTH;              // packed bytes per thread
  static constexpr int W_TPR = W_ROW_BYTES / W_BPT;                 // threads per weight row
  static constexpr int W_K = BITS == 8 ? W_BPT : 2 * W_BPT;         // k per thread (8, 16 or 32)
  static constexpr int X_BPT = BM * kBK * 2 / NTH;                  // activation bytes per thread
  static constexpr int X_TPR = kBK * 2 / X_BPT;                     // threads per activation row
  static constexpr int TN = BN / (32 * NWN), TM = BM / (32 * NWM);  // 32x32 tiles per wave
  static_assert(TN >= 1 && TM >= 1, "tile too small for the wave grid");
  static_assert(W_BPT == 8 || W_BPT == 16 || W_BPT == 32, "weight staging split");
  static_assert(X_BPT == 32 || X_BPT == 64, "activation staging split");
};

template <class C>
struct GemmStage {
  uint32_t w[C::W_BPT / 4];
  f16 s;
  uint4 x[C::X_BPT / 16];
};

// Loads one 64-k stage of this thread's weight segment (and its group scale) and activation
// segment into registers.
template <class C>
__device__ __forceinline__ void gemm_load(GemmStage<C>& st, int k0, const uint8_t* wrow,
                                          const f16* srow, int g, int wk_off, const f16* xrow) {
  constexpr int BITS = C::BITS;
  const uint8_t* wp = wrow + (BITS == 8 ? k0 : k0 / 2);
  if constexpr (C::W_BPT == 8) {
    const uint2 v = *reinterpret_cast<const uint2*>(wp);
    st.w[0] = v.x;
    st.w[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < C::W_BPT / 16; ++i) {
      const uint4 v = ldg16(wp + 16 * i);
      st.w[4 * i] = v.x;
      st.w[4 * i + 1] = v.y;
      st.w[4 * i + 2] = v.z;
      st.w[4 * i + 3] = v.w;
    }
  }
  // A segment never straddles a group: it is 16 or 32 k, aligned, and g % 32 == 0.
  st.s = srow[(k0 + wk_off) / g];
#pragma unroll
  for (int i = 0; i < C::X_BPT / 16; ++i) st.x[i] = ldg16(xrow + k0 + 8 * i);
}

// Writes weight chunk c (8 k) of this thread's staged segment to LDS, dequantised: the exact
// integer code when PC (per-channel scales, applied to the fp32 sums in the epilogue), else
// code * scale rounded to fp16 once, as the reference's dequantize_groupwise does.
template <class C, bool PC>
__device__ __forceinline__ void gemm_store_w(const GemmStage<C>& st, int c, _Float16* sw, int wr,
                                             int wc0) {
  constexpr int BITS = C::BITS;
  h2 p[4];
  if constexpr (BITS == 8) {
    if constexpr (PC) {
      const h2 bias = {_Float16(1152.f), _Float16(1152.f)};
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint32_t wx = st.w[2 * c + q] ^ 0x80808080u;
        p[2 * q] = as_h2(__builtin_amdgcn_perm(0x64646464u, wx, 0x04010400u)) - bias;
        p[2 * q + 1] = as_h2(__builtin_amdgcn_perm(0x64646464u, wx, 0x04030402u)) - bias;
      }
    } else {
      const _Float16 s1 = __builtin_bit_cast(_Float16, st.s);
      const h2 s2 = {s1, s1};
      deq_i8_word(st.w[2 * c], s2, p[0], p[1]);
      deq_i8_word(st.w[2 * c + 1], s2, p[2], p[3]);
    }
  } else {
    const _Float16 s1 = __builtin_bit_cast(_Float16, st.s);
    const h2 s2 = {s1, s1};
    deq_i4_word(st.w[c], s2, p);
  }
  *reinterpret_cast<h8*>(sw + lds_off(wr, wc0 + c)) = pack_h8(p[0], p[1], p[2], p[3]);
}

// Writes activation chunk i (8 k) of this thread's staged segment to LDS. Activation rows past M
// were loaded from row M - 1: they only feed accumulator columns that are never stored.
template <class C>
__device__ __forceinline__ void gemm_store_x(const GemmStage<C>& st, int i, _Float16* sx, int xr,
                                             int xc0) {
  *reinterpret_cast<uint4*>(sx + lds_off(xr, xc0 + i)) = st.x[i];
}

// y[M, N] = x . W^T for one BN x BM tile of y^T. Waves form a 2 x 2 grid; wave (wn, wm) owns
// rows [wn BN/2, +BN/2) of the weight tile and [wm BM/2, +BM/2) of the activation tile, as
// TN x TM 32x32 MFMA tiles. Operand lane layout of v_mfma_f32_32x32x16_f16: lane l reads row
// l % 32, k chunk 2 ks + l / 32 of a 16-k step; accumulator register i of lane l holds
// row 8 (i / 4) + 4 (l / 32) + i % 4 of A (weight row) and column l % 32 (activation row).
// PC: per-channel INT8 (one scale per weight row), applied to the fp32 sums.
// SPLIT: blockIdx.z is one of gridDim.z equal k ranges (split K). The workgroup writes its fp32
// partial tile to sk.part and stops; qlinear_split_reduce_kernel, the next launch on the stream,
// adds the partials in split order and applies the epilogue.
// By value to every tiled-GEMM launch: the split partials, or the RoPE epilogue's operands.
struct GemmArgs {
  float* part;  // [tiles][splits][BN * BM] fp32 partial tiles
  EpiArgs ea;
};
// Epilogues of the tiled GEMM: y = the projection; SiLU(gate) * up; or q / k with RoPE and k / v
// appended to the pools (the RoPE epilogue writes no y).
constexpr int kGemmPlain = 0, kGemmSwiglu = 1, kGemmRope = 2;

// GEPI kGemmSwiglu: the weight is [gate; up] (N = 2 I rows) and y is I wide: each wave's two
// 32-row tiles hold 32 gate rows and the matching 32 up rows, and the epilogue writes
// fp16(silu(gate) * up) with the roundings of the projection followed by silu_mul (one fp16
// rounding of each projection, of the SiLU, of the product).
// GEPI kGemmRope: the weight is [q; k; v] with head_dim 64, so each wave's 64 rows are one head,
// dims 0..31 in its first tile and 32..63 in its second: the rotate_half partner of every value
// is in the same lane. The epilogue rounds the projection to fp16 as the plain launch does, then
// writes q with RoPE to ea.q_out and k with RoPE / v to the pools at each token's slot, with the
// arithmetic of rope_append.
template <int BITS, int BN, int BM, bool PC, int NTH, int NS, bool SPLIT = false,
          int GEPI = kGemmPlain>
__global__ __launch_bounds__(NTH, EDGERAG_GEMM_MIN_WG) void qlinear_gemm_kernel(
    const f16* __restrict__ x, int64_t xs, int32_t m, int32_t k,
    const uint8_t* __restrict__ packed, const f16* __restrict__ scales,
    const f16* __restrict__ bias, int32_t n, int32_t g, f16* __restrict__ y, int64_t ys,
    GemmArgs sk) {
  using C = GemmCfg<BITS, BN, BM, NTH>;
  static_assert(NS % 2 == 0, "the register ring must keep the LDS buffer parity of a step");
  constexpr int NWC = C::W_K / 8, NXC = C::X_BPT / 16;  // LDS chunks this thread stages per step
  __shared__ __attribute__((aligned(16))) _Float16 sw[2][BN * kLdsRow];
  __shared__ __attribute__((aligned(16))) _Float16 sx[2][BM * kLdsRow];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave % C::NWN, wm = wave / C::NWN;
  const int nb = blockIdx.x * BN, mb = blockIdx.y * BM;
  const int64_t row_bytes = BITS == 8 ? k : k / 2;
  const int groups = k / g;

  // Staging roles: weight row wr (segment wseg), activation row xr (segment xseg); the threads
  // of one row are adjacent lanes, so each global load instruction touches few cache lines.
  const int wr = tid / C::W_TPR, wseg = tid % C::W_TPR;
  const int xr = tid / C::X_TPR, xseg = tid % C::X_TPR;
  // Weight row of tile row lr. kGemmSwiglu: wave wn's rows 64 wn .. + 31 are gate rows (output
  // columns nb2 + 32 wn ..) and 64 wn + 32 .. + 63 the matching up rows.
  static_assert(GEPI == kGemmPlain || (C::TN == 2 && !SPLIT),
                "the SwiGLU / RoPE epilogues pair a wave's two 32-row tiles");
  const int inter = n / 2, nb2 = int(blockIdx.x) * (BN / 2);
  auto weight_row = [&](int lr) {
    if constexpr (GEPI == kGemmSwiglu) {
      const int c = min(nb2 + 32 * (lr / 64) + lr % 32, inter - 1);
      return (lr / 32) % 2 == 0 ? c : inter + c;
    } else {
      return min(nb + lr, n - 1);
    }
  };
  const int wrow_g = weight_row(wr);
  const uint8_t* wrow = packed + int64_t(wrow_g) * row_bytes + wseg * C::W_BPT;
  const f16* srow = scales + int64_t(wrow_g) * groups;
  const int wk_off = wseg * C::W_K;  // k offset of this thread's weight segment in a stage
  const f16* xrow = x + int64_t(min(mb + xr, m - 1)) * xs + xseg * (C::X_BPT / 2);
  const int wc0 = wk_off / 8, xc0 = xseg * (C::X_BPT / 16);

  f32x16 acc[C::TN][C::TM];
#pragma unroll
  for (int i = 0; i < C::TN; ++i)
#pragma unroll
    for (int j = 0; j < C::TM; ++j) acc[i][j] = f32x16{};

  const int nk = SPLIT ? k / kBK / int(gridDim.z) : k / kBK;  // 64-k steps of this workgroup
  const int kbase = SPLIT ? int(blockIdx.z) * nk * kBK : 0;
  const int col = lane & 31, half = lane >> 5;
  auto read_ops = [&](const _Float16* swb, const _Float16* sxb, int ks, h8 (&a)[C::TN],
                      h8 (&b)[C::TM]) {
#pragma unroll
    for (int i = 0; i < C::TN; ++i)
      a[i] = *reinterpret_cast<const h8*>(swb + lds_off(wn * (32 * C::TN) + 32 * i + col, 2 * ks + half));
#pragma unroll
    for (int j = 0; j < C::TM; ++j)
      b[j] = *reinterpret_cast<const h8*>(sxb + lds_off(wm * (32 * C::TM) + 32 * j + col, 2 * ks + half));
  };
  // One 64-k step on the LDS buffers of parity p, interleaved with staging the next step's
  // registers `stn` into the buffers of parity p ^ 1: each of the four 16-k MFMA steps is paired
  // with a share of the dequantisation and LDS writes, so the VALU and LDS work of the next step
  // overlaps this step's matrix-core work. The operands of 16-k step ks + 1 are read from LDS
  // before the MFMAs of step ks are issued, so their latency hides behind those MFMAs.
  auto step = [&](int p, const GemmStage<C>& stn) {
    constexpr int KS = kBK / 16, RA = EDGERAG_GEMM_READ_AHEAD;  // 16-k steps read ahead
    h8 a[RA + 1][C::TN], b[RA + 1][C::TM];
#pragma unroll
    for (int ks = 0; ks < RA && ks < KS; ++ks) read_ops(sw[p], sx[p], ks, a[ks], b[ks]);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + RA < KS) read_ops(sw[p], sx[p], ks + RA, a[(ks + RA) % (RA + 1)], b[(ks + RA) % (RA + 1)]);
#pragma unroll
      for (int c = ks * NWC / 4; c < (ks + 1) * NWC / 4; ++c)
        gemm_store_w<C, PC>(stn, c, sw[p ^ 1], wr, wc0);
#pragma unroll
      for (int i = ks * NXC / 4; i < (ks + 1) * NXC / 4; ++i)
        gemm_store_x<C>(stn, i, sx[p ^ 1], xr, xc0);
#pragma unroll
      for (int i = 0; i < C::TN; ++i)
#pragma unroll
        for (int j = 0; j < C::TM; ++j)
          acc[i][j] = mfma32(a[ks % (RA + 1)][i], b[ks % (RA + 1)][j], acc[i][j]);
    }
  };
  // One barrier per step: it orders this step's LDS writes (the next step's operands) before
  // their reads, and every wave's reads of a buffer before its next rewrite. Loads are
  // unconditional (a step past the end reloads the last one) so that the compiler never has to
  // wait for a load right after issuing it, and a step's loads are issued on every path (a last
  // partial round of the ring skips only LDS and matrix work, under a wave-uniform branch).
  // Epilogue operands: thread t < BN loads the scale (PC) and bias of weight row nb + t now (row
  // clamped into [0, N)), waits for them once the first stages' loads are in flight, and puts
  // them in LDS after the main loop for the lanes that write that row.
  __shared__ uint32_t ep_lds[BN];  // scale bits | bias bits << 16
  const uint16_t* scales16 = reinterpret_cast<const uint16_t*>(scales);
  const uint16_t* bias16 = reinterpret_cast<const uint16_t*>(bias);
  const int ep_row = weight_row(tid < BN ? tid : 0);
  uint32_t ep_s = PC ? scales16[ep_row] : 0u;
  uint32_t ep_b = bias != nullptr ? bias16[ep_row] : 0u;

  // NS register stages form a ring: step t is loaded into st[t % NS] right after the barrier that
  // ends step t - NS - 1 and is staged to LDS during step t - 1, so NS - 1 whole steps of matrix
  // work cover each load's latency. The loop is unrolled by NS so that every ring index is a
  // compile-time register name (and, NS being even, every LDS buffer parity a constant).
  GemmStage<C> st[NS];
  const int last = kbase + (nk - 1) * kBK;
  auto load = [&](GemmStage<C>& dst, int t) {
    gemm_load<C>(dst, min(kbase + t * kBK, last), wrow, srow, g, wk_off, xrow);
  };
#pragma unroll
  for (int j = 0; j < NS; ++j) load(st[j], j);
  issue_fence();
  asm volatile("" : "+v"(ep_s), "+v"(ep_b));
#pragma unroll
  for (int c = 0; c < NWC; ++c) gemm_store_w<C, PC>(st[0], c, sw[0], wr, wc0);
#pragma unroll
  for (int i = 0; i < NXC; ++i) gemm_store_x<C>(st[0], i, sx[0], xr, xc0);
  __syncthreads();
  load(st[0], NS);
  issue_fence();
  for (int kt = 0; kt < nk; kt += NS) {
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      if (j == 0 || kt + j < nk) step(j & 1, st[(j + 1) % NS]);
      __syncthreads();
      load(st[(j + 1) % NS], kt + j + NS + 1);
      issue_fence();
    }
  }

  if constexpr (SPLIT) {
    // Register group r of tile (i, j) of wave w: 64 consecutive float4 (one per lane) at
    // ((w TN + i) TM + j) 256 + 64 r, so the partial writes are contiguous 1 KiB stores.
    const int tile = int(blockIdx.y * gridDim.x + blockIdx.x);
    float4* part = reinterpret_cast<float4*>(sk.part) +
                   (int64_t(tile) * gridDim.z + blockIdx.z) * (BN * BM / 4);
#pragma unroll
    for (int i = 0; i < C::TN; ++i)
#pragma unroll
      for (int j = 0; j < C::TM; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          part[((wave * C::TN + i) * C::TM + j) * 256 + r * 64 + lane] =
              float4{acc[i][j][4 * r], acc[i][j][4 * r + 1], acc[i][j][4 * r + 2],
                     acc[i][j][4 * r + 3]};
    return;
  }

  // Epilogue: register 4q + r of tile (i, j) is y[mrow][nrow + r], 4 consecutive outputs per q,
  // stored as one 8-byte write when the row stride and the tile edge allow. (The main loop ended
  // with a barrier, so ep_lds is free of other uses.)
  if (tid < BN) ep_lds[tid] = ep_s | (ep_b << 16);
  __syncthreads();
  const bool vec_out = (ys % 4) == 0 && (reinterpret_cast<uintptr_t>(y) & 7) == 0;
  if constexpr (GEPI == kGemmSwiglu) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int lrow = wn * 64 + 8 * q + 4 * half;  // gate row in the tile
      const int ncol = nb2 + wn * 32 + 8 * q + 4 * half;  // output column
      float sg[4], bg[4], su[4], bu[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t eg = ep_lds[lrow + r], eu = ep_lds[lrow + 32 + r];
        sg[r] = float(__builtin_bit_cast(_Float16, uint16_t(eg & 0xFFFFu)));
        bg[r] = float(__builtin_bit_cast(_Float16, uint16_t(eg >> 16)));
        su[r] = float(__builtin_bit_cast(_Float16, uint16_t(eu & 0xFFFFu)));
        bu[r] = float(__builtin_bit_cast(_Float16, uint16_t(eu >> 16)));
      }
#pragma unroll
      for (int j = 0; j < C::TM; ++j) {
        const int mrow = mb + wm * (32 * C::TM) + 32 * j + col;
        if (mrow >= m) continue;
        f16* yr = y + int64_t(mrow) * ys;
        _Float16 o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float vg = PC ? sg[r] * acc[0][j][4 * q + r] + bg[r] : acc[0][j][4 * q + r] + bg[r];
          float vu = PC ? su[r] * acc[1][j][4 * q + r] + bu[r] : acc[1][j][4 * q + r] + bu[r];
          // The fp32 results first, then fp16, as the plain epilogue rounds them (left alone, the
          // compiler fuses each into one v_fma_mixlo_f16, which rounds once and can differ).
          asm volatile("" : "+v"(vg), "+v"(vu));
          const float gr = __half2float(__float2half_rn(vg));
          const float ur = __half2float(__float2half_rn(vu));
          o[r] = __builtin_bit_cast(_Float16, __float2half_rn(silu_rounded_f16(gr) * ur));
        }
        if (vec_out && ncol + 3 < inter) {
          const h2 lo = {o[0], o[1]}, hi = {o[2], o[3]};
          *reinterpret_cast<uint2*>(yr + ncol) = uint2{as_u32(lo), as_u32(hi)};
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (ncol + r < inter) yr[ncol + r] = __builtin_bit_cast(f16, o[r]);
        }
      }
    }
    return;
  }
  if constexpr (GEPI == kGemmRope) {
    const EpiArgs& ea = sk.ea;
    const int head = nb / 64 + wn;  // 64 rows per wave: one head
    const int heads = n / 64, nq = ea.n_q_heads, nkv = ea.n_kv_heads;
    const int64_t pool_rows = int64_t(ea.num_blocks) * ea.block_size;
    if (head >= heads) return;
    const bool rotate = head < nq + nkv;  // q or k; v is copied
    // The lane's dims: d0(q) .. + 3 in the first tile and 32 + d0(q) .. + 3 in the second.
#pragma unroll
    for (int j = 0; j < C::TM; ++j) {
      const int mrow = mb + wm * (32 * C::TM) + 32 * j + col;
      if (mrow >= m) continue;
      // Everything this row reads, before any store: its slot and the 8-byte runs of cos / sin
      // at its 16 dims (the stores could alias them as far as the compiler knows).
      const int64_t slot = head >= nq ? int64_t(ea.slots[mrow]) : 0;
      uint2 cv[4][2], sv[4][2];
      if (rotate) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const int64_t off = int64_t(mrow) * 64 + 32 * i + 8 * q + 4 * half;
            cv[q][i] = *reinterpret_cast<const uint2*>(ea.cos_tok + off);
            sv[q][i] = *reinterpret_cast<const uint2*>(ea.sin_tok + off);
          }
      }
      f16* dst;
      if (head < nq) {
        dst = ea.q_out + int64_t(mrow) * ea.q_st + int64_t(head) * 64;
      } else {
        if (slot < 0 || slot >= pool_rows) continue;
        const int kvh = rotate ? head - nq : head - nq - nkv;
        dst = (rotate ? ea.kpool : ea.vpool) +
              ((int64_t(kvh) * ea.num_blocks + slot / ea.block_size) * ea.block_size +
               slot % ea.block_size) * 64;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int d0 = 8 * q + 4 * half;
        // The projection rounded to fp16 as the plain epilogue rounds it (fp32 first).
        float v[2][4];
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint32_t e = ep_lds[wn * 64 + 32 * i + d0 + r];
            const float sc = float(__builtin_bit_cast(_Float16, uint16_t(e & 0xFFFFu)));
            const float bv = float(__builtin_bit_cast(_Float16, uint16_t(e >> 16)));
            float t = PC ? sc * acc[i][j][4 * q + r] + bv : acc[i][j][4 * q + r] + bv;
            asm volatile("" : "+v"(t));
            v[i][r] = __half2float(__float2half_rn(t));
          }
        f16 o[2][4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const _Float16* cw = reinterpret_cast<const _Float16*>(&cv[q][i]);
          const _Float16* sw = reinterpret_cast<const _Float16*>(&sv[q][i]);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if (rotate) {
              // One element at a time: paired across the two tiles, the vectoriser forms
              // two-float vector negations this target cannot select without packed fp32 ops.
              float own = v[i][r], partner = v[1 - i][r];
              asm volatile("" : "+v"(own), "+v"(partner));
              o[i][r] = rope_elem(own, partner, i == 1, float(cw[r]), float(sw[r]));
            } else {
              o[i][r] = __float2half_rn(v[i][r]);
            }
          }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          f16* p = dst + 32 * i + d0;
          if ((reinterpret_cast<uintptr_t>(p) & 7) == 0) {
            const h2 lo = {__builtin_bit_cast(_Float16, o[i][0]),
                           __builtin_bit_cast(_Float16, o[i][1])};
            const h2 hi = {__builtin_bit_cast(_Float16, o[i][2]),
                           __builtin_bit_cast(_Float16, o[i][3])};
            *reinterpret_cast<uint2*>(p) = uint2{as_u32(lo), as_u32(hi)};
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) p[r] = o[i][r];
          }
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < C::TN; ++i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int nrow_l = wn * (32 * C::TN) + 32 * i + 8 * q + 4 * half;  // row within the tile
      const int nrow = nb + nrow_l;
      float sc[4], bv[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t e = ep_lds[nrow_l + r];
        sc[r] = float(__builtin_bit_cast(_Float16, uint16_t(e & 0xFFFFu)));
        bv[r] = float(__builtin_bit_cast(_Float16, uint16_t(e >> 16)));
      }
#pragma unroll
      for (int j = 0; j < C::TM; ++j) {
        const int mrow = mb + wm * (32 * C::TM) + 32 * j + col;
        if (mrow >= m) continue;
        f16* yr = y + int64_t(mrow) * ys;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = PC ? sc[r] * acc[i][j][4 * q + r] + bv[r]
                                              : acc[i][j][4 * q + r] + bv[r];
        if (vec_out && nrow + 3 < n) {
          const h2 lo = {_Float16(v[0]), _Float16(v[1])}, hi = {_Float16(v[2]), _Float16(v[3])};
          *reinterpret_cast<uint2*>(yr + nrow) = uint2{as_u32(lo), as_u32(hi)};
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (nrow + r < n) yr[nrow + r] = __float2half_rn(v[r]);
        }
      }
    }
  }
}

// Loads in flight per batch, bounded by the activation registers (MT m-tiles x k-steps).
template <int BITS, int MT>
constexpr int skinny_u() {
  return BITS == 8 ? (MT <= 2 ? 4 : 2) : (MT <= 2 ? 2 : 1);
}

template <int BITS, int NT, int MT>
void launch_skinny(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                   const f16* scales, const f16* bias, int32_t n, int32_t g, f16* y, int64_t ys,
                   hipStream_t s) {
  constexpr int U = skinny_u<BITS, MT>();
  // Waves per workgroup split K: enough that each holds about one batch of U chunks, at most
  // kMaxSkinnyWaves -- or 16 for one-tile, one-m-tile launches over a long K (the down
  // projection), where 1024-thread workgroups still fit the register file and halve the round
  // trips per wave. The split depends on K, the row tiles (N) and the m-tiles (M), never on the
  // values, so a launch shape always sums a row in the same order.
  const int nkb = k / SkinnyCfg<BITS>::KB;
  const int kw_max = (NT == 1 && MT == 1 && nkb > kMaxSkinnyWaves * U) ? 16 : kMaxSkinnyWaves;
  int kw = 1;
  while (kw < kw_max && kw * U < nkb) kw *= 2;
  const int per_wave = (nkb + kw - 1) / kw;
  if constexpr (NT > 1) {
    // Two super-batches of two row tiles would not fit the register file: one tile per wave.
    if (per_wave > U) {
      launch_skinny<BITS, 1, MT>(x, xs, m, k, packed, scales, bias, n, g, y, ys, s);
      return;
    }
  }
  const unsigned blocks = unsigned((n + 16 * NT - 1) / (16 * NT));
  const bool pg = k / g > 1;
#define EDGERAG_SKINNY(NB, PG, KWM)                                                            \
  hipLaunchKernelGGL((qlinear_skinny_kernel<BITS, NT, MT, U, NB, PG, KWM>), dim3(blocks),      \
                     dim3(kw * kWave), 0, s, x, xs, packed, scales, m, k, n, g, kw, bias, y, ys)
  if (kw > kMaxSkinnyWaves) {
    if constexpr (NT == 1 && MT == 1) {
      if (per_wave <= U) {
        if (pg) EDGERAG_SKINNY(1, true, 16); else EDGERAG_SKINNY(1, false, 16);
      } else {
        if (pg) EDGERAG_SKINNY(2, true, 16); else EDGERAG_SKINNY(2, false, 16);
      }
    }
  } else if (per_wave <= U) {
    if (pg) EDGERAG_SKINNY(1, true, 8); else EDGERAG_SKINNY(1, false, 8);
  } else {
    if (pg) EDGERAG_SKINNY(2, true, 8); else EDGERAG_SKINNY(2, false, 8);
  }
#undef EDGERAG_SKINNY
}

template <int BITS, int BN, int BM, int NTH, int NS>
void launch_gemm(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                 const f16* scales, const f16* bias, int32_t n, int32_t g, f16* y, int64_t ys,
                 hipStream_t s) {
  const dim3 grid(unsigned((n + BN - 1) / BN), unsigned((m + BM - 1) / BM));
  const GemmArgs none{nullptr};
  if (BITS == 8 && g == k)
    hipLaunchKernelGGL((qlinear_gemm_kernel<BITS, BN, BM, BITS == 8, NTH, NS>), grid, dim3(NTH),
                       0, s, x, xs, m, k, packed, scales, bias, n, g, y, ys, none);
  else
    hipLaunchKernelGGL((qlinear_gemm_kernel<BITS, BN, BM, false, NTH, NS>), grid, dim3(NTH), 0, s,
                       x, xs, m, k, packed, scales, bias, n, g, y, ys, none);
}

// SwiGLU GEMM: 128 weight rows per tile (64 gate + 64 up), so the grid covers I = N / 2 output
// columns 64 at a time: the same workgroups and k order as the plain launch of the [gate; up]
// weight with BN = 128.
template <int BM, int NTH, int NS>
void launch_gemm_swiglu(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                        const f16* scales, const f16* bias, int32_t n, f16* y, int64_t ys,
                        hipStream_t s) {
  const dim3 grid(unsigned((n / 2 + 63) / 64), unsigned((m + BM - 1) / BM));
  const GemmArgs none{nullptr};
  hipLaunchKernelGGL((qlinear_gemm_kernel<8, 128, BM, true, NTH, NS, false, kGemmSwiglu>), grid,
                     dim3(NTH), 0, s, x, xs, m, k, packed, scales, bias, n, k, y, ys, none);
}

// RoPE GEMM: the plain launch's 128-row weight tiles (two 64-dim heads per workgroup); writes q
// to ea.q_out and k / v to the pools, no y.
template <int BM, int NTH, int NS>
void launch_gemm_rope(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                      const f16* scales, const f16* bias, int32_t n, const EpiArgs& ea,
                      hipStream_t s) {
  const dim3 grid(unsigned((n + 127) / 128), unsigned((m + BM - 1) / BM));
  const GemmArgs ga{nullptr, ea};
  hipLaunchKernelGGL((qlinear_gemm_kernel<8, 128, BM, true, NTH, NS, false, kGemmRope>), grid,
                     dim3(NTH), 0, s, x, xs, m, k, packed, scales, bias, n, k, nullptr, 0, ga);
}

// Split-K launches use 64x64 tiles: the tile grid alone would leave CUs idle.
constexpr int kSplitTile = 64;
static_assert(EDGERAG_SPLITK_MAX <= 16, "the reduce launch is instantiated for 2, 4, 8, 16 splits");
// Partial tiles a split may write: EDGERAG_QUANT_WORKSPACE_MAX / 16 KB.
constexpr int64_t kSplitMaxPartials =
    int64_t(EDGERAG_QUANT_WORKSPACE_MAX) / (kSplitTile * kSplitTile * 4);

// Sums the split partials of the 64x64 tiles (as qlinear_gemm_kernel<..., SPLIT> wrote them, with
// its 2 x 2 grid of 32x32 wave tiles) in split order and writes y = fp16(scale * sum + bias)
// (PC) or fp16(sum + bias). Thread t of a tile owns float4 t: wave w = t / 256, register group
// r = t / 64 % 4, lane l = t % 64, i.e. weight rows 32 (w % 2) + 8 r + 4 (l / 32) + 0..3 and token
// row 32 (w / 2) + l % 32 of the tile: four consecutive outputs, one 8-byte store.
template <bool PC, int S>
__global__ __launch_bounds__(256) void qlinear_split_reduce_kernel(
    const float4* __restrict__ part, int32_t tiles_x, int32_t m, int32_t n,
    const f16* __restrict__ scales, const f16* __restrict__ bias, f16* __restrict__ y,
    int64_t ys) {
  constexpr int kTileF4 = kSplitTile * kSplitTile / 4;  // 1024 float4 per tile
  const int tile = int(blockIdx.x) / (kTileF4 / 256);
  const int t = (int(blockIdx.x) % (kTileF4 / 256)) * 256 + int(threadIdx.x);
  const int w = t / 256, r = (t / 64) % 4, l = t % 64;
  const int nrow = (tile % tiles_x) * kSplitTile + 32 * (w % 2) + 8 * r + 4 * (l / 32);
  const int mrow = (tile / tiles_x) * kSplitTile + 32 * (w / 2) + l % 32;
  const float4* p = part + int64_t(tile) * S * kTileF4 + t;
  float4 pv[S];
#pragma unroll
  for (int z = 0; z < S; ++z) pv[z] = p[int64_t(z) * kTileF4];  // all loads in flight
  float4 sum = pv[0];
#pragma unroll
  for (int z = 1; z < S; ++z) {
    sum.x += pv[z].x;
    sum.y += pv[z].y;
    sum.z += pv[z].z;
    sum.w += pv[z].w;
  }
  if (mrow >= m) return;
  const float s4[4] = {sum.x, sum.y, sum.z, sum.w};
  float v[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = min(nrow + q, n - 1);
    const float sc = PC ? __half2float(scales[row]) : 1.f;
    const float b = bias != nullptr ? __half2float(bias[row]) : 0.f;
    v[q] = PC ? sc * s4[q] + b : s4[q] + b;
  }
  f16* yr = y + int64_t(mrow) * ys;
  if (nrow + 3 < n && (ys % 4) == 0 && (reinterpret_cast<uintptr_t>(y) & 7) == 0) {
    const h2 lo = {_Float16(v[0]), _Float16(v[1])}, hi = {_Float16(v[2]), _Float16(v[3])};
    *reinterpret_cast<uint2*>(yr + nrow) = uint2{as_u32(lo), as_u32(hi)};
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (nrow + q < n) yr[nrow + q] = __float2half_rn(v[q]);
  }
}

template <int BITS>
void launch_gemm_split(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                       const f16* scales, const f16* bias, int32_t n, int32_t g, f16* y,
                       int64_t ys, const SplitPlan& p, void* ws, hipStream_t s) {
  const int tiles_x = (n + kSplitTile - 1) / kSplitTile;
  const dim3 grid(unsigned(tiles_x), unsigned((m + kSplitTile - 1) / kSplitTile),
                  unsigned(p.splits));
  float* part = static_cast<float*>(ws);
  const GemmArgs sk{part};
  constexpr int T = kSplitTile;
  const bool pc = BITS == 8 && g == k;
  if (pc)
    hipLaunchKernelGGL((qlinear_gemm_kernel<BITS, T, T, BITS == 8, EDGERAG_GEMM_THREADS_64,
                                            EDGERAG_GEMM_STAGES_64, true>),
                       grid, dim3(EDGERAG_GEMM_THREADS_64), 0, s, x, xs, m, k, packed, scales,
                       bias, n, g, y, ys, sk);
  else
    hipLaunchKernelGGL((qlinear_gemm_kernel<BITS, T, T, false, EDGERAG_GEMM_THREADS_64,
                                            EDGERAG_GEMM_STAGES_64, true>),
                       grid, dim3(EDGERAG_GEMM_THREADS_64), 0, s, x, xs, m, k, packed, scales,
                       bias, n, g, y, ys, sk);
  const unsigned rblocks = unsigned(int64_t(grid.x) * grid.y * (T * T / 4 / 256));
  const float4* part4 = reinterpret_cast<const float4*>(part);
#define EDGERAG_SPLIT_REDUCE(SPLITS)                                                              \
  do {                                                                                            \
    if (pc)                                                                                       \
      hipLaunchKernelGGL((qlinear_split_reduce_kernel<true, SPLITS>), dim3(rblocks), dim3(256),   \
                         0, s, part4, tiles_x, m, n, scales, bias, y, ys);                        \
    else                                                                                          \
      hipLaunchKernelGGL((qlinear_split_reduce_kernel<false, SPLITS>), dim3(rblocks), dim3(256),  \
                         0, s, part4, tiles_x, m, n, scales, bias, y, ys);                        \
  } while (0)
  switch (p.splits) {
    case 2: EDGERAG_SPLIT_REDUCE(2); break;
    case 4: EDGERAG_SPLIT_REDUCE(4); break;
    case 8: EDGERAG_SPLIT_REDUCE(8); break;
    default: EDGERAG_SPLIT_REDUCE(16); break;
  }
#undef EDGERAG_SPLIT_REDUCE
}

// The streaming kernel's shape: k-slices F and row tiles NT from N alone (two k-slices when
// 16-row tiles would leave CUs idle, two row tiles when 32-row tiles still cover them), waves KW and
// steps per batch U from K alone, so that a row's summation order, and so its bits, do not depend
// on M or on the other rows of the launch. Returns false when the shape does not fit (the caller
// then uses the skinny kernel).
template <int F, int NT, int MT, int KW, int U, int EPI, bool NORM, int RH = 0>
void launch_stream(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                   const f16* scales, const f16* bias, int32_t n, f16* y, int64_t ys,
                   const EpiArgs& ea, hipStream_t s) {
  constexpr int rows = NT * 16 / F;
  // SwiGLU: one workgroup per 16 / F activation columns (a gate tile and its up twin); RoPE: one
  // per NT 16 / F rows, half of them elements of a head's first half and half their rotate_half
  // twins.
  const unsigned blocks = EPI == kEpiSwiglu ? unsigned((n / 2 + 16 / F - 1) / (16 / F))
                                            : unsigned((n + rows - 1) / rows);
  // One token on two k-slices: its activations go through LDS (X1), the same values in the same
  // operands. (With one k-slice, 16 lane rows share each operand load and a batch holds half
  // the steps: measured 8.16 -> 8.41 us on 2048->16384, so those keep the direct loads.)
  constexpr bool kX1 = MT == 1 && F == 2;
#define EDGERAG_STREAM_X(EX, X1)                                                                 \
  hipLaunchKernelGGL((qlinear_stream_kernel<F, NT, MT, KW, U, EX, EPI, NORM, X1, RH>),            \
                     dim3(blocks), dim3(KW * kWave), 0, s, x, xs, m, k, packed, scales, bias, n, y, \
                     ys, ea)
  const bool exact = (k / (64 * F)) % (KW * U) == 0;
  if (kX1 && m == 1) {
    if (exact) EDGERAG_STREAM_X(true, kX1); else EDGERAG_STREAM_X(false, kX1);
  } else {
    if (exact) EDGERAG_STREAM_X(true, false); else EDGERAG_STREAM_X(false, false);
  }
#undef EDGERAG_STREAM_X
}

// Waves per workgroup and steps per batch of the streaming kernel for F k-slices, NT row tiles
// and MT m-tiles: one batch of at most 8 steps per wave; at least 4 waves (one per SIMD), or 8
// for two row tiles (one output per thread); at most 16 for one k-slice with one row tile and
// up to two m-tiles, else 8 (the registers of 16 such waves would not fit; two k-slices stop at
// 8 for one m-tile too, so that their one- and two-m-tile launches split K alike). The waves
// depend on K, F, NT and MT; for up to 16 tokens MT does not change them, so a decode token's
// summation order, and so its bits, depend on K and N alone. Several m-tiles take batches of 4
// steps to bound their activation registers.
struct StreamWaves {
  int kw;
  bool u8;
};
StreamWaves stream_waves(int f, int nt, int mt, int k) {
  const int nc = k / (64 * f);
  const int kw_min = nt == 1 ? 4 : 8;
  const int kw_max = nt == 1 && mt < 4 && f == 1 ? 16 : 8;
  int kw = kw_min;
  while (kw < kw_max && kw * 8 < nc) kw *= 2;
  return {kw, mt == 1 && (nc + kw - 1) / kw > 4 && nc >= 8};
}

// Launches the shape with the given waves (KW in {4, 8, 16}) and batch (U in {4, 8}).
template <int F, int NT, int MT, int EPI, bool NORM = false, int RH = 0>
void launch_stream_w(StreamWaves sw, const f16* x, int64_t xs, int32_t m, int32_t k,
                     const uint8_t* packed, const f16* scales, const f16* bias, int32_t n, f16* y,
                     int64_t ys, const EpiArgs& ea, hipStream_t s) {
#define EDGERAG_STREAM(KW)                                                                      \
  do {                                                                                         \
    if constexpr (MT == 1) {                                                                   \
      if (sw.u8) {                                                                             \
        launch_stream<F, NT, MT, KW, 8, EPI, NORM, RH>(x, xs, m, k, packed, scales, bias, n, y, \
                                                       ys, ea, s);                             \
        return;                                                                                \
      }                                                                                        \
    }                                                                                          \
    launch_stream<F, NT, MT, KW, 4, EPI, NORM, RH>(x, xs, m, k, packed, scales, bias, n, y, ys,  \
                                                   ea, s);                                     \
    return;                                                                                    \
  } while (0)
  // Only the combinations stream_waves can pick are instantiated: 4 waves for one row tile (and
  // for RoPE launches, which take the waves of the plain one-tile launch), 16 where registers fit.
  if constexpr (NT == 1 || EPI == kEpiRope) {
    if (sw.kw == 4) EDGERAG_STREAM(4);
  }
  if constexpr (NT == 1 && MT < 4 && F == 1) {
    if (sw.kw == 16) EDGERAG_STREAM(16);
  }
  EDGERAG_STREAM(8);
#undef EDGERAG_STREAM
}

template <int F, int NT, int MT, int EPI = kEpiPlain, bool NORM = false>
void launch_stream_k(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                     const f16* scales, const f16* bias, int32_t n, f16* y, int64_t ys,
                     hipStream_t s, const EpiArgs& ea = EpiArgs{}) {
  launch_stream_w<F, NT, MT, EPI, NORM>(stream_waves(F, NT, MT, k), x, xs, m, k, packed, scales,
                                        bias, n, y, ys, ea, s);
}

// The k-slices (1 or 2) dispatch_stream uses for (M, K, N), 0 when it does not take the shape:
// two (8-row tiles) when 16-row tiles would leave CUs idle (N < 4096) for up to 16 tokens, and for
// 17..32 tokens (M = 32, K 8192 -> N 2048: 21.4 -> 18.8 us; for 33..64 tokens two such launches
// measured slower than one k-slice). Also when the one-slice workgroups (one per 16 rows, fewer
// than 512) would give some CUs two and others one while the 8-row ones are spread more evenly:
// N = 6144 (the q/k/v projection) 384 -> 768 workgroups, 6.41 -> 4.80 us at M = 1, 7.58 -> 6.53
// us at M = 8; N = 4096 (256 workgroups either way) gained nothing. The rule holds for all of
// 1..16 tokens so that a decode token's bits stay independent of the batch, although at 16 tokens
// the two 8-token m-tiles cost more than they gain (8.9 -> 11.4 us).
int stream_slices(int32_t m, int32_t k, int32_t n) {
  const int64_t tiles16 = (int64_t(n) + 15) / 16;
  const bool one = k % 64 == 0 && k / 64 >= 4, two = k % 128 == 0 && k / 128 >= 4;
  if (m < 1 || m > 64) return 0;
  if (EDGERAG_STREAM_NARROW_F2 && m > 16 && m <= 32 && tiles16 < 256 && two) return 2;
  if (m > 16) return one ? 1 : 0;
  if (tiles16 < EDGERAG_STREAM_F2_TILES) return two ? 2 : 0;
  if (tiles16 < EDGERAG_STREAM_NT2_TILES && two) {
    // Rounds of workgroups over the 256 CUs, against a perfectly even spread.
    auto imbalance = [](int64_t wgs) { return double((wgs + 255) / 256) * 256.0 / double(wgs); };
    if (imbalance(2 * tiles16) < imbalance(tiles16) - 1e-9) return 2;
  }
  return one ? 1 : 0;
}

bool dispatch_stream(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                     const f16* scales, const f16* bias, int32_t n, f16* y, int64_t ys,
                     hipStream_t s) {
  const int slices = stream_slices(m, k, n);
  if (slices == 0) return false;
  if (slices == 2) {  // 8-row tiles and 8-token m-tiles
    if (m <= 8) launch_stream_k<2, 1, 1>(x, xs, m, k, packed, scales, bias, n, y, ys, s);
    else if (m <= 16) launch_stream_k<2, 1, 2>(x, xs, m, k, packed, scales, bias, n, y, ys, s);
    else launch_stream_k<2, 1, 4>(x, xs, m, k, packed, scales, bias, n, y, ys, s);
    return true;
  }
  // One k-slice: 16-row tiles (two per workgroup when 32-row workgroups still cover the CUs),
  // up to four 16-token m-tiles.
  const bool two = (int64_t(n) + 15) / 16 >= EDGERAG_STREAM_NT2_TILES;
  if (m <= 16) {
    if (two) launch_stream_k<1, 2, 1>(x, xs, m, k, packed, scales, bias, n, y, ys, s);
    else launch_stream_k<1, 1, 1>(x, xs, m, k, packed, scales, bias, n, y, ys, s);
  } else if (m <= 32) {
    if (two) launch_stream_k<1, 2, 2>(x, xs, m, k, packed, scales, bias, n, y, ys, s);
    else launch_stream_k<1, 1, 2>(x, xs, m, k, packed, scales, bias, n, y, ys, s);
  } else {
    if (two) launch_stream_k<1, 2, 4>(x, xs, m, k, packed, scales, bias, n, y, ys, s);
    else launch_stream_k<1, 1, 4>(x, xs, m, k, packed, scales, bias, n, y, ys, s);
  }
  return true;
}

// The residual-epilogue form of the plain launch for decode batches (M <= 16): same shapes, so the
// same bits of y. Returns the number of workgroups (partial sums per token), 0 if not covered.
int residual_parts(int32_t m, int32_t k, int32_t n) {
  if (m > 16 || m > EDGERAG_STREAM_MAX_M) return 0;
  const int slices = stream_slices(m, k, n);
  if (slices == 0) return 0;
  const int rows = slices == 2 ? 8 : ((int64_t(n) + 15) / 16 >= EDGERAG_STREAM_NT2_TILES ? 32 : 16);
  return (n + rows - 1) / rows;
}

void dispatch_stream_residual(const f16* x, int64_t xs, int32_t m, int32_t k,
                              const uint8_t* packed, const f16* scales, const f16* bias, int32_t n,
                              const EpiArgs& ea, hipStream_t s) {
  if (stream_slices(m, k, n) == 2) {
    if (m <= 8)
      launch_stream_k<2, 1, 1, kEpiResidual>(x, xs, m, k, packed, scales, bias, n, nullptr, 0, s,
                                             ea);
    else
      launch_stream_k<2, 1, 2, kEpiResidual>(x, xs, m, k, packed, scales, bias, n, nullptr, 0, s,
                                             ea);
  } else if ((int64_t(n) + 15) / 16 >= EDGERAG_STREAM_NT2_TILES) {
    launch_stream_k<1, 2, 1, kEpiResidual>(x, xs, m, k, packed, scales, bias, n, nullptr, 0, s, ea);
  } else {
    launch_stream_k<1, 1, 1, kEpiResidual>(x, xs, m, k, packed, scales, bias, n, nullptr, 0, s, ea);
  }
}

// The streaming shapes with two row tiles of one k-slice: the only ones the SwiGLU form covers.
// dispatch_stream picks exactly these for the same (M, K, N), so the fused launch computes the
// same gate and up bits as the plain one.
// The tiled GEMM's tile for M x N: the largest whose grid still covers the 256 CUs, 128x128,
// else 128x64 (this test), else 64x64.
inline bool gemm_tiles_128x64(int32_t m, int32_t n) {
  const int64_t tn = (n + 127) / 128;
  return tn * ((m + 127) / 128) < EDGERAG_GEMM_TARGET_WGS &&
         tn * ((m + 63) / 64) >= EDGERAG_GEMM_TARGET_WGS;
}

bool stream_swiglu_shape(int32_t m, int32_t k, int32_t n) {
  return m <= EDGERAG_STREAM_MAX_M && stream_slices(m, k, n) == 1 && n % 2 == 0 &&
         (int64_t(n) + 15) / 16 >= EDGERAG_STREAM_NT2_TILES;
}

// The tiled GEMM with the SwiGLU epilogue (per-channel INT8, M > 64) where the plain launch of
// the [gate; up] weight uses 128-row weight tiles (128x128 or 128x64), so that the fused launch
// sums every output in the plain launch's order; a remainder the plain launch hands to the
// streaming path goes to the streaming SwiGLU kernel.
bool gemm_swiglu_shape(int32_t m, int32_t k, int32_t n) {
  if (m <= EDGERAG_SKINNY_MAX_M || n % 2 != 0 || k % kBK != 0) return false;
  const int rem = m % 64;
  if (rem > 0 && rem <= 16 && m - rem >= 128 && !gemm_tiles_128x64(m, n))
    return gemm_swiglu_shape(m - rem, k, n) && stream_swiglu_shape(rem, k, n);
  return int64_t((n + 127) / 128) * ((m + 127) / 128) >= EDGERAG_GEMM_TARGET_WGS ||
         gemm_tiles_128x64(m, n);
}

void dispatch_stream_swiglu(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                            const f16* scales, const f16* bias, int32_t n, f16* y, int64_t ys,
                            const EpiArgs& ea, hipStream_t s);

void dispatch_gemm_swiglu(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                          const f16* scales, const f16* bias, int32_t n, f16* y, int64_t ys,
                          hipStream_t s) {
  const int rem = m % 64;
  if (rem > 0 && rem <= 16 && m - rem >= 128 && !gemm_tiles_128x64(m, n)) {
    dispatch_gemm_swiglu(x, xs, m - rem, k, packed, scales, bias, n, y, ys, s);
    dispatch_stream_swiglu(x + int64_t(m - rem) * xs, xs, rem, k, packed, scales, bias, n,
                           y + int64_t(m - rem) * ys, ys, EpiArgs{}, s);
    return;
  }
  if (int64_t((n + 127) / 128) * ((m + 127) / 128) >= EDGERAG_GEMM_TARGET_WGS)
    launch_gemm_swiglu<128, EDGERAG_GEMM_THREADS_128, EDGERAG_GEMM_STAGES_128>(
        x, xs, m, k, packed, scales, bias, n, y, ys, s);
  else
    launch_gemm_swiglu<64, EDGERAG_GEMM_THREADS_128x64, EDGERAG_GEMM_STAGES_128x64>(
        x, xs, m, k, packed, scales, bias, n, y, ys, s);
}

void dispatch_stream_swiglu(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                            const f16* scales, const f16* bias, int32_t n, f16* y, int64_t ys,
                            const EpiArgs& ea, hipStream_t s) {
  if (ea.norm_part != nullptr)  // normed input: decode batches of up to 16 tokens
    launch_stream_k<1, 2, 1, kEpiSwiglu, true>(x, xs, m, k, packed, scales, bias, n, y, ys, s, ea);
  else if (m <= 16)
    launch_stream_k<1, 2, 1, kEpiSwiglu>(x, xs, m, k, packed, scales, bias, n, y, ys, s);
  else if (m <= 32)
    launch_stream_k<1, 2, 2, kEpiSwiglu>(x, xs, m, k, packed, scales, bias, n, y, ys, s);
  else
    launch_stream_k<1, 2, 4, kEpiSwiglu>(x, xs, m, k, packed, scales, bias, n, y, ys, s);
}

template <int BITS>
void dispatch(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
              const f16* scales, const f16* bias, int32_t n, int32_t g, f16* y, int64_t ys,
              hipStream_t s) {
  if constexpr (BITS == 8) {
    if (g == k && m <= EDGERAG_STREAM_MAX_M &&
        dispatch_stream(x, xs, m, k, packed, scales, bias, n, y, ys, s))
      return;
  }
  if (m <= EDGERAG_SKINNY_MAX_M) {
    const bool wide = (n + 31) / 32 >= 256;  // enough workgroups with 32 rows each
    if (m <= 16) {
      if (wide) launch_skinny<BITS, 2, 1>(x, xs, m, k, packed, scales, bias, n, g, y, ys, s);
      else launch_skinny<BITS, 1, 1>(x, xs, m, k, packed, scales, bias, n, g, y, ys, s);
    } else if (m <= 32) {
      launch_skinny<BITS, 1, 2>(x, xs, m, k, packed, scales, bias, n, g, y, ys, s);
    } else {
      launch_skinny<BITS, 1, 4>(x, xs, m, k, packed, scales, bias, n, g, y, ys, s);
    }
    return;
  }
  // A remainder of at most 16 rows past a whole number of 64-row tiles (the decode tokens packed
  // after a prefill chunk) runs on the streaming (or skinny) path as a second launch, where an
  // extra row of 128x128 or 64x64 tiles would be mostly empty. 128x64 tiles (up to three
  // workgroups per CU) take the extra row at almost no cost, less than a second pass over the
  // weights (2048->6144, M = 519: 28.1 against 33.5 us; M = 512: 28.2).
  const int rem = m % 64;
  if (rem > 0 && rem <= 16 && m - rem >= 128 && !gemm_tiles_128x64(m, n)) {
    dispatch<BITS>(x, xs, m - rem, k, packed, scales, bias, n, g, y, ys, s);
    dispatch<BITS>(x + int64_t(m - rem) * xs, xs, rem, k, packed, scales, bias, n, g,
                   y + int64_t(m - rem) * ys, ys, s);
    return;
  }
  // Tiles: the largest whose grid still covers the 256 CUs.
  const int64_t t128 = int64_t((n + 127) / 128) * ((m + 127) / 128);
  if (t128 >= EDGERAG_GEMM_TARGET_WGS)
    launch_gemm<BITS, 128, 128, EDGERAG_GEMM_THREADS_128, EDGERAG_GEMM_STAGES_128>(
        x, xs, m, k, packed, scales, bias, n, g, y, ys, s);
  else if (gemm_tiles_128x64(m, n))
    launch_gemm<BITS, 128, 64, EDGERAG_GEMM_THREADS_128x64, EDGERAG_GEMM_STAGES_128x64>(
        x, xs, m, k, packed, scales, bias, n, g, y, ys, s);
  else
    launch_gemm<BITS, 64, 64, EDGERAG_GEMM_THREADS_64, EDGERAG_GEMM_STAGES_64>(
        x, xs, m, k, packed, scales, bias, n, g, y, ys, s);
}

}  // namespace

// The workspace route of the tiled GEMM (edgerag_quant_linear_ws): batches of 17..64 tokens where
// the streaming / skinny GEMV, which re-reads every activation row once per 16-row tile, is
// slower (measured crossovers on MI355X, config-4 and config-5 shapes: from 17 tokens for
// K >= 4096 or N >= 16384, from 40 tokens for layers of more than 4M codes, from 64 tokens for
// 2M..4M codes, never for smaller ones), and larger M whose 64x64 tile grid leaves CUs idle. Its
// time is modelled in 64-k steps of one workgroup:
//   cost(s) = fixed(s) + (steps per split) x (rounds of workgroups over the 256 CUs),
// fixed(1) = 0 and fixed(s > 1) = EDGERAG_SPLITK_FIXED_STEPS (the partial tiles' round trip and
// the second launch); the plan takes the cheapest s of 1, 2, 4, .. EDGERAG_SPLITK_MAX (each split
// at least EDGERAG_SPLITK_MIN_STEPS steps, all splits equal).
SplitPlan qlinear_split_plan(int32_t m, int32_t k, int32_t n, int32_t bits, int32_t g) {
  SplitPlan p{0, 0};
  // At most 16 rows past whole 64-row tiles go to the streaming path (launch_qlinear_split): the
  // plan covers the tiles.
  if (m > EDGERAG_SKINNY_MAX_M && m % 64 > 0 && m % 64 <= 16 && m - m % 64 >= 128) m -= m % 64;
  if (m < 17 || n <= 0 || k % kBK != 0) return p;
  if ((bits != 8 && bits != 4) || g % 32 != 0) return p;
  const int64_t tiles = int64_t((n + kSplitTile - 1) / kSplitTile) *
                        ((m + kSplitTile - 1) / kSplitTile);
  if (m > EDGERAG_SKINNY_MAX_M) {
    // Larger M: only where the plain launch would also use 64x64 tiles.
    const int64_t t128x64 = int64_t((n + 127) / 128) * ((m + 63) / 64);
    if (t128x64 >= EDGERAG_GEMM_TARGET_WGS) return p;
  } else if (m < 40) {
    if (k < 4096 && n < 16384) return p;
  } else {
    const int64_t codes = int64_t(n) * k;
    if (codes <= (int64_t(1) << 22) && (m < 64 || codes < (int64_t(1) << 21))) return p;
  }
  const int nk = k / kBK;
  auto rounds = [&](int64_t wgs) {
    return (wgs + EDGERAG_GEMM_TARGET_WGS - 1) / EDGERAG_GEMM_TARGET_WGS;
  };
  int best = 1;
  int64_t best_cost = int64_t(nk) * rounds(tiles);
  for (int sp = 2; sp <= EDGERAG_SPLITK_MAX; sp *= 2) {
    if (nk % sp != 0 || nk / sp < EDGERAG_SPLITK_MIN_STEPS) break;
    if (tiles * sp > kSplitMaxPartials) break;  // the workspace bound
    const int64_t cost = EDGERAG_SPLITK_FIXED_STEPS + int64_t(nk / sp) * rounds(tiles * sp);
    if (cost < best_cost) {
      best = sp;
      best_cost = cost;
    }
  }
  p.splits = best;
  p.bytes = best > 1 ? tiles * best * kSplitTile * kSplitTile * 4 : 0;
  return p;
}

bool launch_qlinear_split(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                          const f16* scales, const f16* bias, int32_t n, int32_t bits, int32_t g,
                          f16* y, int64_t ys, void* ws, int64_t ws_bytes, hipStream_t s) {
  // As in dispatch: at most 16 rows past whole 64-row tiles run on the streaming path, the tiles
  // on this route (8192->2048, M = 519: 47 against 53 us as one launch with a ninth tile row).
  const int rem = m % 64;
  if (m > EDGERAG_SKINNY_MAX_M && rem > 0 && rem <= 16 && m - rem >= 128) {
    if (!launch_qlinear_split(x, xs, m - rem, k, packed, scales, bias, n, bits, g, y, ys, ws,
                              ws_bytes, s))
      return false;  // nothing launched: the caller runs the whole product on the plain path
    if (bits == 8)
      dispatch<8>(x + int64_t(m - rem) * xs, xs, rem, k, packed, scales, bias, n, g,
                  y + int64_t(m - rem) * ys, ys, s);
    else
      dispatch<4>(x + int64_t(m - rem) * xs, xs, rem, k, packed, scales, bias, n, g,
                  y + int64_t(m - rem) * ys, ys, s);
    return true;
  }
  const SplitPlan p = qlinear_split_plan(m, k, n, bits, g);
  if (p.splits < 1 ||
      (p.splits > 1 && (ws == nullptr || ws_bytes < p.bytes || !aligned16(ws))))  // float4 partials
    return false;
  constexpr int T = kSplitTile;
  if (p.splits == 1) {
    if (bits == 8)
      launch_gemm<8, T, T, EDGERAG_GEMM_THREADS_64, EDGERAG_GEMM_STAGES_64>(
          x, xs, m, k, packed, scales, bias, n, g, y, ys, s);
    else
      launch_gemm<4, T, T, EDGERAG_GEMM_THREADS_64, EDGERAG_GEMM_STAGES_64>(
          x, xs, m, k, packed, scales, bias, n, g, y, ys, s);
  } else if (bits == 8) {
    launch_gemm_split<8>(x, xs, m, k, packed, scales, bias, n, g, y, ys, p, ws, s);
  } else {
    launch_gemm_split<4>(x, xs, m, k, packed, scales, bias, n, g, y, ys, p, ws, s);
  }
  return true;
}

bool qlinear_mfma_supported(int32_t k, int32_t bits, int32_t g, const void* x, int64_t x_stride,
                            const void* packed) {
  const int kb = bits == 8 ? 64 : 128;
  return (bits == 8 || bits == 4) && k % kb == 0 && g % 32 == 0 && aligned16(x) &&
         aligned16(packed) && (x_stride * 2) % 16 == 0;
}

// The fused RoPE launch takes the waves and batch of the plain launch of the same (M, K, N), which
// must itself be a one-k-slice streaming launch: then every q / k / v value it rotates or copies
// has the plain launch's bits.
// With two k-slices the RoPE launch takes 8-row tiles whose rows pair every element with its
// rotate_half twin, the plain launch's waves and k-slices; with one, two 16-row tiles per
// workgroup (a run of a head's first half and its twin), the plain launch's waves.
bool stream_rope_shape(int32_t m, int32_t k, int32_t n, int32_t heads, int32_t head_dim) {
  const int slices = m > EDGERAG_STREAM_MAX_M ? 0 : stream_slices(m, k, n);
  if (slices == 0 || head_dim % 32 != 0 || int64_t(heads) * head_dim != n) return false;
  if (slices == 2) return m <= 32;
  const int64_t tiles16 = (int64_t(n) + 15) / 16;
  const int nt = tiles16 >= EDGERAG_STREAM_NT2_TILES ? 2 : 1;
  const int mt = m <= 16 ? 1 : m <= 32 ? 2 : 4;
  return stream_waves(1, nt, mt, k).kw <= 8;
}

// The tiled GEMM with the RoPE epilogue (per-channel INT8, M > 64, head_dim 64) where the plain
// launch of the [q; k; v] weight uses 128-row weight tiles; a remainder the plain launch hands
// to the streaming path goes to the streaming RoPE kernel.
bool gemm_rope_shape(int32_t m, int32_t k, int32_t n, int32_t heads, int32_t head_dim) {
  if (head_dim != 64 || int64_t(heads) * head_dim != n || m <= EDGERAG_SKINNY_MAX_M ||
      k % kBK != 0)
    return false;
  const int rem = m % 64;
  if (rem > 0 && rem <= 16 && m - rem >= 128 && !gemm_tiles_128x64(m, n))
    return gemm_rope_shape(m - rem, k, n, heads, head_dim) &&
           stream_rope_shape(rem, k, n, heads, head_dim);
  return int64_t((n + 127) / 128) * ((m + 127) / 128) >= EDGERAG_GEMM_TARGET_WGS ||
         gemm_tiles_128x64(m, n);
}

template <int MT, bool NORM = false>
void launch_rope(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                 const f16* scales, const f16* bias, int32_t n, const EpiArgs& ea,
                 hipStream_t s) {
  const int nt = (int64_t(n) + 15) / 16 >= EDGERAG_STREAM_NT2_TILES ? 2 : 1;
  if (ea.head_dim == 64)
    launch_stream_w<1, 2, MT, kEpiRope, NORM, 32>(stream_waves(1, nt, MT, k), x, xs, m, k, packed,
                                                  scales, bias, n, nullptr, 0, ea, s);
  else
    launch_stream_w<1, 2, MT, kEpiRope, NORM>(stream_waves(1, nt, MT, k), x, xs, m, k, packed,
                                              scales, bias, n, nullptr, 0, ea, s);
}

// Two k-slices: 8-row tiles with 8-token m-tiles, the plain launch's shape for M <= 32.
template <bool NORM = false>
void launch_rope8(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                  const f16* scales, const f16* bias, int32_t n, const EpiArgs& ea,
                  hipStream_t s) {
#define EDGERAG_ROPE8(MT)                                                                        \
  do {                                                                                           \
    if (ea.head_dim == 64)                                                                       \
      launch_stream_w<2, 1, MT, kEpiRope, NORM, 32>(stream_waves(2, 1, MT, k), x, xs, m, k,      \
                                                    packed, scales, bias, n, nullptr, 0, ea, s); \
    else                                                                                         \
      launch_stream_w<2, 1, MT, kEpiRope, NORM>(stream_waves(2, 1, MT, k), x, xs, m, k, packed,  \
                                                scales, bias, n, nullptr, 0, ea, s);             \
  } while (0)
  if (m <= 8) {
    EDGERAG_ROPE8(1);
  } else if constexpr (NORM) {
    EDGERAG_ROPE8(2);  // normed inputs come with at most 16 tokens (set_norm refuses more)
  } else {
    if (m <= 16) EDGERAG_ROPE8(2);
    else EDGERAG_ROPE8(4);
  }
#undef EDGERAG_ROPE8
}

bool qlinear_rope_supported(int32_t m, int32_t k, int32_t n, int32_t bits, int32_t g,
                            int32_t heads, int32_t head_dim, const void* x, int64_t x_stride,
                            const void* packed) {
  return bits == 8 && g == k && qlinear_mfma_supported(k, bits, g, x, x_stride, packed) &&
         (stream_rope_shape(m, k, n, heads, head_dim) ||
          gemm_rope_shape(m, k, n, heads, head_dim));
}

void launch_qlinear_rope(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                         const f16* scales, const f16* bias, int32_t n, const EpiArgs& ea,
                         hipStream_t s) {
  if (!stream_rope_shape(m, k, n, ea.n_q_heads + 2 * ea.n_kv_heads, ea.head_dim)) {
    const int rem = m % 64;
    if (rem > 0 && rem <= 16 && m - rem >= 128 && !gemm_tiles_128x64(m, n)) {
      launch_qlinear_rope(x, xs, m - rem, k, packed, scales, bias, n, ea, s);
      const int t0 = m - rem;
      EpiArgs er = ea;
      er.cos_tok += int64_t(t0) * ea.head_dim;
      er.sin_tok += int64_t(t0) * ea.head_dim;
      er.slots += t0;
      er.q_out += int64_t(t0) * ea.q_st;
      launch_qlinear_rope(x + int64_t(t0) * xs, xs, rem, k, packed, scales, bias, n, er, s);
    } else if (int64_t((n + 127) / 128) * ((m + 127) / 128) >= EDGERAG_GEMM_TARGET_WGS) {
      launch_gemm_rope<128, EDGERAG_GEMM_THREADS_128, EDGERAG_GEMM_STAGES_128>(
          x, xs, m, k, packed, scales, bias, n, ea, s);
    } else {
      launch_gemm_rope<64, EDGERAG_GEMM_THREADS_128x64, EDGERAG_GEMM_STAGES_128x64>(
          x, xs, m, k, packed, scales, bias, n, ea, s);
    }
    return;
  }
  if (stream_slices(m, k, n) == 2) {
    if (ea.norm_part != nullptr)
      launch_rope8<true>(x, xs, m, k, packed, scales, bias, n, ea, s);
    else
      launch_rope8(x, xs, m, k, packed, scales, bias, n, ea, s);
  } else if (ea.norm_part != nullptr)  // normed input: decode batches of up to 16 tokens
    launch_rope<1, true>(x, xs, m, k, packed, scales, bias, n, ea, s);
  else if (m <= 16)
    launch_rope<1>(x, xs, m, k, packed, scales, bias, n, ea, s);
  else if (m <= 32)
    launch_rope<2>(x, xs, m, k, packed, scales, bias, n, ea, s);
  else
    launch_rope<4>(x, xs, m, k, packed, scales, bias, n, ea, s);
}

bool qlinear_swiglu_supported(int32_t m, int32_t k, int32_t n, int32_t bits, int32_t g,
                              const void* x, int64_t x_stride, const void* packed) {
  return bits == 8 && g == k && qlinear_mfma_supported(k, bits, g, x, x_stride, packed) &&
         (stream_swiglu_shape(m, k, n) || gemm_swiglu_shape(m, k, n));
}

void launch_qlinear_swiglu(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                           const f16* scales, const f16* bias, int32_t n, f16* y, int64_t ys,
                           const EpiArgs& ea, hipStream_t s) {
  if (stream_swiglu_shape(m, k, n))
    dispatch_stream_swiglu(x, xs, m, k, packed, scales, bias, n, y, ys, ea, s);
  else
    dispatch_gemm_swiglu(x, xs, m, k, packed, scales, bias, n, y, ys, s);
}

int qlinear_residual_parts(int32_t m, int32_t k, int32_t n, int32_t bits, int32_t g,
                           const void* x, int64_t x_stride, const void* packed) {
  if (bits != 8 || g != k || !qlinear_mfma_supported(k, bits, g, x, x_stride, packed)) return 0;
  return residual_parts(m, k, n);
}

void launch_qlinear_residual(const f16* x, int64_t xs, int32_t m, int32_t k,
                             const uint8_t* packed, const f16* scales, const f16* bias, int32_t n,
                             const EpiArgs& ea, hipStream_t s) {
  dispatch_stream_residual(x, xs, m, k, packed, scales, bias, n, ea, s);
}

void launch_qlinear_mfma(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                         const f16* scales, const f16* bias, int32_t n, int32_t bits, int32_t g,
                         f16* y, int64_t ys, hipStream_t s) {
  if (bits == 8)
    dispatch<8>(x, xs, m, k, packed, scales, bias, n, g, y, ys, s);
  else
    dispatch<4>(x, xs, m, k, packed, scales, bias, n, g, y, ys, s);
}

}  // namespace edgerag
