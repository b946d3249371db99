// Ragged paged attention over the head-major pool, for a packed batch that mixes single-token
// decodes with chunked-prefill slices.
//
// Semantics (per request r, c = q_len, L = context after append): query i sits at logical
// position L - c + i and attends keys [0, L - c + i]. This is build_causal_mask(c, L - c) +
// sdpa_attention (edgerag/core/layers.py:137-167, :227-254) over PagedKVCache.gather
// (edgerag/cache/paged.py:208-238), and for c == 1 the blockwise online softmax of
// paged_attention_reference (edgerag/cache/fused.py:89-167).
//
// Execution model:
//   1. edgerag_attn_plan (host) cuts every (request, kv head) into KV splits and writes a flat
//      work list: "row" items (decodes: c * n_rep <= kMaxRowVecs query vectors) first, then
//      "tile" items (prefill slices in query tiles), each group heaviest first. Long contexts are
//      split so that a 32-way decode batch still yields thousands of independent waves.
//   2. attn_decode_kernel: one wavefront per row item. Lanes are grouped LPT per token (16 bytes
//      each, so a group covers one head_dim row); each load instruction covers TPW consecutive
//      tokens = a fully coalesced 1 KiB slice of a 2 KiB block row, and U such slices are in
//      flight per lane. Every lane group keeps its own fp32 online-softmax state (m, l, acc), so
//      the K/V loop needs no cross-group communication; groups merge once at the end. Block ids
//      of the split are held one per lane and broadcast with v_readlane. Q.K uses v_dot2_f32_f16.
//   3. attn_rows_kernel: the general version of (2) for shapes the fast path does not cover
//      (block_size not a multiple of the tokens-per-load, or prefill tiles before the MFMA path).
//   4. attn_combine_kernel merges the fp32 split partials (m, l, acc) of split requests, one
//      thread per (token, query head, 4 output elements); unsplit requests are written directly
//      by (2)/(3).
// Scores are kept in the log2 domain (scaled by scale * log2(e)) so each exponential is one
// v_exp_f32.
#include <algorithm>
#include <cmath>
#include <mutex>
#include <vector>

#include "attention_merge.h"
#include "attention_plan.h"

namespace edgerag {
namespace {

using namespace plan;
constexpr int32_t kPlanMagic = plan::kMagic;
constexpr int32_t kPlanVersion = plan::kVersion;

// Tuning constants; the EDGERAG_* macros let a build override them for sweeps.
#ifndef EDGERAG_MIN_SPLIT
#define EDGERAG_MIN_SPLIT 256
#endif
#ifndef EDGERAG_TARGET_ITEMS
#define EDGERAG_TARGET_ITEMS 4096
#endif
#ifndef EDGERAG_WG_QR_MAX
#define EDGERAG_WG_QR_MAX 4  // query vectors per pass of a workgroup row (fp16 / fp32)
#endif
#ifndef EDGERAG_WG_QR_MAX_BF16
#define EDGERAG_WG_QR_MAX_BF16 4  // ... bf16
#endif
#ifndef EDGERAG_COMBINE_THREADS
// Threads of a merge workgroup. The merges of small batches are a few hundred threads (batch 1:
// 32 heads x 16 channels): one-wave workgroups spread them over as many CUs, where 256-thread
// workgroups would put all of them on two. The kernels take it as a constant (not blockDim), so
// no thread index waits for a load of the workgroup size from the hidden kernel arguments.
#define EDGERAG_COMBINE_THREADS 64
#endif
#ifndef EDGERAG_DECODE_U
#define EDGERAG_DECODE_U 2
#endif
#ifndef EDGERAG_DECODE_NT
#define EDGERAG_DECODE_NT 1  // decode rows read the pools with non-temporal loads
#endif
#ifndef EDGERAG_ROW_WG
#define EDGERAG_ROW_WG 1  // decode rows as one workgroup per (request, kv head), merged in LDS
#endif
#ifndef EDGERAG_ROW_WG_PART
#define EDGERAG_ROW_WG_PART 256  // longest part (tokens) a wave of a workgroup-split row takes
#endif
#ifndef EDGERAG_ROW_WG_PART_TILES
#define EDGERAG_ROW_WG_PART_TILES 512  // the same, in a batch with prefill tiles beside the rows
#endif
#ifndef EDGERAG_ROW_WG_MAX_ITEMS
// A decode batch takes (request, kv head) workgroup rows when they make one round over the CUs,
// or up to EDGERAG_ROW_WG_MAX_ITEMS of them when no context passes EDGERAG_ROW_WG_SHORT tokens;
// otherwise KV splits. A 16-wave row workgroup holds a CU alone, so past one round the splits'
// one-wave workgroups, more of them in flight per CU, win despite their merge launch, except on
// short contexts, on one stream (32/32 heads, fp16, contexts of 1,000 / 2,000 /
// 4,000 tokens, rows against splits: 8 requests 15.7 / 26.3 / 46.2 against 29.8 / 38.8 / 48.3
// us; 12: 27.8 / 43.7 / 77.2 against 34.7 / 39.3 / 65.3; 16: 27.9 / 48.3 / 86.0 against
// 34.6 / 46.4 / 85.5; 24: 41.4 / 71.1 / 127.2 against 38.7 / 65.8 / 124.0; 64: 107.6 / 182.4 /
// 334.9 against 83.0 / 158.8 / 315.5) and beside prefill tiles on a second stream (config 3:
// 768 row workgroups, step 181-189 against 176-177 us with KV splits).
#define EDGERAG_ROW_WG_MAX_ITEMS 512
#endif
#ifndef EDGERAG_ROW_WG_SHORT
#define EDGERAG_ROW_WG_SHORT 1536
#endif
#ifndef EDGERAG_ROW_WG_WAVES
#define EDGERAG_ROW_WG_WAVES 16  // waves of a workgroup over a whole context
#endif
#ifndef EDGERAG_ROW_PART_WAVES
#define EDGERAG_ROW_PART_WAVES 8  // waves of a workgroup over a part of a context
#endif
#ifndef EDGERAG_ROW_TARGET_WGS
#define EDGERAG_ROW_TARGET_WGS 512  // row workgroups a batch of few decodes is cut into
#endif
#ifndef EDGERAG_ROW_MIN_WAVE_TOKENS
#define EDGERAG_ROW_MIN_WAVE_TOKENS 32  // shortest stream a wave of a context part takes
#endif
// ... when no context is longer than EDGERAG_ROW_SHORT_CTX: short contexts are cut into twice as
// many parts. Single sequence (32 heads) at 512 / 1,024 / 2,048 tokens: 9.48 / 9.71 / 10.21 ->
// 8.0 / 8.3 / 9.85 us; batch-1 decode iteration at 600 / 1,500 tokens: 0.894-0.911 /
// 0.913-0.924 -> 0.873 / 0.889-0.897 ms. Applied up to 4,096 tokens it gained nothing at 3,000.
#ifndef EDGERAG_ROW_MIN_WAVE_TOKENS_SHORT
#define EDGERAG_ROW_MIN_WAVE_TOKENS_SHORT 16
#endif
#ifndef EDGERAG_ROW_SHORT_CTX
#define EDGERAG_ROW_SHORT_CTX 2048
#endif
#ifndef EDGERAG_ROW_WG_LONG
#define EDGERAG_ROW_WG_LONG 0  // 1: contexts past the per-wave cap in part workgroups too
#endif
constexpr int kRowWgWaves = EDGERAG_ROW_WG_WAVES;
constexpr int kRowPartWaves = EDGERAG_ROW_PART_WAVES;
constexpr int kRowTargetWgs = EDGERAG_ROW_TARGET_WGS;
constexpr int kRowMinWaveTokens = EDGERAG_ROW_MIN_WAVE_TOKENS;
constexpr int kMaxRowVecs = 8;  // query vectors a decode item may carry (c * n_rep)
constexpr int kQTile = 16;      // query rows per prefill tile item
constexpr int kMinSplit = EDGERAG_MIN_SPLIT;  // tokens; shorter splits are not worth a partial
constexpr int kTargetItems = EDGERAG_TARGET_ITEMS;  // decode work items a batch is cut into
constexpr int kDecodeU = EDGERAG_DECODE_U;  // token loads in flight per lane group
constexpr int kMaxSplitBlocks = 64;  // one block id per lane in the decode kernel
#ifndef EDGERAG_TARGET_TILES
#define EDGERAG_TARGET_TILES 512
#endif
#ifndef EDGERAG_TILE_BALANCE
#define EDGERAG_TILE_BALANCE 1  // split the longest tile items however many tile items there are
#endif
#ifndef EDGERAG_MIN_TILE_SPLIT
#define EDGERAG_MIN_TILE_SPLIT 1024
#endif
constexpr int kMinTileSplit = EDGERAG_MIN_TILE_SPLIT;  // keys: tiles split no finer than this
constexpr int kTargetTiles = EDGERAG_TARGET_TILES;  // prefill tile items a batch aims for
constexpr int kPlanCUs = 256;  // compute units the planner fills (MI355X)
// K/V bytes decode rows must read for the planner to put them beside prefill tiles.
constexpr int64_t kOverlapRowBytes = int64_t(256) << 20;

// Cross-lane moves inside a 16-lane row via DPP (plain VALU instructions, no LDS crossbar).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Reduce over the LPT consecutive lanes of a token group. xor 1 / xor 2 are quad permutes; after
// them every lane of a quad holds the quad's value, so a half-row mirror (lane i <-> 7 - i)
// completes 8 lanes and a row mirror (i <-> 15 - i) completes 16.
template <int LPT, bool MAX>
__device__ __forceinline__ float group_reduce(float v) {
  auto op = [](float a, float b) { return MAX ? fmaxf(a, b) : a + b; };
  if constexpr (LPT >= 2) v = op(v, dpp<0xB1>(v));
  if constexpr (LPT >= 4) v = op(v, dpp<0x4E>(v));
  if constexpr (LPT >= 8) v = op(v, dpp<0x141>(v));
  if constexpr (LPT >= 16) v = op(v, dpp<0x140>(v));
  if constexpr (LPT >= 32) v = op(v, __shfl_xor(v, 16, kWave));
  if constexpr (LPT >= 64) v = op(v, __shfl_xor(v, 32, kWave));
  return v;
}

template <typename T, int D>
struct RowCfg {
  static constexpr int VEC = 16 / sizeof(T);
  static constexpr int LPT = D / VEC;      // lanes sharing one token
  static constexpr int TPW = kWave / LPT;  // tokens per load instruction
  static constexpr int LOG_LPT = ilog2(LPT);
  static_assert(D % VEC == 0 && LPT >= 1 && LPT <= kWave, "unsupported head_dim");
};

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// q . k over this lane's VEC elements (q already in registers), widened to fp32.
template <typename T, int VEC>
struct QReg {
  float f[VEC];  // fp32 / bf16 path: pre-scaled by scale*log2(e)
  half2_t h[VEC / 2 > 0 ? VEC / 2 : 1];  // fp16 path: raw fp16 values

  __device__ __forceinline__ void load(const T* p, float scale_log2) {
    if constexpr (__is_same(T, f16)) {
      const Vec16 raw = load16(p);
#pragma unroll
      for (int i = 0; i < VEC / 2; ++i) h[i] = *reinterpret_cast<const half2_t*>(&raw.w[i]);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) f[e] = to_f32<T>(p[e]) * scale_log2;
    }
  }
  __device__ __forceinline__ void zero() {
#pragma unroll
    for (int e = 0; e < VEC; ++e) f[e] = 0.f;
#pragma unroll
    for (int i = 0; i < (VEC / 2 > 0 ? VEC / 2 : 1); ++i) h[i] = half2_t{0, 0};
  }
  // Partial dot product; the fp16 path is scaled after the group reduction.
  __device__ __forceinline__ float dot(const Vec16& k) const {
    float s = 0.f;
    if constexpr (__is_same(T, f16)) {
#pragma unroll
      for (int i = 0; i < VEC / 2; ++i)
        s = __builtin_amdgcn_fdot2(h[i], *reinterpret_cast<const half2_t*>(&k.w[i]), s, false);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) s = fmaf(f[e], vec_elem<T>(k, e), s);
    }
    return s;
  }
  static constexpr bool kScaleAfter = __is_same(T, f16);
};

// ---- fast decode kernel --------------------------------------------------------------------------
// Requires block_size % TPW == 0 and at most kMaxSplitBlocks blocks per split (checked by the
// launcher from the plan header).
// APPEND: the step's own tokens (positions L - c .. L - 1 of each request) are read from the new
// K/V rows instead of the pools, and the split that reads them also writes them to the pools at
// their slots (kv_append fused in: no other wave reads those pool rows in this launch).
// WG: one workgroup per row item (blockDim / 64 waves); wave w takes the w-th of equal,
// block-aligned parts of the item's keys, and the waves' (m, l, acc) merge in LDS before wave 0
// writes the output, or, when the item is one of several parts of a context, the part's fp32
// partial for the merge launch. Otherwise one wave per item (a KV split).
// The arguments of the first loads (plan, request arrays, block table) lead the list: the library
// is built to preload the leading kernel arguments into SGPRs at wave launch, so the work item's
// load does not wait for a kernel-argument fetch from memory.
template <typename T, int D, int QR, int U, bool APPEND, bool WG>
__global__ __launch_bounds__(WG ? kMaxRowWaves * kWave : kWave) void attn_decode_kernel(
    const int32_t* __restrict__ plan, int32_t item_base, int32_t limit_word,
    const int32_t* __restrict__ qsl, const int32_t* __restrict__ ctx,
    const int32_t* __restrict__ block_tables, int64_t bt_stride, int32_t num_blocks,
    int32_t block_size, const T* __restrict__ q, int64_t q_st, int64_t q_sh,
    const T* __restrict__ kpool, const T* __restrict__ vpool, int32_t n_q_heads,
    int32_t n_kv_heads, float scale_log2, T* __restrict__ out, int64_t o_st, int64_t o_sh, float2* __restrict__ part_ml,
    float* __restrict__ part_acc, const T* __restrict__ nk, const T* __restrict__ nv,
    int64_t n_st, int64_t n_sh, const int32_t* __restrict__ slots, T* __restrict__ kdst,
    T* __restrict__ vdst) {
  using C = RowCfg<T, D>;
  constexpr int VEC = C::VEC, LPT = C::LPT, TPW = C::TPW, LOG_LPT = C::LOG_LPT;
  constexpr int STEP = TPW * U;

  // The grid may exceed the work list (fixed-size launches replayed from a graph): the item
  // count of this launch's kind is read from the device plan. The item is read in the same
  // round trip (items follow the header, and a fixed-capacity plan buffer holds every slot the
  // grid covers), not after it.
  const int64_t idx = int64_t(item_base) + blockIdx.x;
  const int32_t* it = plan + kHeaderWords + idx * kItemWords;
  const int4 ia = reinterpret_cast<const int4*>(it)[0], ib = reinterpret_cast<const int4*>(it)[1];
  int r = ia.x, h = ia.y, qb = ia.z, qc = ia.w;  // I_REQ, I_HEAD, I_QBEGIN, I_QCOUNT
  int kb = ib.x, ke = ib.y;                       // I_KVBEGIN, I_KVEND
  int split = ib.z;                               // I_SPLIT
  int limit = plan[limit_word], req_off = plan[H_REQ_OFF];
  const int nw = WG ? int(blockDim.x >> 6) : 1;
  // The prologue's dependent loads take three round trips: (1) the item, the count, the request
  // table's offset and the kernel arguments that are not preloaded; (2) the request's entries
  // and the split's block ids; (3) q and the first K/V rows. Used here, the first group is loaded
  // together, not each after the exit test or where first needed (the compiler would sink them).
  // (The item's unused last word is used too: left dead, its register is handed to another load
  // of the group, which then has to wait for the item's load to land.)
  asm volatile("" : "+s"(limit), "+s"(req_off), "+s"(r), "+s"(h), "+s"(qb), "+s"(qc), "+s"(kb),
               "+s"(ke), "+s"(split)
               : "s"(ib.w), "s"(nw), "s"(n_q_heads), "s"(n_kv_heads), "s"(q), "s"(q_st),
                 "s"(q_sh), "s"(kpool), "s"(vpool), "s"(scale_log2), "s"(out), "s"(o_st),
                 "s"(o_sh), "s"(part_ml), "s"(part_acc));
  if constexpr (APPEND)
    asm volatile("" ::"s"(nk), "s"(nv), "s"(n_st), "s"(n_sh), "s"(slots), "s"(kdst), "s"(vdst));
  if (idx >= limit) return;
  const int wave = WG ? __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6)) : 0;
  if constexpr (WG) {
    // This wave's part of the keys: equal parts of whole blocks (a part never straddles the
    // wave's block-id registers), empty for waves past the end.
    const int per = (ke - kb + nw - 1) / nw;
    const int part = (per + block_size - 1) / block_size * block_size;
    const int b0 = min(ke, kb + wave * part);
    ke = min(ke, b0 + part);
    kb = b0;
  }
  const int lane = threadIdx.x & (kWave - 1);
  // Block ids of this split, one per lane; broadcast per load with v_readlane. The load is
  // unconditional (lanes past the split re-read its last entry, always inside the table row) and
  // the ids are checked only after the request's entries are loaded as well: one round trip.
  const int blk0 = kb / block_size;
  const int nblk = (ke - kb + block_size - 1) / block_size;
  int32_t b_raw = -1;
  if (nblk > 0)  // wave-uniform
    b_raw = block_tables[int64_t(r) * bt_stride + blk0 + min(lane, nblk - 1)];
  const int32_t* rq = plan + req_off + r * kReqWords;
  int nsplit = rq[R_NSPLIT], part_off = rq[R_PARTOFF], pstride = rq[R_PSTRIDE];
  int q0 = qsl[r], q1 = qsl[r + 1], L = ctx[r];
  asm volatile("" : "+s"(nsplit), "+s"(part_off), "+s"(pstride), "+s"(q0), "+s"(q1), "+s"(L));
  const int c = q1 - q0;
  issue_fence();
  const int my_blk = (lane < nblk && b_raw >= 0 && b_raw < num_blocks) ? b_raw : -1;
  const int n_rep = n_q_heads / n_kv_heads;

  const int sub = lane & (LPT - 1);
  const int tslot = lane >> LOG_LPT;
  const int64_t head_base = int64_t(h) * num_blocks;

  const int nvec = qc * n_rep;
  for (int v0 = 0; v0 < nvec; v0 += QR) {
    QReg<T, VEC> qr[QR];
    float m[QR], l[QR], acc[QR][VEC];
    int lim[QR];
#pragma unroll
    for (int j = 0; j < QR; ++j) {
      const int v = v0 + j;
      const int t = qb + v / n_rep;
      const int hq = h * n_rep + (v % n_rep);
      lim[j] = v < nvec ? L - c + (t - q0) : -1;  // -1: inactive slot, sees nothing
      if (v < nvec)
        qr[j].load(q + int64_t(t) * q_st + int64_t(hq) * q_sh + sub * VEC, scale_log2);
      else
        qr[j].zero();
      m[j] = -INFINITY;
      l[j] = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[j][e] = 0.f;
    }

    for (int g0 = kb; g0 < ke; g0 += STEP) {
      Vec16 kr[U], vr[U];
      int tok[U];
      bool valid[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int first = g0 + u * TPW;  // wave-uniform
        tok[u] = first + tslot;
        const bool live = first < ke;
        const int blk = __builtin_amdgcn_readlane(my_blk, live ? (first - kb) / block_size : 0);
        valid[u] = live && tok[u] < ke && blk >= 0;
        const int i_new = tok[u] - (L - c);  // >= 0: one of this step's tokens
        if (APPEND && valid[u] && i_new >= 0) {
          const int64_t noff = int64_t(q0 + i_new) * n_st + int64_t(h) * n_sh + sub * VEC;
          kr[u] = load16(nk + noff);
          vr[u] = load16(nv + noff);
          const int64_t slot = slots[q0 + i_new];
          if (slot >= 0 && slot < int64_t(num_blocks) * block_size) {
            const int64_t doff =
                ((head_base + slot / block_size) * block_size + slot % block_size) * D + sub * VEC;
            store16(kdst + doff, kr[u]);
            store16(vdst + doff, vr[u]);
          }
        } else if (valid[u]) {
          const int64_t off =
              ((head_base + blk) * block_size + (tok[u] % block_size)) * D + sub * VEC;
          // A launch reads each pool byte of a decode row once: non-temporal loads stream it
          // without evicting reused lines (prefill tiles' K/V beside the rows). Measured on a
          // 32-request decode step: 5.69 -> 6.40 TB/s; on the mixed step: 0.212 -> 0.199 ms.
          if constexpr (EDGERAG_DECODE_NT) {
            kr[u] = load16_stream(kpool + off);
            vr[u] = load16_stream(vpool + off);
          } else {
            kr[u] = load16(kpool + off);
            vr[u] = load16(vpool + off);
          }
        } else {
          kr[u] = Vec16{};
          vr[u] = Vec16{};
        }
      }
#pragma unroll
      for (int j = 0; j < QR; ++j) {
        float s[U];
        float mloc = -INFINITY;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          float d = group_reduce<LPT, false>(qr[j].dot(kr[u]));
          if constexpr (QReg<T, VEC>::kScaleAfter) d *= scale_log2;
          s[u] = (valid[u] && tok[u] <= lim[j]) ? d : -INFINITY;
          mloc = fmaxf(mloc, s[u]);
        }
        const float mnew = fmaxf(m[j], mloc);
        if (__any(mnew > m[j])) {
          const float alpha = mnew == -INFINITY ? 1.f : exp2_fast(m[j] - mnew);
          l[j] *= alpha;
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[j][e] *= alpha;
          m[j] = mnew;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float p = s[u] == -INFINITY ? 0.f : exp2_fast(s[u] - m[j]);
          l[j] += p;
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[j][e] = fmaf(p, vec_elem<T>(vr[u], e), acc[j][e]);
        }
      }
    }

    // Merge the TPW lane groups of each query vector, then write.
    if constexpr (WG) {
      // The waves' partials (log2-domain max, sum, acc) meet in LDS; wave 0 merges and writes.
      __shared__ float wg_ml[kMaxRowWaves][QR][2];
      __shared__ float wg_acc[kMaxRowWaves][QR][D];
#pragma unroll
      for (int j = 0; j < QR; ++j) {
        float mm = m[j];
#pragma unroll
        for (int b = LOG_LPT; b < 6; ++b) mm = fmaxf(mm, __shfl_xor(mm, 1 << b, kWave));
        const float w = m[j] == -INFINITY ? 0.f : exp2_fast(m[j] - mm);
        float lsum = w * l[j];
#pragma unroll
        for (int b = LOG_LPT; b < 6; ++b) lsum += __shfl_xor(lsum, 1 << b, kWave);
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          float a = w * acc[j][e];
#pragma unroll
          for (int b = LOG_LPT; b < 6; ++b) a += __shfl_xor(a, 1 << b, kWave);
          if (tslot == 0) wg_acc[wave][j][sub * VEC + e] = a;
        }
        if (lane == 0) {
          wg_ml[wave][j][0] = mm;
          wg_ml[wave][j][1] = lsum;
        }
      }
      __syncthreads();
      if (wave == 0) {
        const int nw = int(blockDim.x >> 6);
#pragma unroll
        for (int j = 0; j < QR; ++j) {
          const int v = v0 + j;
          if (v >= nvec) break;
          float mx = -INFINITY;
          for (int wv = 0; wv < nw; ++wv) mx = fmaxf(mx, wg_ml[wv][j][0]);
          float lsum = 0.f;
          float a[(D + kWave - 1) / kWave];
#pragma unroll
          for (int e = 0; e < (D + kWave - 1) / kWave; ++e) a[e] = 0.f;
          for (int wv = 0; wv < nw; ++wv) {
            const float mw = wg_ml[wv][j][0];
            const float wgt = mw == -INFINITY ? 0.f : exp2_fast(mw - mx);
            lsum = fmaf(wgt, wg_ml[wv][j][1], lsum);
#pragma unroll
            for (int e = 0; e < (D + kWave - 1) / kWave; ++e) {
              const int d = lane + e * kWave;
              if (d < D) a[e] = fmaf(wgt, wg_acc[wv][j][d], a[e]);
            }
          }
          const int t = qb + v / n_rep;
          const int hq = h * n_rep + (v % n_rep);
          if (pstride == 1) {
            const float inv = 1.f / fmaxf(lsum, 1.17549435e-38f);
            T* op = out + int64_t(t) * o_st + int64_t(hq) * o_sh;
#pragma unroll
            for (int e = 0; e < (D + kWave - 1) / kWave; ++e) {
              const int d = lane + e * kWave;
              if (d < D) op[d] = from_f32<T>(a[e] * inv);
            }
          } else {  // one of several parts of the context (or a slot): a partial for the merge
            const int64_t row0 = int64_t(part_off) + (int64_t(t - q0) * n_q_heads + hq) * pstride;
            const int64_t idx = row0 + split;
            if (lane == 0) part_ml[idx] = make_float2(mx, lsum);
            // Slotted plans: the last part also marks the row's unused slots empty, so that a
            // merge reading all of them gives them weight 0.
            if (split == nsplit - 1 && nsplit + lane < pstride)
              part_ml[row0 + nsplit + lane] = make_float2(-INFINITY, 0.f);
            float* pa = part_acc + idx * D;
#pragma unroll
            for (int e = 0; e < (D + kWave - 1) / kWave; ++e) {
              const int d = lane + e * kWave;
              if (d < D) pa[d] = a[e];
            }
          }
        }
      }
      __syncthreads();  // the LDS is rewritten by the next pass over query vectors
      continue;
    }
#pragma unroll
    for (int j = 0; j < QR; ++j) {
      const int v = v0 + j;
      if (v >= nvec) break;
      float mm = m[j];
#pragma unroll
      for (int b = LOG_LPT; b < 6; ++b) mm = fmaxf(mm, __shfl_xor(mm, 1 << b, kWave));
      const float w = m[j] == -INFINITY ? 0.f : exp2_fast(m[j] - mm);
      float lsum = w * l[j];
#pragma unroll
      for (int b = LOG_LPT; b < 6; ++b) lsum += __shfl_xor(lsum, 1 << b, kWave);
      float a[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        a[e] = w * acc[j][e];
#pragma unroll
        for (int b = LOG_LPT; b < 6; ++b) a[e] += __shfl_xor(a[e], 1 << b, kWave);
      }
      if (tslot != 0) continue;
      const int t = qb + v / n_rep;
      const int hq = h * n_rep + (v % n_rep);
      if (nsplit == 1) {
        const float inv = 1.f / fmaxf(lsum, 1.17549435e-38f);
        T* op = out + int64_t(t) * o_st + int64_t(hq) * o_sh + sub * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) op[e] = from_f32<T>(a[e] * inv);
      } else {
        const int64_t idx =
            int64_t(part_off) + (int64_t(t - q0) * n_q_heads + hq) * pstride + split;
        if (sub == 0) part_ml[idx] = make_float2(mm, lsum);
        float* pa = part_acc + idx * D + sub * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) pa[e] = a[e];
      }
    }
  }
}

// ---- general row kernel ----------------------------------------------------------------------------
// Any block size and split length; per-lane block lookups; QR query vectors per pass.
template <typename T, int D, int QR>
__global__ __launch_bounds__(kWave) void attn_rows_kernel(
    const int32_t* __restrict__ plan, int32_t item_base, int32_t limit_word,
    const int32_t* __restrict__ qsl, const int32_t* __restrict__ ctx,
    const int32_t* __restrict__ block_tables, int64_t bt_stride, int32_t num_blocks,
    int32_t block_size, const T* __restrict__ q, int64_t q_st, int64_t q_sh,
    const T* __restrict__ kpool, const T* __restrict__ vpool, int32_t n_q_heads,
    int32_t n_kv_heads, float scale_log2, T* __restrict__ out, int64_t o_st, int64_t o_sh, float2* __restrict__ part_ml,
    float* __restrict__ part_acc) {
  using C = RowCfg<T, D>;
  constexpr int VEC = C::VEC, LPT = C::LPT, TPW = C::TPW, LOG_LPT = C::LOG_LPT;

  // The grid may exceed the work list (fixed-size launches replayed from a graph): the item
  // count of this launch's kind is read from the device plan.
  if (item_base + int(blockIdx.x) >= plan[limit_word]) return;
  const int32_t* it = plan + plan[H_ITEM_OFF] + int64_t(item_base + blockIdx.x) * kItemWords;
  const int r = it[I_REQ], h = it[I_HEAD], qb = it[I_QBEGIN], qc = it[I_QCOUNT];
  const int kb = it[I_KVBEGIN], ke = it[I_KVEND], split = it[I_SPLIT];
  const int32_t* rq = plan + plan[H_REQ_OFF] + r * kReqWords;
  const int nsplit = rq[R_NSPLIT], part_off = rq[R_PARTOFF], pstride = rq[R_PSTRIDE];
  const int q0 = qsl[r], c = qsl[r + 1] - q0, L = ctx[r];
  const int n_rep = n_q_heads / n_kv_heads;

  const int lane = threadIdx.x;
  const int sub = lane & (LPT - 1);
  const int tslot = lane >> LOG_LPT;
  const int32_t* table = block_tables + int64_t(r) * bt_stride;
  const int64_t head_base = int64_t(h) * num_blocks;

  const int nvec = qc * n_rep;
  for (int v0 = 0; v0 < nvec; v0 += QR) {
    QReg<T, VEC> qr[QR];
    float m[QR], l[QR], acc[QR][VEC];
    int lim[QR];
#pragma unroll
    for (int j = 0; j < QR; ++j) {
      const int v = v0 + j;
      const int t = qb + v / n_rep;
      const int hq = h * n_rep + (v % n_rep);
      lim[j] = v < nvec ? L - c + (t - q0) : -1;
      if (v < nvec)
        qr[j].load(q + int64_t(t) * q_st + int64_t(hq) * q_sh + sub * VEC, scale_log2);
      else
        qr[j].zero();
      m[j] = -INFINITY;
      l[j] = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[j][e] = 0.f;
    }

    for (int g0 = kb; g0 < ke; g0 += TPW) {
      const int tok = g0 + tslot;
      bool valid = tok < ke;
      Vec16 kr{}, vr{};
      if (valid) {
        const int32_t blk = table[tok / block_size];
        valid = blk >= 0 && blk < num_blocks;
        if (valid) {
          const int64_t off = ((head_base + blk) * block_size + (tok % block_size)) * D + sub * VEC;
          kr = load16(kpool + off);
          vr = load16(vpool + off);
        }
      }
#pragma unroll
      for (int j = 0; j < QR; ++j) {
        float s = group_reduce<LPT, false>(qr[j].dot(kr));
        if constexpr (QReg<T, VEC>::kScaleAfter) s *= scale_log2;
        const bool vis = valid && tok <= lim[j];
        s = vis ? s : -INFINITY;
        const float mnew = fmaxf(m[j], s);
        if (__any(mnew > m[j])) {
          const float alpha = mnew == -INFINITY ? 1.f : exp2_fast(m[j] - mnew);
          l[j] *= alpha;
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[j][e] *= alpha;
          m[j] = mnew;
        }
        const float p = vis ? exp2_fast(s - m[j]) : 0.f;
        l[j] += p;
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[j][e] = fmaf(p, vec_elem<T>(vr, e), acc[j][e]);
      }
    }

#pragma unroll
    for (int j = 0; j < QR; ++j) {
      const int v = v0 + j;
      if (v >= nvec) break;
      float mm = m[j];
#pragma unroll
      for (int b = LOG_LPT; b < 6; ++b) mm = fmaxf(mm, __shfl_xor(mm, 1 << b, kWave));
      const float w = m[j] == -INFINITY ? 0.f : exp2_fast(m[j] - mm);
      float lsum = w * l[j];
#pragma unroll
      for (int b = LOG_LPT; b < 6; ++b) lsum += __shfl_xor(lsum, 1 << b, kWave);
      float a[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        a[e] = w * acc[j][e];
#pragma unroll
        for (int b = LOG_LPT; b < 6; ++b) a[e] += __shfl_xor(a[e], 1 << b, kWave);
      }
      if (tslot != 0) continue;
      const int t = qb + v / n_rep;
      const int hq = h * n_rep + (v % n_rep);
      if (nsplit == 1) {
        const float inv = 1.f / fmaxf(lsum, 1.17549435e-38f);
        T* op = out + int64_t(t) * o_st + int64_t(hq) * o_sh + sub * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) op[e] = from_f32<T>(a[e] * inv);
      } else {
        const int64_t idx =
            int64_t(part_off) + (int64_t(t - q0) * n_q_heads + hq) * pstride + split;
        if (sub == 0) part_ml[idx] = make_float2(mm, lsum);
        float* pa = part_acc + idx * D + sub * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) pa[e] = a[e];
      }
    }
  }
}

// ---- combine -----------------------------------------------------------------------------------
// Merges split partials (m, l, acc[D]) into the output: one thread per (row, query head, 4
// consecutive output elements), so a (row, head) pair takes D / 4 adjacent lanes and every partial
// load is one 16-byte access. A thread issues the (m, l) and acc loads of up to kCombineBatch
// splits together (the acc loads do not depend on (m, l)); more splits are merged batch by batch
// with a running maximum.
// * attn_combine_kernel reads each row's combine-list entry first: the chain of dependent loads
//   is entry -> {(m, l), acc}. n_rows < 0 / combine_off < 0: the list's length / offset are read
//   from the device plan header (fixed-capacity launches).
// * attn_combine_slots_kernel serves slotted plans with row requests only: row t's partials sit in
//   the H_SLOTS slots (t * n_q_heads + hq) * S + [0, S), the unused ones marked empty by the
//   decode kernel, so every load address follows from the thread index alone and the merge takes
//   one round trip.
// Both fold the partials with merge_partials in slot order, so a row merges to the same values.
template <typename T, bool VEC_OUT>
__device__ __forceinline__ void store_merged(T* op, float4 acc, float l) {
  const float inv = merge_inv(l);
  const T o0 = from_f32<T>(acc.x * inv), o1 = from_f32<T>(acc.y * inv),
          o2 = from_f32<T>(acc.z * inv), o3 = from_f32<T>(acc.w * inv);
  if constexpr (VEC_OUT) {
    struct alignas(4 * sizeof(T)) Quad {
      T e[4];
    };
    *reinterpret_cast<Quad*>(op) = Quad{{o0, o1, o2, o3}};
  } else {
    op[0] = o0;
    op[1] = o1;
    op[2] = o2;
    op[3] = o3;
  }
}

template <typename T, bool VEC_OUT>
__global__ __launch_bounds__(EDGERAG_COMBINE_THREADS) void attn_combine_kernel(
    const int32_t* __restrict__ plan, int32_t n_rows, int32_t combine_off, int32_t n_q_heads,
    int32_t ch_log2, const float2* __restrict__ part_ml, const float4* __restrict__ part_acc,
    T* __restrict__ out, int64_t o_st, int64_t o_sh) {
  const int gid = int(blockIdx.x) * EDGERAG_COMBINE_THREADS + int(threadIdx.x);
  const int ch = gid & ((1 << ch_log2) - 1);
  const int pair = gid >> ch_log2;
  const int row = pair / n_q_heads;
  const int hq = pair - row * n_q_heads;
  if (row >= (n_rows >= 0 ? n_rows : plan[H_N_COMBINE])) return;
  const int off = combine_off >= 0 ? combine_off : plan[H_COMBINE_OFF];
  const int4* e4 = reinterpret_cast<const int4*>(plan + off + int64_t(row) * kCombineWords);
  const int4 ea = e4[0], eb = e4[1];  // {tok, q0, c, L}, {nsplit, split_len, part_off, pstride}
  const int t = ea.x, q0 = ea.y, c = ea.z, L = ea.w;
  const int nsplit = eb.x, split_len = eb.y, part_off = eb.z, pstride = eb.w;
  // Splits that start past this row's causal limit were never computed (lim >= 0 for every row
  // the planner writes, since c <= L; the clamp keeps the arithmetic branch-free).
  const int lim = max(L - c + (t - q0), 0);
  const int n_valid = min(nsplit, lim / split_len + 1);
  const int64_t base = int64_t(part_off) + (int64_t(t - q0) * n_q_heads + hq) * pstride;
  float m = -INFINITY, l = 0.f;
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < n_valid; s0 += kCombineBatch) {
    float2 ml[kCombineBatch];
    float4 v[kCombineBatch];
    bool take[kCombineBatch];
#pragma unroll
    for (int k = 0; k < kCombineBatch; ++k) {
      const int64_t p = base + min(s0 + k, n_valid - 1);  // clamped: extra splits weigh 0
      ml[k] = part_ml[p];
      v[k] = part_acc[(p << ch_log2) + ch];
      take[k] = s0 + k < n_valid;
    }
    merge_partials(ml, v, take, m, l, acc);
  }
  store_merged<T, VEC_OUT>(out + int64_t(t) * o_st + int64_t(hq) * o_sh + ch * 4, acc, l);
}

// n_rows < 0: the token count is read from the device plan header (fixed-capacity launches), in
// the same round trip as the partials (rows past it load in-bounds slots and store nothing). A
// plan whose H_SLOTS differs from `slots` gets NaN rows: a launch shape that does not match the
// staged plan fails loudly.
template <typename T, bool VEC_OUT>
__global__ __launch_bounds__(EDGERAG_COMBINE_THREADS) void attn_combine_slots_kernel(
    const int32_t* __restrict__ plan, int32_t n_rows, int32_t slots, int32_t n_q_heads,
    int32_t ch_log2, const float2* __restrict__ part_ml, const float4* __restrict__ part_acc,
    T* __restrict__ out, int64_t o_st, int64_t o_sh) {
  const int gid = int(blockIdx.x) * EDGERAG_COMBINE_THREADS + int(threadIdx.x);
  const int ch = gid & ((1 << ch_log2) - 1);
  const int pair = gid >> ch_log2;
  const int t = pair / n_q_heads;
  const int hq = pair - t * n_q_heads;
  const int rows = n_rows >= 0 ? n_rows : plan[H_NUM_TOKENS_HINT];
  const int plan_slots = plan[H_SLOTS];
  const int64_t base = (int64_t(t) * n_q_heads + hq) * slots;
  float m = -INFINITY, l = 0.f;
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < slots; s0 += kCombineBatch) {
    float2 ml[kCombineBatch];
    float4 v[kCombineBatch];
    bool take[kCombineBatch];
#pragma unroll
    for (int k = 0; k < kCombineBatch; ++k) {
      const int64_t p = base + min(s0 + k, slots - 1);
      ml[k] = part_ml[p];
      v[k] = part_acc[(p << ch_log2) + ch];
      take[k] = s0 + k < slots;
    }
    issue_fence();  // every load of the batch is in flight before the row bound is looked at
    merge_partials(ml, v, take, m, l, acc);
  }
  if (t >= rows) return;
  if (plan_slots != slots) acc.x = acc.y = acc.z = acc.w = l = __builtin_nanf("");
  store_merged<T, VEC_OUT>(out + int64_t(t) * o_st + int64_t(hq) * o_sh + ch * 4, acc, l);
}

// Enqueues the merge of n_rows rows (n_rows < 0: capacity `cap_rows`, the count read on the
// device): combine-list rows, or with slots > 0 the tokens of a slotted plan.
template <typename T>
int launch_combine(hipStream_t s, const int32_t* plan_dev, int32_t n_rows, int32_t cap_rows,
                   int32_t combine_off, int32_t slots, int32_t n_q_heads, int32_t head_dim,
                   const float2* ml, const float* pacc, void* out, int64_t o_st, int64_t o_sh) {
  const int rows = n_rows >= 0 ? n_rows : cap_rows;
  const int ch_log2 = log2_exact(head_dim / 4);
  const int64_t threads = (int64_t(rows) * n_q_heads) << ch_log2;
  if (ch_log2 < 0 || head_dim % 4 != 0)
    return fail(EDGERAG_EUNSUPPORTED, "attention combine: head_dim %d", head_dim);
  if (threads > INT32_MAX - 256)
    return fail(EDGERAG_EUNSUPPORTED, "attention combine: %d rows x %d heads too many", rows,
                n_q_heads);
  if (threads == 0) return EDGERAG_OK;
  constexpr int kThreads = EDGERAG_COMBINE_THREADS;
  const dim3 block(kThreads), grid(unsigned((threads + kThreads - 1) / kThreads));
  const auto* acc4 = reinterpret_cast<const float4*>(pacc);
  T* o = static_cast<T*>(out);
  const bool vec = reinterpret_cast<uintptr_t>(out) % (4 * sizeof(T)) == 0 && o_st % 4 == 0 &&
                   o_sh % 4 == 0;
  if (slots > 0) {
    if (vec)
      hipLaunchKernelGGL((attn_combine_slots_kernel<T, true>), grid, block, 0, s, plan_dev, n_rows,
                         slots, n_q_heads, ch_log2, ml, acc4, o, o_st, o_sh);
    else
      hipLaunchKernelGGL((attn_combine_slots_kernel<T, false>), grid, block, 0, s, plan_dev,
                         n_rows, slots, n_q_heads, ch_log2, ml, acc4, o, o_st, o_sh);
  } else if (vec) {
    hipLaunchKernelGGL((attn_combine_kernel<T, true>), grid, block, 0, s, plan_dev, n_rows,
                       combine_off, n_q_heads, ch_log2, ml, acc4, o, o_st, o_sh);
  } else {
    hipLaunchKernelGGL((attn_combine_kernel<T, false>), grid, block, 0, s, plan_dev, n_rows,
                       combine_off, n_q_heads, ch_log2, ml, acc4, o, o_st, o_sh);
  }
  return EDGERAG_OK;
}

int elem_size(int32_t dtype) {
  switch (dtype) {
    case EDGERAG_F32: return 4;
    case EDGERAG_F16: return 2;
    case EDGERAG_BF16: return 2;
    default: return 0;
  }
}

bool head_dim_supported(int32_t d) {
  return d == 8 || d == 16 || d == 32 || d == 64 || d == 128 || d == 256;
}

int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

int pow2_at_least(int v) {
  int p = 1;
  while (p < v) p <<= 1;
  return p;
}

// One (request, query tile, KV split) of the plan: it becomes one work item per kv head. All
// heads of a group cost the same, so the planner orders groups, not items.
struct PlanGroup {
  int32_t req, q_begin, q_count, kv_begin, kv_end, split;
  int64_t cost;
};

// Workspace: [(m, l) pairs | acc rows] of the split partials.
struct WorkspaceLayout {
  int64_t acc_off, total;
};

WorkspaceLayout workspace_layout(int64_t n_partials, int64_t head_dim) {
  WorkspaceLayout w{};
  w.acc_off = round_up(n_partials * int64_t(sizeof(float2)), 256);
  w.total = w.acc_off + round_up(n_partials * head_dim * int64_t(sizeof(float)), 256);
  return w;
}

using Launch = AttnLaunch;

// waves > 0: workgroup-split rows (one workgroup of `waves` waves per item), else one wave per
// item.
template <typename T, int D, int QR, int U, bool WG>
void launch_decode_mode(const Launch& a, int base, int count, int limit_word, int waves) {
  const dim3 grid(count), block(WG ? waves * kWave : kWave);
  if (a.nk != nullptr)
    hipLaunchKernelGGL((attn_decode_kernel<T, D, QR, U, true, WG>), grid, block, 0, a.s,
                       a.plan, base, limit_word, a.qsl, a.ctx, a.bt, a.bt_stride, a.nb, a.bs,
                       static_cast<const T*>(a.q), a.q_st, a.q_sh, static_cast<const T*>(a.kp),
                       static_cast<const T*>(a.vp), a.hq, a.hkv, a.scale_log2,
                       static_cast<T*>(a.out), a.o_st, a.o_sh, a.ml, a.pacc,
                       static_cast<const T*>(a.nk), static_cast<const T*>(a.nv), a.n_st, a.n_sh,
                       a.slots, static_cast<T*>(const_cast<void*>(a.kp)),
                       static_cast<T*>(const_cast<void*>(a.vp)));
  else
    hipLaunchKernelGGL((attn_decode_kernel<T, D, QR, U, false, WG>), grid, block, 0, a.s,
                       a.plan, base, limit_word, a.qsl, a.ctx, a.bt, a.bt_stride, a.nb, a.bs,
                       static_cast<const T*>(a.q), a.q_st, a.q_sh, static_cast<const T*>(a.kp),
                       static_cast<const T*>(a.vp), a.hq, a.hkv, a.scale_log2,
                       static_cast<T*>(a.out), a.o_st, a.o_sh, a.ml, a.pacc,
                       nullptr, nullptr, 0, 0, nullptr, nullptr, nullptr);
}

template <typename T, int D, int QR, int U>
void launch_decode(const Launch& a, int base, int count, int limit_word, int waves) {
  // Workgroup rows never get more query vectors per pass than dispatch_decode_qr allows them.
  constexpr int kWgQr = __is_same(T, bf16) ? EDGERAG_WG_QR_MAX_BF16 : EDGERAG_WG_QR_MAX;
  if constexpr (D <= 128 && QR <= kWgQr) {
    if (waves > 0) {
      launch_decode_mode<T, D, QR, U, true>(a, base, count, limit_word, waves);
      return;
    }
  }
  launch_decode_mode<T, D, QR, U, false>(a, base, count, limit_word, 0);
}

template <typename T, int D, int QR>
void launch_rows(const Launch& a, int base, int count, int limit_word) {
  hipLaunchKernelGGL((attn_rows_kernel<T, D, QR>), dim3(count), dim3(kWave), 0, a.s, a.plan,
                     base, limit_word, a.qsl, a.ctx, a.bt, a.bt_stride, a.nb, a.bs,
                     static_cast<const T*>(a.q), a.q_st, a.q_sh, static_cast<const T*>(a.kp),
                     static_cast<const T*>(a.vp), a.hq, a.hkv, a.scale_log2,
                     static_cast<T*>(a.out), a.o_st, a.o_sh, a.ml, a.pacc);
}

template <typename T, int D>
void dispatch_decode_qr(const Launch& a, int qr, int base, int count, int limit_word,
                        int waves) {
  constexpr int U = D >= 256 ? 2 : kDecodeU;
  // Workgroup rows (up to 16 waves, 128 registers per lane) take at most 4 query vectors per
  // pass: a pass of 8 spills 236-264 B per lane to scratch (fp16; ~430 B for bf16, whose query
  // vectors are fp32). GQA groups of 8 then take two passes over the keys, the second mostly from
  // L2: 32 q / 4 kv heads, 64 decodes of 4,000 tokens, 309.6 -> 116.5 us (fp16), 291 -> 138 (bf16).
  if (waves > 0) qr = min(qr, __is_same(T, bf16) ? EDGERAG_WG_QR_MAX_BF16 : EDGERAG_WG_QR_MAX);
#ifdef EDGERAG_WG_U
  if (waves > 0 && waves < kMaxRowWaves && qr == 1) {
    launch_decode<T, D, 1, (D >= 256 ? 2 : EDGERAG_WG_U)>(a, base, count, limit_word, waves);
    return;
  }
#endif
  switch (qr) {
    case 1: launch_decode<T, D, 1, U>(a, base, count, limit_word, waves); break;
    case 2: launch_decode<T, D, 2, U>(a, base, count, limit_word, waves); break;
    case 4: launch_decode<T, D, 4, U>(a, base, count, limit_word, waves); break;
    default: launch_decode<T, D, 8, 2>(a, base, count, limit_word, waves); break;
  }
}

template <typename T, int D>
void dispatch_rows_qr(const Launch& a, int qr, int base, int count, int limit_word) {
  switch (qr) {
    case 1: launch_rows<T, D, 1>(a, base, count, limit_word); break;
    case 2: launch_rows<T, D, 2>(a, base, count, limit_word); break;
    case 4: launch_rows<T, D, 4>(a, base, count, limit_word); break;
    default: launch_rows<T, D, 8>(a, base, count, limit_word); break;
  }
}

// Tile items (prefill slices) first: the MFMA tile kernel for fp16 / head_dim 64, the general
// row kernel with 8 query vectors per pass otherwise. Row items: the fast decode kernel when
// every split's load groups stay inside one block, the general kernel otherwise.
template <typename T, int D>
int run_items(const Launch& a, const int32_t* ph, int parts) {
  using C = RowCfg<T, D>;
  const int n_items = ph[H_N_ITEMS], n_row = ph[H_N_ROW_ITEMS];
  if ((parts & EDGERAG_ATTN_TILES) && n_items > n_row) {
    if constexpr (__is_same(T, f16) && D == 64) {
      if (ph[H_TILE_KIND] == 1 && prefill_tiles_supported(a.nb, a.bs)) {
        launch_prefill_tiles_f16_d64(a, n_row, n_items - n_row,
                                     (parts & EDGERAG_ATTN_TILES_SHARED) != 0);
      } else {
        dispatch_rows_qr<T, D>(a, 8, n_row, n_items - n_row, H_N_ITEMS);
      }
    } else {
      dispatch_rows_qr<T, D>(a, 8, n_row, n_items - n_row, H_N_ITEMS);
    }
  }
  const int qr = std::min(8, pow2_at_least(std::max(1, ph[H_MAX_ROW_VECS])));
  const bool fast = a.bs % C::TPW == 0 && ph[H_MAX_SPLIT_BLOCKS] <= kMaxSplitBlocks;
  if ((parts & EDGERAG_ATTN_ROWS) && n_row > 0) {
    if (fast)
      dispatch_decode_qr<T, D>(a, qr, 0, n_row, H_N_ROW_ITEMS, ph[H_ROW_WAVES]);
    else  // (workgroup-split rows are only planned for the fast kernel)
      dispatch_rows_qr<T, D>(a, qr, 0, n_row, H_N_ROW_ITEMS);
  }
  return check_launch("edgerag_paged_attention");
}

template <typename T>
int run_dtype(const Launch& a, const int32_t* ph, int32_t D, int parts) {
  switch (D) {
    case 8: return run_items<T, 8>(a, ph, parts);
    case 16: return run_items<T, 16>(a, ph, parts);
    case 32: return run_items<T, 32>(a, ph, parts);
    case 64: return run_items<T, 64>(a, ph, parts);
    case 128: return run_items<T, 128>(a, ph, parts);
    case 256: return run_items<T, 256>(a, ph, parts);
  }
  return fail(EDGERAG_EUNSUPPORTED, "edgerag_paged_attention: head_dim %d", D);
}

}  // namespace
}  // namespace edgerag

using namespace edgerag;

extern "C" int edgerag_attn_plan_ex(const int32_t* query_start_loc, const int32_t* context_lens,
                                    int32_t num_reqs, int32_t n_q_heads, int32_t n_kv_heads,
                                    int32_t head_dim, int32_t block_size,
                                    int32_t max_blocks_per_seq, int32_t dtype, int32_t flags,
                                    int32_t* plan, int64_t plan_capacity_words,
                                    int64_t* plan_words, int64_t* workspace_bytes) {
  clear_error();
  if ((flags & ~(EDGERAG_PLAN_SPLIT_ROWS | EDGERAG_PLAN_OVERLAP)) != 0)
    return fail(EDGERAG_EINVAL, "edgerag_attn_plan: flags %d", flags);
  if (plan_words == nullptr || workspace_bytes == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_attn_plan: plan_words/workspace_bytes are NULL");
  if (num_reqs < 0) return fail(EDGERAG_EINVAL, "edgerag_attn_plan: num_reqs < 0");
  if (num_reqs > 0 && (query_start_loc == nullptr || context_lens == nullptr))
    return fail(EDGERAG_EINVAL, "edgerag_attn_plan: NULL metadata");
  if (n_q_heads <= 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads != 0)
    return fail(EDGERAG_EINVAL,
                "edgerag_attn_plan: %d query heads against %d kv heads (need a positive multiple)",
                n_q_heads, n_kv_heads);
  if (!head_dim_supported(head_dim))
    return fail(EDGERAG_EUNSUPPORTED, "edgerag_attn_plan: head_dim %d (supported: 8..256, pow2)",
                head_dim);
  if (elem_size(dtype) == 0) return fail(EDGERAG_EINVAL, "edgerag_attn_plan: dtype %d", dtype);
  if (block_size <= 0 || max_blocks_per_seq < 0)
    return fail(EDGERAG_EINVAL, "edgerag_attn_plan: block_size %d, max_blocks %d", block_size,
                max_blocks_per_seq);

  const int n_rep = n_q_heads / n_kv_heads;
  // Prefill tiles run on MFMA for fp16 / head_dim 64: 128 virtual rows (token x head-in-group).
  const bool mfma_tiles = dtype == EDGERAG_F16 && head_dim == 64 && n_rep <= kMfmaTileRows;
  const int tile_rows = mfma_tiles ? kMfmaTileRows / n_rep : kQTile;
  int64_t work = 0;       // KV token-heads the decode rows read, to size their splits
  int64_t tile_work = 0;  // tile x keys of the prefill slices, to size theirs
  int64_t n_tiles = 0;    // prefill tile items before any KV split
  int64_t max_len = 0;
  for (int r = 0; r < num_reqs; ++r) {
    const int64_t c = int64_t(query_start_loc[r + 1]) - query_start_loc[r];
    const int64_t L = context_lens[r];
    if (c < 0) return fail(EDGERAG_EINVAL, "edgerag_attn_plan: query_start_loc decreases at %d", r);
    if (L < 0 || c > L)
      return fail(EDGERAG_EINVAL,
                  "edgerag_attn_plan: request %d has %lld queries but context %lld (append the "
                  "new tokens before attending)",
                  r, (long long)c, (long long)L);
    if ((L + block_size - 1) / block_size > max_blocks_per_seq)
      return fail(EDGERAG_EINVAL,
                  "edgerag_attn_plan: request %d needs %lld blocks, block table holds %d", r,
                  (long long)((L + block_size - 1) / block_size), max_blocks_per_seq);
    if (c > 0 && c * n_rep <= kMaxRowVecs) work += L * n_kv_heads;
    if (c * n_rep > kMaxRowVecs) {
      tile_work += (c + tile_rows - 1) / tile_rows * n_kv_heads * L;
      n_tiles += (c + tile_rows - 1) / tile_rows * n_kv_heads;
    }
    max_len = std::max(max_len, L);
  }
  // Decode rows as one workgroup of kRowWgWaves waves per (request, kv head) whose waves split
  // the keys and merge in LDS, when the fast decode kernel takes them and every row's context
  // fits kRowWgWaves parts of at most EDGERAG_ROW_WG_PART tokens. Longer contexts would leave
  // each wave a long, latency-bound stream while the chip idles (measured: cfg2 -2%, cfg5 with 8
  // long requests -5%), so those batches (or any, when asked) keep one workgroup per KV split,
  // merged by the combine launch through fp32 partials. Beside prefill tiles, when the rows'
  // workgroups cover every CU, the chip does not idle (the tiles take the slack), so parts of up
  // to EDGERAG_ROW_WG_PART_TILES tokens stay workgroup-split (as long as the rows are few enough
  // for EDGERAG_ROW_WG_MAX_ITEMS). Fewer row workgroups than CUs (a 512-token chunk beside 7
  // decodes, 224 of them) left a few CUs with long streams: -2.5% output tokens/s end to end.
  static_assert(kRowWgWaves >= 1 && kRowWgWaves <= kMaxRowWaves, "row workgroup size");
  static_assert(kRowPartWaves >= 1 && kRowPartWaves <= kMaxRowWaves, "part workgroup size");
  int64_t row_items = 0, max_row_len = 0;
  for (int r = 0; r < num_reqs; ++r) {
    const int64_t c = int64_t(query_start_loc[r + 1]) - query_start_loc[r];
    if (c > 0 && c * n_rep <= kMaxRowVecs) {
      row_items += n_kv_heads;
      max_row_len = std::max<int64_t>(max_row_len, context_lens[r]);
    }
  }
  const int es = elem_size(dtype);
  // Tiles and rows on two streams (the tiles at one workgroup per CU, the rows in the rest of
  // each CU) pay only when both sides are heavy: the tiles fill every CU and the rows stream at
  // least kOverlapRowBytes of K/V. Otherwise one stream runs the tiles at full occupancy and then
  // the rows, which also saves the host the fork and join of the streams. (Three 512-token
  // slices beside 24 decodes of up to 7,472 tokens, 707 MB of rows: 0.175 against 0.258 ms on
  // one stream. One 512-token chunk, 128 tiles, beside 7 decodes of 32-256 MB: every prefill
  // iteration of the config-5 serving trace was faster on one stream.)
  const bool overlap = n_tiles > 0 && row_items > 0 &&
                       ((flags & EDGERAG_PLAN_OVERLAP) ||
                        (n_tiles >= kPlanCUs && work * head_dim * 2 * es >= kOverlapRowBytes));
  // Batches with fewer row workgroups than CUs (one or a few long decodes: 32 workgroups for a
  // single request of 32 kv heads) instead cut every context into parts, one workgroup each, so
  // that about kRowTargetWgs workgroups cover the chip; a context's parts write fp32 partials
  // that the merge launch combines. Parts are whole blocks, at least kRowMinWaveTokens tokens per
  // wave (16 when every context is short; shorter streams are all fixed cost) and at most the
  // per-wave cap above.
  const bool wg_capable =
      EDGERAG_ROW_WG && !(flags & EDGERAG_PLAN_SPLIT_ROWS) && row_items > 0 && head_dim <= 128 &&
      head_dim % (16 / es) == 0 && head_dim / (16 / es) <= kWave &&
      block_size % (kWave / (head_dim / (16 / es))) == 0;
  const int64_t wave_cap = std::min<int64_t>(
      overlap && row_items >= kPlanCUs ? EDGERAG_ROW_WG_PART_TILES : EDGERAG_ROW_WG_PART,
      int64_t(kMaxSplitBlocks) * block_size);
  const int64_t part_cap = int64_t(kRowWgWaves) * round_up(wave_cap, block_size);
  bool wg_rows = false;
  int row_waves = 0;
  int slots = 0;        // partial slots per (token, q head) of the row requests (0: nsplit)
  int64_t wg_part = 0;  // longest part of a context one row workgroup takes (0: whole contexts)
  if (wg_capable && kRowTargetWgs > 0 && row_items < kPlanCUs) {
    // Parts take kRowPartWaves waves: single-sequence attention over 6,758 tokens measured
    // 17.7 us at 8 waves against 21.5 us at 16 and 19.4 us at 4 (with the merge launch).
    // At most kRowTargetWgs workgroups plus one per (request, kv head) for the rounding: the
    // parts are never shorter than work / kRowTargetWgs (the waves' block-id registers bound
    // them only for contexts far past any BASELINE shape).
    const int min_wave_tokens = max_row_len <= EDGERAG_ROW_SHORT_CTX
                                    ? EDGERAG_ROW_MIN_WAVE_TOKENS_SHORT
                                    : kRowMinWaveTokens;
    const int64_t min_part = int64_t(kRowPartWaves) * round_up(min_wave_tokens, block_size);
    const int64_t want = (work + kRowTargetWgs - 1) / kRowTargetWgs;
    const int64_t cap = int64_t(kRowPartWaves) * kMaxSplitBlocks * block_size;
    wg_part = std::min(cap, std::max(min_part, round_up(want, block_size)));
    wg_rows = true;
    row_waves = kRowPartWaves;
    // The parts write their partials to S fixed slots per (token, q head), the unused ones
    // marked empty, so that a merge addresses every partial from its thread index alone and
    // needs one round trip (attn_combine_slots_kernel). S (a power of two) covers the parts
    // kRowTargetWgs workgroups give one request; contexts that would need more take longer parts.
    // A batch whose contexts all fit one part has nothing to merge and stays unslotted.
    const int64_t want_slots = (kRowTargetWgs + n_kv_heads - 1) / n_kv_heads;
    int s = 2;
    while (s < want_slots && s < kMaxPartSlots) s *= 2;
    const int64_t slot_part = round_up((max_row_len + s - 1) / s, block_size);
    if (slot_part <= cap && max_row_len > std::max(wg_part, slot_part)) {
      wg_part = std::max(wg_part, slot_part);
      slots = s;
    }
  } else if (wg_capable && max_row_len <= part_cap &&
             (row_items <= kPlanCUs ||
              (row_items <= EDGERAG_ROW_WG_MAX_ITEMS && max_row_len <= EDGERAG_ROW_WG_SHORT))) {
    wg_rows = true;
    row_waves = kRowWgWaves;
  } else if (wg_capable && EDGERAG_ROW_WG_LONG) {
    wg_part = part_cap;
    wg_rows = true;
    row_waves = kRowWgWaves;
  }
  // Tokens of a row request's parts: equal whole-block parts of at most wg_part tokens.
  auto wg_split_len = [&](int64_t L) -> int64_t {
    if (wg_part == 0 || L <= wg_part) return std::max<int64_t>(L, 1);
    const int64_t n = (L + wg_part - 1) / wg_part;
    return round_up((L + n - 1) / n, block_size);
  };
  const int64_t longest_part = wg_rows ? wg_split_len(max_row_len) : 0;
  const int wg_split_blocks =
      wg_rows ? int(((longest_part + row_waves - 1) / row_waves + block_size - 1) / block_size)
              : 0;
  int64_t split_len = std::max<int64_t>(kMinSplit, (work + kTargetItems - 1) / kTargetItems);
  split_len = round_up(split_len, block_size);
  split_len = std::min<int64_t>(split_len, int64_t(kMaxSplitBlocks) * block_size);
  const int split_blocks = int((split_len + block_size - 1) / block_size);
  // Prefill tiles: split the keys only when there are too few tiles to fill the GPU's tile slots,
  // and then only as far as needed for about that many items, in whole 64-key LDS tiles; every
  // extra split costs a partial write and a merge. Beside decode rows (overlap) the tiles run at
  // one workgroup per CU (the rows take the rest of each CU), otherwise at two: kTargetTiles / 2
  // or kTargetTiles items. (Three 512-token slices, 384 tiles, beside 24 decodes: splitting them to
  // 768 items for the larger target measured 0.225 against 0.215 ms per step.)
  // A split may span at most kMaxTileBlocks blocks (the MFMA tile kernel stages its block ids).
  const int64_t target_tiles = overlap ? kTargetTiles / 2 : kTargetTiles;
  const int64_t tile_split_cap =
      std::max<int64_t>(64, int64_t(kMaxTileBlocks - 1) * block_size / 64 * 64);
  const int64_t tile_share = round_up(
      std::max<int64_t>(kMinTileSplit, (tile_work + target_tiles - 1) / target_tiles), 64);
  const int64_t tile_part = std::min(
      tile_split_cap, (EDGERAG_TILE_BALANCE || n_tiles < target_tiles)
                          ? tile_share
                          : round_up(std::max<int64_t>(max_len, 1), 64));
  // Keys of a tile request's splits: equal 64-key multiples of at most tile_part.
  auto tile_split_len = [&](int64_t L) -> int64_t {
    const int64_t n = std::max<int64_t>(1, (L + tile_part - 1) / tile_part);
    return std::min(tile_split_cap, round_up((std::max<int64_t>(L, 1) + n - 1) / n, 64));
  };

  // Scratch reused across calls on a thread: the planner runs once per step on the host.
  thread_local std::vector<PlanGroup> rows, tiles;
  thread_local std::vector<int32_t> reqs, combine;
  rows.clear();
  tiles.clear();
  combine.clear();
  reqs.assign(size_t(num_reqs) * kReqWords, 0);
  int64_t n_partials = 0;
  int max_row_vecs = 0;
  for (int r = 0; r < num_reqs; ++r) {
    const int q0 = query_start_loc[r];
    const int c = query_start_loc[r + 1] - q0;
    const int L = context_lens[r];
    int32_t* rq = reqs.data() + size_t(r) * kReqWords;
    const bool row = c * n_rep <= kMaxRowVecs;
    // Workgroup-split rows: one item per part of the context (the waves split the part).
    const int64_t slen = row ? (wg_rows ? wg_split_len(L) : split_len) : tile_split_len(L);
    const int nsplit = c == 0 ? 0 : int((L + slen - 1) / slen);
    // Slotted row requests write partials (and get merge rows) even when not split.
    const bool slotted = slots > 0 && row;
    const int pstride = slotted ? slots : nsplit;
    rq[R_NSPLIT] = nsplit;
    rq[R_SPLITLEN] = int32_t(slen);
    rq[R_PARTOFF] = int32_t(n_partials);
    rq[R_PSTRIDE] = pstride;
    if (c == 0) continue;
    if (nsplit > 1 || slotted) {
      for (int t = q0; t < q0 + c; ++t) {
        const int32_t e[kCombineWords] = {t, q0, c, L, nsplit, int32_t(slen),
                                          int32_t(n_partials), pstride};
        combine.insert(combine.end(), e, e + kCombineWords);
      }
      n_partials += int64_t(c) * n_q_heads * pstride;
    }
    if (n_partials > INT32_MAX)
      return fail(EDGERAG_EUNSUPPORTED, "edgerag_attn_plan: batch needs > 2^31 split partials");
    const int rows_per_item = row ? c : tile_rows;
    if (row) max_row_vecs = std::max(max_row_vecs, c * n_rep);
    auto& groups = row ? rows : tiles;
    for (int tile = 0; tile < c; tile += rows_per_item) {
      const int qc = std::min(rows_per_item, c - tile);
      const int last_visible = L - c + tile + qc - 1;  // causal limit of the tile's last row
      for (int s = 0; s < nsplit; ++s) {
        const int kb = int(s * slen);
        if (kb > last_visible) break;
        const int ke = int(std::min<int64_t>(L, (s + 1) * slen));
        const int ke_eff = std::min(ke, last_visible + 1);
        groups.push_back(PlanGroup{r, q0 + tile, qc, kb, ke_eff, s,
                                   int64_t(ke_eff - kb) * (row ? 1 : qc * n_rep)});
      }
    }
  }
  // Heaviest first: the dispatcher hands blocks out in index order, so this is LPT scheduling.
  // Stable, so equal costs keep request order; a group's heads stay adjacent in head order.
  auto heavier = [](const PlanGroup& a, const PlanGroup& b) { return a.cost > b.cost; };
  std::stable_sort(rows.begin(), rows.end(), heavier);
  std::stable_sort(tiles.begin(), tiles.end(), heavier);

  const int64_t n_row_items = int64_t(rows.size()) * n_kv_heads;
  const int64_t n_items = n_row_items + int64_t(tiles.size()) * n_kv_heads;
  const int64_t item_off = kHeaderWords;  // the decode kernel reads items at this offset
  const int64_t req_off = item_off + n_items * kItemWords;
  const int64_t combine_off = req_off + int64_t(num_reqs) * kReqWords;  // 16-byte aligned
  const int64_t words = combine_off + int64_t(combine.size());
  *plan_words = words;
  *workspace_bytes = workspace_layout(n_partials, head_dim).total;
  if (plan == nullptr) return EDGERAG_OK;
  if (plan_capacity_words < words)
    return fail(EDGERAG_EWORKSPACE, "edgerag_attn_plan: plan needs %lld words, capacity %lld",
                (long long)words, (long long)plan_capacity_words);
  if (words > INT32_MAX) return fail(EDGERAG_EUNSUPPORTED, "edgerag_attn_plan: plan too large");
  std::fill(plan, plan + kHeaderWords, 0);
  plan[H_MAGIC] = kPlanMagic;
  plan[H_VERSION] = kPlanVersion;
  plan[H_N_ITEMS] = int32_t(n_items);
  plan[H_N_REQS] = num_reqs;
  plan[H_ITEM_OFF] = int32_t(item_off);
  plan[H_REQ_OFF] = int32_t(req_off);
  plan[H_N_PARTIALS] = int32_t(n_partials);
  plan[H_N_Q_HEADS] = n_q_heads;
  plan[H_N_KV_HEADS] = n_kv_heads;
  plan[H_HEAD_DIM] = head_dim;
  plan[H_BLOCK_SIZE] = block_size;
  plan[H_DTYPE] = dtype;
  plan[H_NUM_TOKENS_HINT] = num_reqs > 0 ? query_start_loc[num_reqs] : 0;
  plan[H_N_ROW_ITEMS] = int32_t(n_row_items);
  plan[H_MAX_ROW_VECS] = max_row_vecs;
  plan[H_MAX_SPLIT_BLOCKS] = wg_rows ? wg_split_blocks : split_blocks;
  plan[H_N_COMBINE] = int32_t(combine.size() / kCombineWords);
  plan[H_COMBINE_OFF] = int32_t(combine_off);
  plan[H_TILE_KIND] = mfma_tiles ? 1 : 0;
  plan[H_ROW_WAVES] = row_waves;
  plan[H_OVERLAP] = overlap ? 1 : 0;
  plan[H_SLOTS] = slots;
  std::copy(combine.begin(), combine.end(), plan + combine_off);
  int32_t* dst = plan + item_off;
  for (const auto* groups : {&rows, &tiles})
    for (const PlanGroup& g : *groups)
      for (int h = 0; h < n_kv_heads; ++h, dst += kItemWords) {
        dst[I_REQ] = g.req;
        dst[I_HEAD] = h;
        dst[I_QBEGIN] = g.q_begin;
        dst[I_QCOUNT] = g.q_count;
        dst[I_KVBEGIN] = g.kv_begin;
        dst[I_KVEND] = g.kv_end;
        dst[I_SPLIT] = g.split;
        dst[I_PAD] = 0;
      }
  std::copy(reqs.begin(), reqs.end(), plan + req_off);
  return EDGERAG_OK;
}

extern "C" int64_t edgerag_attn_fixed_row_items(int32_t max_reqs, int32_t n_kv_heads,
                                                int32_t max_context, int32_t block_size) {
  if (max_reqs < 0 || n_kv_heads <= 0 || max_context < 0 || block_size <= 0) return -1;
  // The planner's row workgroups for decode-only batches (no tiles beside them): whole contexts,
  // one per (request, kv head); a batch of fewer such workgroups than CUs cut into parts of at
  // least ceil(work / kRowTargetWgs) tokens (at most kRowTargetWgs plus one per (request, kv
  // head) for the rounding) or of the per-wave cap, whichever is longer; contexts past the cap
  // in parts of the cap.
  const int64_t rh = int64_t(max_reqs) * n_kv_heads;
  const int64_t wave_cap =
      std::min<int64_t>(EDGERAG_ROW_WG_PART, int64_t(kMaxSplitBlocks) * block_size);
  const int64_t part_cap = int64_t(kRowWgWaves) * round_up(wave_cap, block_size);
  const int64_t per_req = std::max<int64_t>(1, (int64_t(max_context) + part_cap - 1) / part_cap);
  // Few-row parts: at most kRowTargetWgs + rh, or parts of the block-id cap when that binds.
  const int64_t small_cap = int64_t(kRowPartWaves) * kMaxSplitBlocks * block_size;
  const int64_t per_req_small =
      std::max<int64_t>(1, (int64_t(max_context) + small_cap - 1) / small_cap);
  return std::max<int64_t>(
      {kRowTargetWgs + rh, rh * per_req, std::min<int64_t>(rh, kPlanCUs - 1) * per_req_small});
}

extern "C" int edgerag_attn_plan(const int32_t* query_start_loc, const int32_t* context_lens,
                                 int32_t num_reqs, int32_t n_q_heads, int32_t n_kv_heads,
                                 int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq,
                                 int32_t dtype, int32_t* plan, int64_t plan_capacity_words,
                                 int64_t* plan_words, int64_t* workspace_bytes) {
  return edgerag_attn_plan_ex(query_start_loc, context_lens, num_reqs, n_q_heads, n_kv_heads,
                              head_dim, block_size, max_blocks_per_seq, dtype, 0, plan,
                              plan_capacity_words, plan_words, workspace_bytes);
}

namespace edgerag {
namespace {

// The new K/V rows of an append fused into the decode rows.
struct FusedAppend {
  const void *k, *v;
  int64_t st, sh;
  const int32_t* slots;
};

// Whether the decode rows of this plan run on the fast decode kernel (the one that can fuse the
// append): block_size a multiple of its tokens per load, splits within its block-id registers.
bool fast_decode_rows(int32_t dtype, int32_t head_dim, int32_t block_size, const int32_t* ph) {
  const int es = elem_size(dtype);
  if (es == 0 || head_dim <= 0 || head_dim % (16 / es) != 0) return false;
  const int lpt = head_dim / (16 / es);
  if (lpt < 1 || lpt > kWave) return false;
  return block_size % (kWave / lpt) == 0 && ph[H_MAX_SPLIT_BLOCKS] <= kMaxSplitBlocks;
}

int paged_attention_impl(
    const int32_t* plan_host, const int32_t* plan_dev, int64_t plan_words, const void* q,
    int64_t q_stride_tok, int64_t q_stride_head, const void* key_pool, const void* value_pool,
    int32_t dtype, const int32_t* block_tables, int64_t block_tables_stride,
    const int32_t* query_start_loc, const int32_t* context_lens, int32_t num_reqs,
    int32_t num_tokens, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
    int32_t block_size, int32_t num_blocks, float scale, void* out, int64_t out_stride_tok,
    int64_t out_stride_head, void* workspace, int64_t workspace_bytes, int32_t parts,
    void* stream, const FusedAppend* app) {
  if (parts <= 0 || (parts & ~(EDGERAG_ATTN_ALL | EDGERAG_ATTN_TILES_SHARED)) != 0 ||
      (parts & EDGERAG_ATTN_ALL) == 0)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention: parts mask %d", parts);
  if (plan_host == nullptr || plan_dev == nullptr || plan_words < kHeaderWords ||
      plan_host[H_MAGIC] != kPlanMagic || plan_host[H_VERSION] != kPlanVersion)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention: not a plan from edgerag_attn_plan");
  if (plan_host[H_N_REQS] != num_reqs || plan_host[H_N_Q_HEADS] != n_q_heads ||
      plan_host[H_N_KV_HEADS] != n_kv_heads || plan_host[H_HEAD_DIM] != head_dim ||
      plan_host[H_BLOCK_SIZE] != block_size || plan_host[H_DTYPE] != dtype)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention: plan was made for a different shape");
  if (plan_host[H_NUM_TOKENS_HINT] > num_tokens)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention: plan covers %d tokens, q holds %d",
                plan_host[H_NUM_TOKENS_HINT], num_tokens);
  if (num_blocks <= 0) return fail(EDGERAG_EINVAL, "edgerag_paged_attention: num_blocks <= 0");
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention: scale must be positive and finite");
  const int n_items = plan_host[H_N_ITEMS];
  const int64_t n_partials = plan_host[H_N_PARTIALS];
  const WorkspaceLayout ws = workspace_layout(n_partials, head_dim);
  if (workspace_bytes < ws.total || (ws.total > 0 && workspace == nullptr))
    return fail(EDGERAG_EWORKSPACE, "edgerag_paged_attention: workspace %lld bytes, need %lld",
                (long long)workspace_bytes, (long long)ws.total);
  if (n_items == 0) return EDGERAG_OK;
  if (q == nullptr || key_pool == nullptr || value_pool == nullptr || out == nullptr ||
      block_tables == nullptr || query_start_loc == nullptr || context_lens == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention: NULL pointer");
  const int es = elem_size(dtype);
  if (!aligned16(key_pool) || !aligned16(value_pool) || !aligned16(q) ||
      (q_stride_tok * es) % 16 != 0 || (q_stride_head * es) % 16 != 0)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention: q and pools must be 16-byte aligned");

  Launch a{};
  a.s = static_cast<hipStream_t>(stream);
  a.q = q;
  a.q_st = q_stride_tok;
  a.q_sh = q_stride_head;
  a.kp = key_pool;
  a.vp = value_pool;
  a.bt = block_tables;
  a.bt_stride = block_tables_stride;
  a.qsl = query_start_loc;
  a.ctx = context_lens;
  a.plan = plan_dev;
  a.hq = n_q_heads;
  a.hkv = n_kv_heads;
  a.nb = num_blocks;
  a.bs = block_size;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out = out;
  a.o_st = out_stride_tok;
  a.o_sh = out_stride_head;
  char* wsp = static_cast<char*>(workspace);
  a.ml = reinterpret_cast<float2*>(wsp);
  a.pacc = reinterpret_cast<float*>(wsp + ws.acc_off);
  if (app != nullptr) {
    a.nk = app->k;
    a.nv = app->v;
    a.n_st = app->st;
    a.n_sh = app->sh;
    a.slots = app->slots;
  }
  int rc = EDGERAG_OK;
  switch (dtype) {
    case EDGERAG_F32: rc = run_dtype<float>(a, plan_host, head_dim, parts); break;
    case EDGERAG_F16: rc = run_dtype<f16>(a, plan_host, head_dim, parts); break;
    case EDGERAG_BF16: rc = run_dtype<bf16>(a, plan_host, head_dim, parts); break;
    default: return fail(EDGERAG_EINVAL, "edgerag_paged_attention: dtype %d", dtype);
  }
  const int n_combine = plan_host[H_N_COMBINE];
  if (rc != EDGERAG_OK || n_combine == 0 || !(parts & EDGERAG_ATTN_COMBINE)) return rc;
  // A slotted plan of row requests only lists every token, in order: the one-round-trip merge.
  const int slots =
      plan_host[H_N_ITEMS] == plan_host[H_N_ROW_ITEMS] ? std::max(plan_host[H_SLOTS], 0) : 0;

  switch (dtype) {
#define EDGERAG_COMBINE(TYPE)                                                                     \
  rc = launch_combine<TYPE>(a.s, plan_dev, n_combine, n_combine, plan_host[H_COMBINE_OFF], slots, \
                            n_q_heads, head_dim, a.ml, a.pacc, out, out_stride_tok,               \
                            out_stride_head)
    case EDGERAG_F32: EDGERAG_COMBINE(float); break;
    case EDGERAG_F16: EDGERAG_COMBINE(f16); break;
    case EDGERAG_BF16: EDGERAG_COMBINE(bf16); break;
#undef EDGERAG_COMBINE
  }
  if (rc != EDGERAG_OK) return rc;
  return check_launch("edgerag_paged_attention(combine)");
}

}  // namespace
}  // namespace edgerag

extern "C" int edgerag_paged_attention(
    const int32_t* plan_host, const int32_t* plan_dev, int64_t plan_words, const void* q,
    int64_t q_stride_tok, int64_t q_stride_head, const void* key_pool, const void* value_pool,
    int32_t dtype, const int32_t* block_tables, int64_t block_tables_stride,
    const int32_t* query_start_loc, const int32_t* context_lens, int32_t num_reqs,
    int32_t num_tokens, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
    int32_t block_size, int32_t num_blocks, float scale, void* out, int64_t out_stride_tok,
    int64_t out_stride_head, void* workspace, int64_t workspace_bytes, int32_t parts,
    void* stream) {
  clear_error();
  return paged_attention_impl(plan_host, plan_dev, plan_words, q, q_stride_tok, q_stride_head,
                              key_pool, value_pool, dtype, block_tables, block_tables_stride,
                              query_start_loc, context_lens, num_reqs, num_tokens, n_q_heads,
                              n_kv_heads, head_dim, block_size, num_blocks, scale, out,
                              out_stride_tok, out_stride_head, workspace, workspace_bytes, parts,
                              stream, nullptr);
}

extern "C" int edgerag_paged_attention_append(
    const void* new_key, const void* new_value, int32_t new_dtype, int64_t new_stride_tok,
    int64_t new_stride_head, const int32_t* slot_mapping, const int32_t* plan_host,
    const int32_t* plan_dev, int64_t plan_words, const void* q, int64_t q_stride_tok,
    int64_t q_stride_head, void* key_pool, void* value_pool, int32_t dtype,
    const int32_t* block_tables, int64_t block_tables_stride, const int32_t* query_start_loc,
    const int32_t* context_lens, int32_t num_reqs, int32_t num_tokens, int32_t n_q_heads,
    int32_t n_kv_heads, int32_t head_dim, int32_t block_size, int32_t num_blocks, float scale,
    void* out, int64_t out_stride_tok, int64_t out_stride_head, void* workspace,
    int64_t workspace_bytes, void* stream) {
  clear_error();
  if (new_key == nullptr || new_value == nullptr || slot_mapping == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention_append: NULL new K/V or slot mapping");
  if (plan_host == nullptr || plan_words < kHeaderWords || plan_host[H_MAGIC] != kPlanMagic)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention_append: not a plan from edgerag_attn_plan");
  const int es = elem_size(dtype);
  // One launch when every item is a decode row on the fast decode kernel and the new rows are
  // in the pool dtype, 16-byte aligned; otherwise the append, then the attention.
  const bool fused = plan_host[H_N_ITEMS] == plan_host[H_N_ROW_ITEMS] && new_dtype == dtype &&
                     es > 0 && aligned16(new_key) && aligned16(new_value) &&
                     (new_stride_tok * es) % 16 == 0 && (new_stride_head * es) % 16 == 0 &&
                     fast_decode_rows(dtype, head_dim, block_size, plan_host);
  if (!fused) {
    const int32_t n_new = num_reqs > 0 ? plan_host[H_NUM_TOKENS_HINT] : 0;
    if (int rc = edgerag_kv_append(new_key, new_value, new_dtype, new_stride_tok,
                                   new_stride_head, slot_mapping, n_new, key_pool, value_pool,
                                   dtype, n_kv_heads, num_blocks, block_size, head_dim, stream))
      return rc;
    return paged_attention_impl(plan_host, plan_dev, plan_words, q, q_stride_tok, q_stride_head,
                                key_pool, value_pool, dtype, block_tables, block_tables_stride,
                                query_start_loc, context_lens, num_reqs, num_tokens, n_q_heads,
                                n_kv_heads, head_dim, block_size, num_blocks, scale, out,
                                out_stride_tok, out_stride_head, workspace, workspace_bytes,
                                EDGERAG_ATTN_ALL, stream, nullptr);
  }
  const FusedAppend app{new_key, new_value, new_stride_tok, new_stride_head, slot_mapping};
  return paged_attention_impl(plan_host, plan_dev, plan_words, q, q_stride_tok, q_stride_head,
                              key_pool, value_pool, dtype, block_tables, block_tables_stride,
                              query_start_loc, context_lens, num_reqs, num_tokens, n_q_heads,
                              n_kv_heads, head_dim, block_size, num_blocks, scale, out,
                              out_stride_tok, out_stride_head, workspace, workspace_bytes,
                              EDGERAG_ATTN_ALL, stream, &app);
}

namespace edgerag {
namespace {

// Decode-row items of a fixed-capacity launch: the fast decode kernel when every load group of a
// split stays inside one block, the general row kernel otherwise (both bound-checked on device).
template <typename T, int D>
void run_rows_fixed(const Launch& a, int qr, int max_items, int row_waves) {
  using C = RowCfg<T, D>;
  if (a.bs % C::TPW == 0)
    dispatch_decode_qr<T, D>(a, qr, 0, max_items, H_N_ROW_ITEMS, row_waves);
  else
    dispatch_rows_qr<T, D>(a, qr, 0, max_items, H_N_ROW_ITEMS);
}

template <typename T>
int run_fixed_dtype(const Launch& a, int32_t D, int qr, int max_items, int row_waves) {
  switch (D) {
    case 8: run_rows_fixed<T, 8>(a, qr, max_items, row_waves); break;
    case 16: run_rows_fixed<T, 16>(a, qr, max_items, row_waves); break;
    case 32: run_rows_fixed<T, 32>(a, qr, max_items, row_waves); break;
    case 64: run_rows_fixed<T, 64>(a, qr, max_items, row_waves); break;
    case 128: run_rows_fixed<T, 128>(a, qr, max_items, row_waves); break;
    case 256: run_rows_fixed<T, 256>(a, qr, max_items, row_waves); break;
    default: return fail(EDGERAG_EUNSUPPORTED, "edgerag_paged_attention_fixed: head_dim %d", D);
  }
  return check_launch("edgerag_paged_attention_fixed");
}

}  // namespace
}  // namespace edgerag

extern "C" int edgerag_paged_attention_fixed(
    const int32_t* plan_dev, int32_t max_row_items, int32_t max_combine_rows,
    int32_t max_row_vecs, int64_t max_partials, int32_t row_waves, int32_t slots, const void* q,
    int64_t q_stride_tok,
    int64_t q_stride_head, const void* key_pool, const void* value_pool, int32_t dtype,
    const int32_t* block_tables, int64_t block_tables_stride, const int32_t* query_start_loc,
    const int32_t* context_lens, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
    int32_t block_size, int32_t num_blocks, float scale, void* out, int64_t out_stride_tok,
    int64_t out_stride_head, void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  if (plan_dev == nullptr || q == nullptr || key_pool == nullptr || value_pool == nullptr ||
      out == nullptr || block_tables == nullptr || query_start_loc == nullptr ||
      context_lens == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention_fixed: NULL pointer");
  if (max_row_items < 0 || max_combine_rows < 0 || max_partials < 0 || max_row_vecs < 1 ||
      max_row_vecs > kMaxRowVecs)
    return fail(EDGERAG_EINVAL,
                "edgerag_paged_attention_fixed: capacities (items %d, combine rows %d, row "
                "vectors %d, partials %lld) out of range",
                max_row_items, max_combine_rows, max_row_vecs, (long long)max_partials);
  if (n_q_heads <= 0 || n_kv_heads <= 0 || n_q_heads % n_kv_heads != 0 ||
      !head_dim_supported(head_dim) || block_size <= 0 || num_blocks <= 0)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention_fixed: bad shape");
  if (row_waves < 0 || row_waves > kMaxRowWaves ||
      (row_waves > 0 && (head_dim > 128 || elem_size(dtype) == 0 ||
                         head_dim % (16 / elem_size(dtype)) != 0 ||
                         block_size % (kWave / (head_dim / (16 / elem_size(dtype)))) != 0)))
    return fail(EDGERAG_EINVAL,
                "edgerag_paged_attention_fixed: row_waves %d (1..%d workgroup-split rows need "
                "head_dim <= 128 and the fast decode kernel's block sizes)",
                row_waves, kMaxRowWaves);
  if (slots < 0 || slots > kMaxPartSlots || (slots > 0 && row_waves == 0) ||
      (slots > 0 && max_partials < int64_t(max_combine_rows) * n_q_heads * slots))
    return fail(EDGERAG_EINVAL,
                "edgerag_paged_attention_fixed: slots %d (0, or 1..%d with row_waves > 0 and "
                "partials for every slot of %d rows x %d heads)",
                slots, kMaxPartSlots, max_combine_rows, n_q_heads);
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention_fixed: scale must be positive");
  const int es = elem_size(dtype);
  if (es == 0) return fail(EDGERAG_EINVAL, "edgerag_paged_attention_fixed: dtype %d", dtype);
  if (!aligned16(key_pool) || !aligned16(value_pool) || !aligned16(q) ||
      (q_stride_tok * es) % 16 != 0 || (q_stride_head * es) % 16 != 0)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention_fixed: q and pools must be 16-byte aligned");
  const WorkspaceLayout ws = workspace_layout(max_partials, head_dim);
  const int64_t need = ws.total;
  if (workspace_bytes < need || (need > 0 && workspace == nullptr))
    return fail(EDGERAG_EWORKSPACE, "edgerag_paged_attention_fixed: workspace %lld bytes, need %lld",
                (long long)workspace_bytes, (long long)need);
  Launch a{};
  a.s = static_cast<hipStream_t>(stream);
  a.q = q;
  a.q_st = q_stride_tok;
  a.q_sh = q_stride_head;
  a.kp = key_pool;
  a.vp = value_pool;
  a.bt = block_tables;
  a.bt_stride = block_tables_stride;
  a.qsl = query_start_loc;
  a.ctx = context_lens;
  a.plan = plan_dev;
  a.hq = n_q_heads;
  a.hkv = n_kv_heads;
  a.nb = num_blocks;
  a.bs = block_size;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.out = out;
  a.o_st = out_stride_tok;
  a.o_sh = out_stride_head;
  char* wsp = static_cast<char*>(workspace);
  a.ml = reinterpret_cast<float2*>(wsp);
  a.pacc = reinterpret_cast<float*>(wsp + ws.acc_off);
  const int qr = std::min(8, pow2_at_least(max_row_vecs));
  int rc = EDGERAG_OK;
  if (max_row_items > 0) {
    switch (dtype) {
      case EDGERAG_F32: rc = run_fixed_dtype<float>(a, head_dim, qr, max_row_items, row_waves);
        break;
      case EDGERAG_F16: rc = run_fixed_dtype<f16>(a, head_dim, qr, max_row_items, row_waves);
        break;
      case EDGERAG_BF16: rc = run_fixed_dtype<bf16>(a, head_dim, qr, max_row_items, row_waves);
        break;
    }
  }
  if (rc != EDGERAG_OK || max_combine_rows == 0) return rc;
  // No host plan here: the kernel reads the list's length (and offset) from the device header.
  switch (dtype) {
#define EDGERAG_COMBINE_FIXED(TYPE)                                                               \
  rc = launch_combine<TYPE>(a.s, plan_dev, -1, max_combine_rows, -1, slots, n_q_heads, head_dim, \
                            a.ml, a.pacc, out, out_stride_tok, out_stride_head)
    case EDGERAG_F32: EDGERAG_COMBINE_FIXED(float); break;
    case EDGERAG_F16: EDGERAG_COMBINE_FIXED(f16); break;
    case EDGERAG_BF16: EDGERAG_COMBINE_FIXED(bf16); break;
#undef EDGERAG_COMBINE_FIXED
  }
  if (rc != EDGERAG_OK) return rc;
  return check_launch("edgerag_paged_attention_fixed(combine)");
}

// ---- edgerag_paged_attention_noalloc: split partials in a static device array -----------------
//
// The partials live in `scratch`, a file-scope device array (one copy per GPU, held until the
// process ends). On the host the array's name is only a registration handle, never a device
// address: its address on a device comes from hipGetSymbolAddress, looked up the first time the
// entry point runs on that device (with the device current) and cached per device. Kernels get
// that address as their workspace argument, exactly as they get a caller's workspace.
namespace edgerag {
namespace {

static __device__ __align__(256) char scratch[EDGERAG_ATTN_SCRATCH_BYTES];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxScratchDevices] = {};

// The device address of `scratch` on the current device, which must be the stream's device.
int scratch_address(hipStream_t stream, void** addr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(EDGERAG_EHIP, "edgerag_paged_attention_noalloc: hipGetDevice: %s",
                hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(EDGERAG_EUNSUPPORTED, "edgerag_paged_attention_noalloc: device %d", dev);
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess)
      return fail(EDGERAG_EHIP, "edgerag_paged_attention_noalloc: hipStreamGetDevice: %s",
                  hipGetErrorString(e));
    if (sdev != dev)
      return fail(EDGERAG_EINVAL,
                  "edgerag_paged_attention_noalloc: the stream belongs to device %d, device %d is "
                  "current (make the stream's device current)",
                  int(sdev), dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(EDGERAG_EHIP,
                  "edgerag_paged_attention_noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                  dev, hipGetErrorString(e));
    g_scratch_addr[dev] = p;
  }
  *addr = g_scratch_addr[dev];
  return EDGERAG_OK;
}

}  // namespace
}  // namespace edgerag

extern "C" int edgerag_paged_attention_noalloc(
    const int32_t* plan_host, const int32_t* plan_dev, int64_t plan_words, const void* q,
    int64_t q_stride_tok, int64_t q_stride_head, const void* key_pool, const void* value_pool,
    int32_t dtype, const int32_t* block_tables, int64_t block_tables_stride,
    const int32_t* query_start_loc, const int32_t* context_lens, int32_t num_reqs,
    int32_t num_tokens, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
    int32_t block_size, int32_t num_blocks, float scale, void* out, int64_t out_stride_tok,
    int64_t out_stride_head, int32_t parts, void* stream) {
  clear_error();
  // Size check first, on the host: a plan whose partials do not fit is refused before any HIP call.
  if (plan_host == nullptr || plan_words < kHeaderWords || plan_host[H_MAGIC] != kPlanMagic ||
      plan_host[H_VERSION] != kPlanVersion)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention_noalloc: not a plan from edgerag_attn_plan");
  if (!head_dim_supported(head_dim) || plan_host[H_HEAD_DIM] != head_dim)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention_noalloc: plan was made for a different shape");
  const int64_t need = workspace_layout(plan_host[H_N_PARTIALS], head_dim).total;
  if (need > EDGERAG_ATTN_SCRATCH_BYTES)
    return fail(EDGERAG_EWORKSPACE,
                "edgerag_paged_attention_noalloc: the plan's split partials need %lld bytes, the "
                "static scratch holds %lld (use edgerag_paged_attention with a workspace)",
                (long long)need, (long long)EDGERAG_ATTN_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = scratch_address(static_cast<hipStream_t>(stream), &ws)) return rc;
  }
  return paged_attention_impl(plan_host, plan_dev, plan_words, q, q_stride_tok, q_stride_head,
                              key_pool, value_pool, dtype, block_tables, block_tables_stride,
                              query_start_loc, context_lens, num_reqs, num_tokens, n_q_heads,
                              n_kv_heads, head_dim, block_size, num_blocks, scale, out,
                              out_stride_tok, out_stride_head, ws, need, parts, stream, nullptr);
}
