// Chunked-prefill attention tiles on CDNA4 matrix cores (fp16, head_dim 64).
//
// A work item is (request, kv head, query tile of up to kMfmaTileRows virtual rows, KV split).
// Virtual row rho is query token qb + rho / n_rep of query head h * n_rep + rho % n_rep, so all
// heads of a GQA group share every K/V tile. Each wave owns 32 rows.
//
// Per 64-key tile:
//   * the workgroup stages K row-major and V transposed (V^T[dim][key]) into one of two LDS
//     buffers straight from the paged pool with raw buffer loads: keys without a valid block get
//     an out-of-range offset and load zeros, no branch. A tile's loads are issued two tiles
//     before it is staged, so HBM/L2 latency overlaps two tiles of matrix work; one barrier per
//     tile. LDS rows are 128 bytes with the 16-byte chunk index XOR-swizzled by the row, so the
//     MFMA operand reads and the staging writes are bank-conflict free.
//   * each wave computes S^T = K Q^T with v_mfma_f32_32x32x16_f16: A = 32 keys x 16 dims from
//     LDS, B = Q^T from registers (loaded once per item): per lane, 16 keys of one query.
//   * online softmax in the log2 domain: Q is scaled by softmax_scale * log2(e) once per item
//     (rounded to fp16, as torch's SDPA scales q before the product), and the S accumulators start
//     at -m, so the MFMA leaves s - m and every probability is one v_exp_f32 with no FMA. The max
//     m is only raised when a score beats it by 2^8 (lazy rescale; p <= 256 stays exact in fp16).
//     Masks (causal k <= L - c + i, split end, invalid blocks) are applied only on tiles that need
//     them.
//   * O^T += V^T P^T with the same MFMA: the probabilities, packed to fp16, are already in the
//     B-operand layout once the contraction index is permuted; V^T is stored in that permuted key
//     order, so each A operand is one 16-byte LDS read. l accumulates the same fp16 p (v_dot2).
// The output is O / l (fp16) or, for split items, fp32 partials merged by attn_combine_kernel.
#include "attention_plan.h"

namespace edgerag {
namespace {

using namespace plan;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kD = 64;
#ifndef EDGERAG_ATTN_SHARED_PAD_KB
#define EDGERAG_ATTN_SHARED_PAD_KB 48  // dynamic LDS of a shared-mode tile workgroup
#endif
#ifndef EDGERAG_ATTN_SHARED_TILES_PER_CU
#define EDGERAG_ATTN_SHARED_TILES_PER_CU 1  // tile workgroups per CU that the pad allows
#endif
#ifndef EDGERAG_TILE_PRIO
// Issue priority (s_setprio) of the tile waves. Beside the decode rows (shared mode) the VALU-
// bound tiles then win the SIMDs' issue slots and the memory-bound row waves fill the gaps:
// config 3 227-229 -> 220-221 us (priority 1: 221-224, 3: 221-223; two tile workgroups per CU
// instead of one, at priority 2: 253 us).
#define EDGERAG_TILE_PRIO 2
#endif
constexpr unsigned kSharedLdsPad = EDGERAG_ATTN_SHARED_PAD_KB * 1024;
constexpr int kKeys = 64;            // keys per LDS tile
constexpr int kRow = 64;             // halves per LDS row (K: one key; V^T: one dim)
constexpr float kRescaleLog2 = 8.f;  // lazy rescale: p may grow to 2^8 before the max moves
constexpr int kWaves = kMfmaTileRows / 32;
constexpr int kThreads = kWaves * kWave;
constexpr int kKChunks = kKeys * kD * 2 / 16;  // 16-byte chunks of a K tile (512)
constexpr int kKPerThread = kKChunks / kThreads;
#ifndef EDGERAG_TILE_VKEYS
// Consecutive keys of one dim chunk a thread stages into V^T (2 or 4). With 2, the 256 (key pair,
// dim chunk) units of a V tile give every thread of a 4-wave workgroup one, so no wave carries
// the whole transpose (with 4 half the threads staged V and the other half waited at the barrier).
#define EDGERAG_TILE_VKEYS 2
#endif
constexpr int kVKeys = EDGERAG_TILE_VKEYS;
static_assert(kVKeys == 2 || kVKeys == 4, "V^T staging units of 2 or 4 keys");
constexpr int kVGroups = kKeys / kVKeys;             // key groups of a V tile
constexpr int kVPairs = kVGroups * (kD / 8);         // (key group, dim chunk) units of a V tile
constexpr int kVPerThread = (kVPairs + kThreads - 1) / kThreads;
static_assert(kKChunks % kThreads == 0, "K staging split");
constexpr unsigned kStaticLds = 2 * kKeys * kRow * 2 + 2 * kD * kRow * 2 + kMaxTileBlocks * 4;
constexpr unsigned kSharedTiles = EDGERAG_ATTN_SHARED_TILES_PER_CU;
static_assert((kSharedTiles + 1) * (kStaticLds + kSharedLdsPad) > 160 * 1024 &&
                  kSharedTiles * (kStaticLds + kSharedLdsPad) <= 160 * 1024,
              "shared mode: the pad must leave room for exactly kSharedTiles tile workgroups per CU");

// Byte offset handed to buffer loads for keys with no valid block: beyond num_records, so the
// load returns zeros without a branch (the launcher keeps a head's pool slice below it).
constexpr uint32_t kOutOfRange = 0xFFFFFFF0u;

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// max / sum of v and its value in lane (lane ^ 32) in every lane: v_permlane32_swap exchanges
// the wave's halves in a VALU op, where a shuffle goes through LDS (ds_bpermute, a round trip).
// The swap leaves lane i with (v[i], v[i + 32]) and lane i + 32 with (v[i], v[i + 32]).
__device__ __forceinline__ float halves_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float halves_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ f32x16 mfma32(h8 a, h8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ h8 buffer_load16(__amdgpu_buffer_rsrc_t rsrc, uint32_t byte_off) {
  return __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rsrc, byte_off, 0, 0));
}

// Halves offset of 16-byte chunk `chunk` (0..7) of LDS row `row`, chunk index XOR-swizzled.
__device__ __forceinline__ int lds_chunk(int row, int chunk) {
  return row * kRow + ((chunk ^ (row & 7)) << 3);
}

// V^T keeps keys in the order the P.V k-steps consume them: within every 16 keys, bits 2 and 3
// of the key index are swapped, so lane group g's keys {0-3, 8-11} + 4g of a k-step are one
// contiguous 16-byte run.
__device__ __forceinline__ int vt_slot(int key) {
  return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}

struct StageRegs {
  h8 k[kKPerThread];
  h8 v[kVKeys * kVPerThread];
};

struct Geometry {
  int kb, ke, blk0, bs_shift, bs_mask;
};

// Block id of key position pos (-1 past the split or for an invalid table entry).
__device__ __forceinline__ int block_of(const Geometry& geo, const int* __restrict__ sblk,
                                        int pos) {
  const int i = (pos >> geo.bs_shift) - geo.blk0;
  return (pos < geo.ke && i < kMaxTileBlocks) ? sblk[i] : -1;
}

// Byte offset of (pos, 16-byte dim chunk dc) in one kv head's pool slice, or kOutOfRange.
__device__ __forceinline__ uint32_t pool_offset(const Geometry& geo, int blk, int pos, int dc) {
  return blk >= 0 ? ((uint32_t(blk) << geo.bs_shift) + uint32_t(pos & geo.bs_mask)) *
                            uint32_t(kD * 2) + uint32_t(16 * dc)
                  : kOutOfRange;
}

// The block ids one thread's staging loads of a 64-key tile need, looked up in LDS a tile before
// the loads are issued (so issuing them waits on no LDS round trip).
struct StageIds {
  int k[kKPerThread];
  int v[kVPerThread];
};

// K: chunk c = tid + kThreads * j is key c / 8, dim chunk c % 8 (8 lanes fill one key row).
// V: unit p = tid + kThreads * j is key group p % kVGroups (kVKeys keys), dim chunk p / kVGroups
// (kVGroups lanes fill one V^T row).
__device__ __forceinline__ void stage_ids(StageIds& ids, int tid, int k0, const Geometry& geo,
                                          const int* __restrict__ sblk) {
#pragma unroll
  for (int j = 0; j < kKPerThread; ++j) ids.k[j] = block_of(geo, sblk, k0 + (tid + kThreads * j) / 8);
#pragma unroll
  for (int j = 0; j < kVPerThread; ++j) {
    const int p = tid + kThreads * j;
    ids.v[j] = (kVPairs % kThreads != 0 && p >= kVPairs)
                   ? -1
                   : block_of(geo, sblk, k0 + kVKeys * (p % kVGroups));
  }
}

__device__ __forceinline__ void stage_load(StageRegs& st, const StageIds& ids, int tid, int k0,
                                           const Geometry& geo, __amdgpu_buffer_rsrc_t krs,
                                           __amdgpu_buffer_rsrc_t vrs) {
#pragma unroll
  for (int j = 0; j < kKPerThread; ++j) {
    const int c = tid + kThreads * j;
    st.k[j] = buffer_load16(krs, pool_offset(geo, ids.k[j], k0 + c / 8, c % 8));
  }
#pragma unroll
  for (int j = 0; j < kVPerThread; ++j) {
    const int p = tid + kThreads * j;
    if (kVPairs % kThreads != 0 && p >= kVPairs) break;
    const int a = p % kVGroups, b = p / kVGroups;
    // The keys of a group share one block (blocks hold a multiple of 4 keys): one lookup, then
    // consecutive rows; keys past the split still get the out-of-range offset.
    const int pos = k0 + kVKeys * a;
    const uint32_t base = pool_offset(geo, ids.v[j], pos, b);
#pragma unroll
    for (int kk = 0; kk < kVKeys; ++kk)
      st.v[kVKeys * j + kk] = buffer_load16(
          vrs, (base != kOutOfRange && pos + kk < geo.ke) ? base + uint32_t(kk * kD * 2)
                                                          : kOutOfRange);
  }
}

__device__ __forceinline__ void stage_store(const StageRegs& st, int tid,
                                            _Float16* __restrict__ sk, _Float16* __restrict__ svt) {
#pragma unroll
  for (int j = 0; j < kKPerThread; ++j) {
    const int c = tid + kThreads * j;
    *reinterpret_cast<h8*>(sk + lds_chunk(c / 8, c % 8)) = st.k[j];
  }
#pragma unroll
  for (int j = 0; j < kVPerThread; ++j) {
    const int p = tid + kThreads * j;
    if (kVPairs % kThreads != 0 && p >= kVPairs) break;
    const int a = p % kVGroups, b = p / kVGroups;
    const int slot = vt_slot(kVKeys * a);  // kVKeys-aligned: the group's keys stay contiguous
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      _Float16* dst = svt + lds_chunk(8 * b + d, slot >> 3) + (slot & 7);
      if constexpr (kVKeys == 4) {
        *reinterpret_cast<h4*>(dst) = h4{st.v[4 * j][d], st.v[4 * j + 1][d], st.v[4 * j + 2][d],
                                         st.v[4 * j + 3][d]};
      } else {
        *reinterpret_cast<h2*>(dst) = h2{st.v[2 * j][d], st.v[2 * j + 1][d]};
      }
    }
  }
}

// Two waves per SIMD: the register budget (256 per lane) keeps S, O and the staged tile in VGPRs.
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn_prefill_mfma_kernel(
    const int32_t* __restrict__ plan, int32_t item_base, int32_t bs_shift,
    const int32_t* __restrict__ qsl, const int32_t* __restrict__ ctx,
    const int32_t* __restrict__ block_tables, int64_t bt_stride, int32_t num_blocks,
    int32_t n_q_heads, const _Float16* __restrict__ q, int64_t q_st, int64_t q_sh,
    const _Float16* __restrict__ kpool, const _Float16* __restrict__ vpool, int32_t n_kv_heads,
    float scale_log2, _Float16* __restrict__ out,
    int64_t o_st, int64_t o_sh, float2* __restrict__ part_ml, float* __restrict__ part_acc) {
  __shared__ __align__(16) _Float16 sk[2][kKeys * kRow];
  __shared__ __align__(16) _Float16 svt[2][kD * kRow];
  __shared__ int sblk[kMaxTileBlocks];

  if (EDGERAG_TILE_PRIO > 0) __builtin_amdgcn_s_setprio(EDGERAG_TILE_PRIO);
  const int32_t* it = plan + plan[H_ITEM_OFF] + int64_t(item_base + blockIdx.x) * kItemWords;
  const int r = it[I_REQ], h = it[I_HEAD], qb = it[I_QBEGIN], qc = it[I_QCOUNT];
  const int kb = it[I_KVBEGIN], ke = it[I_KVEND], split = it[I_SPLIT];
  const int32_t* rq = plan + plan[H_REQ_OFF] + r * kReqWords;
  const int nsplit = rq[R_NSPLIT], part_off = rq[R_PARTOFF], pstride = rq[R_PSTRIDE];
  const int q0 = qsl[r], c = qsl[r + 1] - q0, L = ctx[r];
  const int n_rep = n_q_heads / n_kv_heads;
  const int32_t* table = block_tables + int64_t(r) * bt_stride;
  const int64_t head_base = int64_t(h) * num_blocks;
  const int block_size = 1 << bs_shift;

  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int g = lane / 32, col = lane % 32;
  const int nrows = qc * n_rep;
  const int rho = wave * 32 + col;
  const bool active = rho < nrows;
  const int t = qb + (active ? rho / n_rep : 0);
  const int hq = h * n_rep + (active ? rho % n_rep : 0);
  const int lim = active ? L - c + (t - q0) : -1;  // last visible key position of this row
  const bool wave_live = wave * 32 < nrows;
  // Smallest causal limit among the wave's rows: tiles ending at or below it need no mask.
  const int first_row = min(wave * 32, nrows - 1);
  const int wave_min_lim = L - c + (qb + first_row / n_rep - q0);

  Geometry geo;
  geo.kb = kb;
  geo.ke = ke;
  geo.blk0 = kb >> bs_shift;
  geo.bs_shift = bs_shift;
  geo.bs_mask = block_size - 1;
  // Block ids of the whole split, once (the planner caps a split at kMaxTileBlocks blocks).
  // Whether any of them is invalid (never in a well-formed table) decides once per item whether
  // tiles check for invalid keys.
  int any_bad = 0;
  {
    const int nblk = min(((ke - 1) >> bs_shift) - geo.blk0 + 1, kMaxTileBlocks);
    for (int i = tid; i < nblk; i += kThreads) {
      const int32_t b = table[geo.blk0 + i];
      const bool ok = b >= 0 && b < num_blocks;
      sblk[i] = ok ? b : -1;
      any_bad |= ok ? 0 : 1;
    }
  }
  const bool item_has_bad = __syncthreads_or(any_bad) != 0;

  // Q^T as the B operand: k-step ks covers dims 16*ks + 8*g .. +7 of this lane's query, as
  // given. The scale (times log2 e) multiplies the fp32 dot products afterwards, like the decode
  // rows: scaling q first would round every q * scale to fp16, a score error that grows with the
  // score (scores of tens of nats, as with attention sinks, moved outputs by 3e-2).
  h8 qop[4];
  {
    const _Float16* qp = q + int64_t(t) * q_st + int64_t(hq) * q_sh;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      qop[ks] = active ? *reinterpret_cast<const h8*>(qp + 16 * ks + 8 * g) : h8{};
  }
  f32x16 o0 = {}, o1 = {};  // O^T dims 0-31 and 32-63 of this lane's query
  float m = -INFINITY;      // reference max of the log2-domain scores
  float l = 0.f;
  float nm = 0.f;           // -m (0 while m is -inf)
  const f32x16 zero16 = {};
  const h2 ones = {_Float16(1.f), _Float16(1.f)};

  const uint32_t head_bytes = uint32_t(int64_t(num_blocks) * block_size * kD * 2);
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<_Float16*>(kpool + head_base * block_size * kD), 0, head_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<_Float16*>(vpool + head_base * block_size * kD), 0, head_bytes, 0x00020000);

  // One 64-key tile on staged LDS buffers (skb, svb).
  auto tile = [&](int k0, const _Float16* skb, const _Float16* svb) {
    // S^T = K Q^T: two 32-key tiles, 4 k-steps of 16 dims (dim chunk 2ks + g).
    f32x16 s[2];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const h8 ka = *reinterpret_cast<const h8*>(skb + lds_chunk(32 * kt + col, 2 * ks + g));
        s[kt] = mfma32(ka, qop[ks], ks == 0 ? zero16 : s[kt]);
      }
    }
    // log2-domain scores relative to the reference max: q.k * scale * log2(e) - m.
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[kt][i] = __builtin_fmaf(s[kt][i], scale_log2, nm);
    // Register i of tile kt holds key 32kt + (i%4) + 8(i/4) + 4g.
    const int key_end = min(ke - k0, kKeys);  // keys of this tile inside the split
    if (k0 + kKeys - 1 > wave_min_lim || key_end < kKeys) {
      const int vis_end = min(key_end, lim - k0 + 1);  // keys [0, vis_end) are visible
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (32 * kt + (i & 3) + 8 * (i >> 2) + 4 * g >= vis_end) s[kt][i] = -INFINITY;
    }
    // Keys whose block id is invalid (never in a well-formed table): masked too.
    uint64_t bad = 0;
    if (item_has_bad) {
      const int bi =
          min(((k0 + min(lane, key_end - 1)) >> bs_shift) - geo.blk0, kMaxTileBlocks - 1);
      bad = __ballot(lane < key_end && sblk[bi] < 0);
    }
    if (bad != 0) {
      // Lane group g's keys of tile kt are bits (i%4) + 8(i/4) of (bad_kt >> 4g).
      const uint32_t b0 = uint32_t(bad) >> (4 * g), b1 = uint32_t(bad >> 32) >> (4 * g);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int bit = (i & 3) + 8 * (i >> 2);
        if ((b0 >> bit) & 1u) s[0][i] = -INFINITY;
        if ((b1 >> bit) & 1u) s[1][i] = -INFINITY;
      }
    }
    float tmax = s[0][0];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 16; ++i) tmax = fmaxf(tmax, s[kt][i]);
    tmax = halves_max(tmax);  // the other 16 keys of each 32-key tile
    // Lazy rescale: the reference max m only moves when a score beats it by 2^kRescaleLog2 (the
    // scores are s - m here; before the first visible score, m is -inf and s is absolute).
    const bool first = m == -INFINITY;
    const bool up = first ? tmax != -INFINITY : tmax > kRescaleLog2;
    if (__any(up)) {
      const float shift = up ? tmax : 0.f;
      const float alpha = first ? (up ? 0.f : 1.f) : exp2_fast(-shift);
      if (up) m = first ? tmax : m + tmax;
      nm = m == -INFINITY ? 0.f : -m;
      l *= alpha;
      o0 *= alpha;
      o1 *= alpha;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        s[0][i] -= shift;
        s[1][i] -= shift;
      }
    }

    // P = exp2(s - m), packed to fp16 in the B-operand order of each k-step.
    float lsum = 0.f;
#pragma unroll
    for (int st4 = 0; st4 < 4; ++st4) {
      const int kt = st4 >> 1, half = st4 & 1;
      h8 pb;
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        const float p0 = exp2_fast(s[kt][8 * half + j]);
        const float p1 = exp2_fast(s[kt][8 * half + j + 1]);
        const h2 pp = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(p0, p1));
        pb[j] = pp[0];
        pb[j + 1] = pp[1];
        lsum = __builtin_amdgcn_fdot2(pp, ones, lsum, false);
      }
      const int vchunk = 4 * kt + 2 * half + g;  // permuted V^T slots of this k-step
      o0 = mfma32(*reinterpret_cast<const h8*>(svb + lds_chunk(col, vchunk)), pb, o0);
      o1 = mfma32(*reinterpret_cast<const h8*>(svb + lds_chunk(32 + col, vchunk)), pb, o1);
    }
    l += lsum;  // this half's keys only: the halves are added once, after the last tile
  };

  // Register stages st0 / st1 alternate, so a tile's loads are issued two tiles before it is
  // staged to LDS and have two tiles of matrix work to land. Loads past the split need no branch:
  // their positions get out-of-range offsets and load zeros. One barrier per tile: it orders the
  // tile's LDS writes before its reads, and every wave's reads of a buffer before its rewrite.
  // The block ids of each stage's next loads are read from LDS one tile ahead (id0 / id1).
  StageRegs st0, st1;
  StageIds id0, id1;
  stage_ids(id0, tid, kb, geo, sblk);
  stage_ids(id1, tid, kb + kKeys, geo, sblk);
  stage_load(st0, id0, tid, kb, geo, krs, vrs);
  stage_load(st1, id1, tid, kb + kKeys, geo, krs, vrs);
  stage_ids(id0, tid, kb + 2 * kKeys, geo, sblk);
  stage_ids(id1, tid, kb + 3 * kKeys, geo, sblk);
  for (int k0 = kb; k0 < ke; k0 += 2 * kKeys) {
    stage_store(st0, tid, sk[0], svt[0]);
    __syncthreads();
    stage_load(st0, id0, tid, k0 + 2 * kKeys, geo, krs, vrs);
    stage_ids(id0, tid, k0 + 4 * kKeys, geo, sblk);
    if (wave_live) tile(k0, sk[0], svt[0]);
    if (k0 + kKeys < ke) {
      stage_store(st1, tid, sk[1], svt[1]);
      __syncthreads();
      stage_load(st1, id1, tid, k0 + 3 * kKeys, geo, krs, vrs);
      stage_ids(id1, tid, k0 + 5 * kKeys, geo, sblk);
      if (wave_live) tile(k0 + kKeys, sk[1], svt[1]);
    }
  }
  l = halves_sum(l);

  if (!active) return;
  // O^T register i of dim tile dt holds dim 32dt + (i%4) + 8(i/4) + 4g of this lane's query.
  if (nsplit == 1) {
    const float inv = 1.f / fmaxf(l, 1.17549435e-38f);
    _Float16* op = out + int64_t(t) * o_st + int64_t(hq) * o_sh;
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const int d0 = 8 * qd + 4 * g;
      *reinterpret_cast<h4*>(op + d0) =
          h4{_Float16(o0[4 * qd] * inv), _Float16(o0[4 * qd + 1] * inv),
             _Float16(o0[4 * qd + 2] * inv), _Float16(o0[4 * qd + 3] * inv)};
      *reinterpret_cast<h4*>(op + 32 + d0) =
          h4{_Float16(o1[4 * qd] * inv), _Float16(o1[4 * qd + 1] * inv),
             _Float16(o1[4 * qd + 2] * inv), _Float16(o1[4 * qd + 3] * inv)};
    }
  } else {
    // Partials carry the max in the log2 domain, like the decode kernels'.
    const int64_t idx = int64_t(part_off) + (int64_t(t - q0) * n_q_heads + hq) * pstride + split;
    if (g == 0) part_ml[idx] = make_float2(m, l);
    float* pa = part_acc + idx * kD;
#pragma unroll
    for (int qd = 0; qd < 4; ++qd) {
      const int d0 = 8 * qd + 4 * g;
      *reinterpret_cast<float4*>(pa + d0) =
          make_float4(o0[4 * qd], o0[4 * qd + 1], o0[4 * qd + 2], o0[4 * qd + 3]);
      *reinterpret_cast<float4*>(pa + 32 + d0) =
          make_float4(o1[4 * qd], o1[4 * qd + 1], o1[4 * qd + 2], o1[4 * qd + 3]);
    }
  }
}

}  // namespace

bool prefill_tiles_supported(int32_t num_blocks, int32_t block_size) {
  // Power-of-two blocks of at least 4 keys (shift addressing; a V key quad never straddles a
  // block), and one kv head's slice of a pool must fit a buffer resource, below kOutOfRange.
  return log2_exact(block_size) >= 2 &&
         int64_t(num_blocks) * block_size * kD * 2 < int64_t(kOutOfRange);
}

void launch_prefill_tiles_f16_d64(const AttnLaunch& a, int item_base, int count, bool shared) {
  // Shared mode reserves unused dynamic LDS so that a second workgroup no longer fits a CU's
  // 160 KiB (the static arrays take ~34 KiB): the tiles then hold one of each SIMD's two register
  // halves and decode waves keep the other.
  const unsigned pad = shared ? kSharedLdsPad : 0;
  hipLaunchKernelGGL(attn_prefill_mfma_kernel, dim3(count), dim3(kThreads), pad, a.s, a.plan,
                     item_base, log2_exact(a.bs), a.qsl, a.ctx, a.bt, a.bt_stride, a.nb, a.hq,
                     static_cast<const _Float16*>(a.q), a.q_st, a.q_sh,
                     static_cast<const _Float16*>(a.kp), static_cast<const _Float16*>(a.vp),
                     a.hkv, a.scale_log2, static_cast<_Float16*>(a.out), a.o_st,
                     a.o_sh, a.ml, a.pacc);
}

}  // namespace edgerag
