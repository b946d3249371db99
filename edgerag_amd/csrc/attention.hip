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
//   1. edgerag_attn_plan (host) cuts every (request, kv head) into KV splits and query tiles and
//      writes a flat work list, heaviest items first. Long contexts are split so that a 32-way
//      decode batch still yields thousands of independent waves for the 256 CUs.
//   2. attn_rows_kernel: one wavefront per work item. The wave walks its KV split in steps of
//      64 lanes x 16 bytes (fully coalesced 1 KiB loads straight out of the 2 KiB block rows),
//      keeps the fp32 online-softmax state (m, l, acc) of up to kQR query vectors in registers,
//      and reduces scores with cross-lane butterflies -- no LDS, no gather copy. All n_rep query
//      heads of a GQA group share each K/V load.
//   3. attn_combine_kernel merges the fp32 split partials (m, l, acc) of requests that were
//      split; unsplit requests are written directly by step 2.
// Scores are kept in the log2 domain (q pre-multiplied by scale * log2(e)) so every exponential
// is a single v_exp_f32.
#include <algorithm>
#include <cmath>
#include <numeric>
#include <vector>

#include "common.h"

namespace edgerag {
namespace {

// ---- plan layout (int32 words) -----------------------------------------------------------------
constexpr int32_t kPlanMagic = 0x47415245;  // "ERAG"
constexpr int32_t kPlanVersion = 1;
constexpr int kHeaderWords = 16;
constexpr int kItemWords = 8;
constexpr int kReqWords = 4;

enum Header {
  H_MAGIC = 0,
  H_VERSION,
  H_N_ITEMS,
  H_N_REQS,
  H_ITEM_OFF,
  H_REQ_OFF,
  H_N_PARTIALS,
  H_N_Q_HEADS,
  H_N_KV_HEADS,
  H_HEAD_DIM,
  H_BLOCK_SIZE,
  H_DTYPE,
  H_NUM_TOKENS_HINT,
};
enum Item { I_REQ = 0, I_HEAD, I_QBEGIN, I_QCOUNT, I_KVBEGIN, I_KVEND, I_SPLIT, I_KIND };
enum Req { R_NSPLIT = 0, R_SPLITLEN, R_PARTOFF, R_PAD };

constexpr int kQR = 4;          // query vectors carried per pass of a wave
constexpr int kQTile = 16;      // query rows per work item on the row path
constexpr int kMinSplit = 256;  // tokens: below this a split's partial write is not worth it
constexpr int kTargetItems = 8192;

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

template <typename T, int D>
struct RowCfg {
  static constexpr int VEC = 16 / sizeof(T);
  static constexpr int LPT = D / VEC;  // lanes sharing one token
  static constexpr int TPW = kWave / LPT;  // tokens per wave step
  static constexpr int LOG_LPT = ilog2(LPT);
  static_assert(D % VEC == 0 && LPT >= 1 && LPT <= kWave, "unsupported head_dim");
};

template <typename T, int D>
__global__ __launch_bounds__(kWave) void attn_rows_kernel(
    const T* __restrict__ q, int64_t q_st, int64_t q_sh, const T* __restrict__ kpool,
    const T* __restrict__ vpool, const int32_t* __restrict__ block_tables, int64_t bt_stride,
    const int32_t* __restrict__ qsl, const int32_t* __restrict__ ctx,
    const int32_t* __restrict__ plan, int32_t n_q_heads, int32_t n_kv_heads, int32_t num_blocks,
    int32_t block_size, float scale_log2, T* __restrict__ out, int64_t o_st, int64_t o_sh,
    float2* __restrict__ part_ml, float* __restrict__ part_acc) {
  using C = RowCfg<T, D>;
  constexpr int VEC = C::VEC, LPT = C::LPT, TPW = C::TPW, LOG_LPT = C::LOG_LPT;

  const int32_t* it = plan + plan[H_ITEM_OFF] + int64_t(blockIdx.x) * kItemWords;
  const int r = it[I_REQ], h = it[I_HEAD], qb = it[I_QBEGIN], qc = it[I_QCOUNT];
  const int kb = it[I_KVBEGIN], ke = it[I_KVEND], split = it[I_SPLIT];
  const int32_t* rq = plan + plan[H_REQ_OFF] + r * kReqWords;
  const int nsplit = rq[R_NSPLIT], part_off = rq[R_PARTOFF];
  const int q0 = qsl[r], c = qsl[r + 1] - q0, L = ctx[r];
  const int n_rep = n_q_heads / n_kv_heads;

  const int lane = threadIdx.x;
  const int sub = lane & (LPT - 1);
  const int tslot = lane >> LOG_LPT;
  const int32_t* table = block_tables + int64_t(r) * bt_stride;
  const int64_t head_base = int64_t(h) * num_blocks;

  const int nvec = qc * n_rep;
  for (int v0 = 0; v0 < nvec; v0 += kQR) {
    float qv[kQR][VEC];
    float m[kQR], l[kQR], acc[kQR][VEC];
    int lim[kQR];
#pragma unroll
    for (int j = 0; j < kQR; ++j) {
      const int v = v0 + j;
      const int row = v / n_rep;
      const int hq = h * n_rep + (v % n_rep);
      const int t = qb + row;
      lim[j] = v < nvec ? L - c + (t - q0) : -1;  // -1: inactive slot, sees nothing
      if (v < nvec) {
        const T* qp = q + int64_t(t) * q_st + int64_t(hq) * q_sh + sub * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) qv[j][e] = to_f32<T>(qp[e]) * scale_log2;
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) qv[j][e] = 0.f;
      }
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
      float kf[VEC], vf[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        kf[e] = vec_elem<T>(kr, e);
        vf[e] = vec_elem<T>(vr, e);
      }
#pragma unroll
      for (int j = 0; j < kQR; ++j) {
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) s = fmaf(qv[j][e], kf[e], s);
        s = xor_sum<0, LOG_LPT>(s);
        const bool vis = valid && tok <= lim[j];
        s = vis ? s : -INFINITY;
        const float gmax = xor_max<LOG_LPT, 6>(s);
        if (gmax == -INFINITY) continue;  // wave-uniform: nothing visible in this step
        if (gmax > m[j]) {
          const float alpha = exp2_fast(m[j] - gmax);  // m == -inf gives exactly 0
          l[j] *= alpha;
#pragma unroll
          for (int e = 0; e < VEC; ++e) acc[j][e] *= alpha;
          m[j] = gmax;
        }
        const float p = vis ? exp2_fast(s - m[j]) : 0.f;
        l[j] += p;
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[j][e] = fmaf(p, vf[e], acc[j][e]);
      }
    }

#pragma unroll
    for (int j = 0; j < kQR; ++j) {
      const int v = v0 + j;
      if (v >= nvec) break;
      const float lsum = xor_sum<LOG_LPT, 6>(l[j]);
      float a[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) a[e] = xor_sum<LOG_LPT, 6>(acc[j][e]);
      if (tslot != 0) continue;
      const int row = v / n_rep;
      const int hq = h * n_rep + (v % n_rep);
      const int t = qb + row;
      if (nsplit == 1) {
        const float inv = 1.f / fmaxf(lsum, 1.17549435e-38f);
        T* op = out + int64_t(t) * o_st + int64_t(hq) * o_sh + sub * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) op[e] = from_f32<T>(a[e] * inv);
      } else {
        const int64_t idx =
            int64_t(part_off) + (int64_t(t - q0) * n_q_heads + hq) * nsplit + split;
        if (sub == 0) part_ml[idx] = make_float2(m[j], lsum);
        float* pa = part_acc + idx * D + sub * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) pa[e] = a[e];
      }
    }
  }
}

// One block per query token; threadIdx.y walks query heads, threadIdx.x the head dimension.
template <typename T>
__global__ __launch_bounds__(256) void attn_combine_kernel(
    const int32_t* __restrict__ plan, const int32_t* __restrict__ qsl,
    const int32_t* __restrict__ ctx, int32_t n_reqs, int32_t n_q_heads, int32_t head_dim,
    const float2* __restrict__ part_ml, const float* __restrict__ part_acc, T* __restrict__ out,
    int64_t o_st, int64_t o_sh) {
  const int t = blockIdx.x;
  // Request owning token t: the last r with qsl[r] <= t (requests with c == 0 are skipped).
  int lo = 0, hi = n_reqs - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (qsl[mid] <= t) lo = mid; else hi = mid - 1;
  }
  const int r = lo;
  const int q0 = qsl[r], c = qsl[r + 1] - q0;
  if (t < q0 || t >= q0 + c) return;
  const int32_t* rq = plan + plan[H_REQ_OFF] + r * kReqWords;
  const int nsplit = rq[R_NSPLIT], split_len = rq[R_SPLITLEN], part_off = rq[R_PARTOFF];
  if (nsplit <= 1) return;
  const int L = ctx[r];
  const int lim = L - c + (t - q0);
  const int n_valid = lim < 0 ? 0 : min(nsplit, lim / split_len + 1);
  for (int hq = blockIdx.y * blockDim.y + threadIdx.y; hq < n_q_heads;
       hq += gridDim.y * blockDim.y) {
    const int64_t base = int64_t(part_off) + (int64_t(t - q0) * n_q_heads + hq) * nsplit;
    float mmax = -INFINITY;
    for (int s = 0; s < n_valid; ++s) mmax = fmaxf(mmax, part_ml[base + s].x);
    for (int x = threadIdx.x; x < head_dim; x += blockDim.x) {
      float lsum = 0.f, a = 0.f;
      if (mmax != -INFINITY) {
        for (int s = 0; s < n_valid; ++s) {
          const float2 ml = part_ml[base + s];
          const float w = exp2_fast(ml.x - mmax);
          lsum = fmaf(w, ml.y, lsum);
          a = fmaf(w, part_acc[(base + s) * head_dim + x], a);
        }
      }
      out[int64_t(t) * o_st + int64_t(hq) * o_sh + x] =
          from_f32<T>(a / fmaxf(lsum, 1.17549435e-38f));
    }
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

bool head_dim_supported(int32_t d) {
  return d == 8 || d == 16 || d == 32 || d == 64 || d == 128 || d == 256;
}

int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

struct PlanItem {
  int32_t w[kItemWords];
  int64_t cost;
};

template <typename T>
int launch_rows(int32_t D, dim3 grid, hipStream_t s, const void* q, int64_t q_st, int64_t q_sh,
                const void* kp, const void* vp, const int32_t* bt, int64_t bt_stride,
                const int32_t* qsl, const int32_t* ctx, const int32_t* plan, int32_t hq,
                int32_t hkv, int32_t nb, int32_t bs, float scale_log2, void* out, int64_t o_st,
                int64_t o_sh, float2* ml, float* pacc) {
#define EDGERAG_ROWS(DIM)                                                                         \
  case DIM:                                                                                       \
    hipLaunchKernelGGL((attn_rows_kernel<T, DIM>), grid, dim3(kWave), 0, s,                      \
                       static_cast<const T*>(q), q_st, q_sh, static_cast<const T*>(kp),           \
                       static_cast<const T*>(vp), bt, bt_stride, qsl, ctx, plan, hq, hkv, nb, bs, \
                       scale_log2, static_cast<T*>(out), o_st, o_sh, ml, pacc);                   \
    break;
  switch (D) {
    EDGERAG_ROWS(8)
    EDGERAG_ROWS(16)
    EDGERAG_ROWS(32)
    EDGERAG_ROWS(64)
    EDGERAG_ROWS(128)
    EDGERAG_ROWS(256)
    default: return fail(EDGERAG_EUNSUPPORTED, "edgerag_paged_attention: head_dim %d", D);
  }
#undef EDGERAG_ROWS
  return check_launch("edgerag_paged_attention(rows)");
}

}  // namespace
}  // namespace edgerag

using namespace edgerag;

extern "C" int edgerag_attn_plan(const int32_t* query_start_loc, const int32_t* context_lens,
                                 int32_t num_reqs, int32_t n_q_heads, int32_t n_kv_heads,
                                 int32_t head_dim, int32_t block_size, int32_t max_blocks_per_seq,
                                 int32_t dtype, int32_t* plan, int64_t plan_capacity_words,
                                 int64_t* plan_words, int64_t* workspace_bytes) {
  clear_error();
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
  // Total KV token-heads the batch reads, to size the splits.
  int64_t work = 0;
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
    if (c > 0) work += L * n_kv_heads;
  }
  int64_t split_len = std::max<int64_t>(kMinSplit, (work + kTargetItems - 1) / kTargetItems);
  split_len = round_up(split_len, std::max(block_size, 16));

  std::vector<PlanItem> items;
  std::vector<int32_t> reqs(size_t(num_reqs) * kReqWords, 0);
  int64_t n_partials = 0;
  for (int r = 0; r < num_reqs; ++r) {
    const int q0 = query_start_loc[r];
    const int c = query_start_loc[r + 1] - q0;
    const int L = context_lens[r];
    int32_t* rq = reqs.data() + size_t(r) * kReqWords;
    const int nsplit = c == 0 ? 0 : int((L + split_len - 1) / split_len);
    rq[R_NSPLIT] = nsplit;
    rq[R_SPLITLEN] = int32_t(split_len);
    rq[R_PARTOFF] = int32_t(n_partials);
    if (c == 0) continue;
    if (nsplit > 1) n_partials += int64_t(c) * n_q_heads * nsplit;
    if (n_partials > INT32_MAX)
      return fail(EDGERAG_EUNSUPPORTED, "edgerag_attn_plan: batch needs > 2^31 split partials");
    for (int tile = 0; tile < c; tile += kQTile) {
      const int qc = std::min(kQTile, c - tile);
      const int last_visible = L - c + tile + qc - 1;  // causal limit of the tile's last row
      for (int s = 0; s < nsplit; ++s) {
        const int kb = int(s * split_len);
        if (kb > last_visible) break;
        const int ke = int(std::min<int64_t>(L, (s + 1) * split_len));
        const int ke_eff = std::min(ke, last_visible + 1);
        for (int h = 0; h < n_kv_heads; ++h) {
          PlanItem p{};
          p.w[I_REQ] = r;
          p.w[I_HEAD] = h;
          p.w[I_QBEGIN] = q0 + tile;
          p.w[I_QCOUNT] = qc;
          p.w[I_KVBEGIN] = kb;
          p.w[I_KVEND] = ke_eff;
          p.w[I_SPLIT] = s;
          p.w[I_KIND] = 0;
          p.cost = int64_t(ke_eff - kb) * ((qc * n_rep + kQR - 1) / kQR);
          items.push_back(p);
        }
      }
    }
  }
  // Heaviest first: the dispatcher hands blocks out in index order, so this is LPT scheduling.
  std::stable_sort(items.begin(), items.end(),
                   [](const PlanItem& a, const PlanItem& b) { return a.cost > b.cost; });

  const int64_t item_off = kHeaderWords;
  const int64_t req_off = item_off + int64_t(items.size()) * kItemWords;
  const int64_t words = req_off + int64_t(num_reqs) * kReqWords;
  *plan_words = words;
  *workspace_bytes = round_up(n_partials * int64_t(sizeof(float2)), 256) +
                     round_up(n_partials * head_dim * int64_t(sizeof(float)), 256);
  if (plan == nullptr) return EDGERAG_OK;
  if (plan_capacity_words < words)
    return fail(EDGERAG_EWORKSPACE, "edgerag_attn_plan: plan needs %lld words, capacity %lld",
                (long long)words, (long long)plan_capacity_words);
  if (words > INT32_MAX) return fail(EDGERAG_EUNSUPPORTED, "edgerag_attn_plan: plan too large");
  std::fill(plan, plan + kHeaderWords, 0);
  plan[H_MAGIC] = kPlanMagic;
  plan[H_VERSION] = kPlanVersion;
  plan[H_N_ITEMS] = int32_t(items.size());
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
  for (size_t i = 0; i < items.size(); ++i)
    std::copy(items[i].w, items[i].w + kItemWords, plan + item_off + int64_t(i) * kItemWords);
  std::copy(reqs.begin(), reqs.end(), plan + req_off);
  return EDGERAG_OK;
}

extern "C" int edgerag_paged_attention(
    const int32_t* plan_host, const int32_t* plan_dev, int64_t plan_words, const void* q,
    int64_t q_stride_tok, int64_t q_stride_head, const void* key_pool, const void* value_pool,
    int32_t dtype, const int32_t* block_tables, int64_t block_tables_stride,
    const int32_t* query_start_loc, const int32_t* context_lens, int32_t num_reqs,
    int32_t num_tokens, int32_t n_q_heads, int32_t n_kv_heads, int32_t head_dim,
    int32_t block_size, int32_t num_blocks, float scale, void* out, int64_t out_stride_tok,
    int64_t out_stride_head, void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
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
  const int n_items = plan_host[H_N_ITEMS];
  const int64_t n_partials = plan_host[H_N_PARTIALS];
  const int64_t ml_bytes = round_up(n_partials * int64_t(sizeof(float2)), 256);
  const int64_t need = ml_bytes + round_up(n_partials * head_dim * int64_t(sizeof(float)), 256);
  if (workspace_bytes < need || (need > 0 && workspace == nullptr))
    return fail(EDGERAG_EWORKSPACE, "edgerag_paged_attention: workspace %lld bytes, need %lld",
                (long long)workspace_bytes, (long long)need);
  if (n_items == 0) return EDGERAG_OK;
  if (q == nullptr || key_pool == nullptr || value_pool == nullptr || out == nullptr ||
      block_tables == nullptr || query_start_loc == nullptr || context_lens == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention: NULL pointer");
  const int es = elem_size(dtype);
  if (!aligned16(key_pool) || !aligned16(value_pool) || !aligned16(q) ||
      (q_stride_tok * es) % 16 != 0 || (q_stride_head * es) % 16 != 0)
    return fail(EDGERAG_EINVAL, "edgerag_paged_attention: q and pools must be 16-byte aligned");

  auto s = static_cast<hipStream_t>(stream);
  float2* ml = static_cast<float2*>(workspace);
  float* pacc = reinterpret_cast<float*>(static_cast<char*>(workspace) + ml_bytes);
  const float scale_log2 = scale * 1.4426950408889634f;
  int rc = EDGERAG_OK;
  const dim3 grid(n_items);
  switch (dtype) {
    case EDGERAG_F32:
      rc = launch_rows<float>(head_dim, grid, s, q, q_stride_tok, q_stride_head, key_pool,
                              value_pool, block_tables, block_tables_stride, query_start_loc,
                              context_lens, plan_dev, n_q_heads, n_kv_heads, num_blocks, block_size,
                              scale_log2, out, out_stride_tok, out_stride_head, ml, pacc);
      break;
    case EDGERAG_F16:
      rc = launch_rows<f16>(head_dim, grid, s, q, q_stride_tok, q_stride_head, key_pool,
                            value_pool, block_tables, block_tables_stride, query_start_loc,
                            context_lens, plan_dev, n_q_heads, n_kv_heads, num_blocks, block_size,
                            scale_log2, out, out_stride_tok, out_stride_head, ml, pacc);
      break;
    case EDGERAG_BF16:
      rc = launch_rows<bf16>(head_dim, grid, s, q, q_stride_tok, q_stride_head, key_pool,
                             value_pool, block_tables, block_tables_stride, query_start_loc,
                             context_lens, plan_dev, n_q_heads, n_kv_heads, num_blocks, block_size,
                             scale_log2, out, out_stride_tok, out_stride_head, ml, pacc);
      break;
    default:
      return fail(EDGERAG_EINVAL, "edgerag_paged_attention: dtype %d", dtype);
  }
  if (rc != EDGERAG_OK || n_partials == 0) return rc;

  const dim3 cblock(64, 4);
  const dim3 cgrid(num_tokens, (n_q_heads + 3) / 4);
#define EDGERAG_COMBINE(TYPE)                                                                     \
  hipLaunchKernelGGL((attn_combine_kernel<TYPE>), cgrid, cblock, 0, s, plan_dev, query_start_loc, \
                     context_lens, num_reqs, n_q_heads, head_dim, ml, pacc,                       \
                     static_cast<TYPE*>(out), out_stride_tok, out_stride_head)
  switch (dtype) {
    case EDGERAG_F32: EDGERAG_COMBINE(float); break;
    case EDGERAG_F16: EDGERAG_COMBINE(f16); break;
    case EDGERAG_BF16: EDGERAG_COMBINE(bf16); break;
  }
#undef EDGERAG_COMBINE
  return check_launch("edgerag_paged_attention(combine)");
}
