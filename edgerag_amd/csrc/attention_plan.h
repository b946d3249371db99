// Layout of the attention work plan (int32 words) shared by the host planner and the kernels,
// and the launch bundle the run entry point hands to each kernel family.
#pragma once

#include "common.h"

namespace edgerag {
namespace plan {

constexpr int32_t kMagic = 0x47415245;  // "ERAG"
constexpr int32_t kVersion = 6;
constexpr int kHeaderWords = 24;
constexpr int kItemWords = 8;
constexpr int kReqWords = 4;
constexpr int kCombineWords = 8;

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
  H_N_ROW_ITEMS,       // items [0, n_row) are decode-row items
  H_MAX_ROW_VECS,      // largest c * n_rep among row items
  H_MAX_SPLIT_BLOCKS,  // blocks in the longest decode split
  H_N_COMBINE,         // rows (query tokens of split requests) attn_combine_kernel merges
  H_COMBINE_OFF,       // word offset of the combine list
  H_TILE_KIND,         // 0: prefill tiles run on the row kernel, 1: on the MFMA tile kernel
  H_ROW_WAVES,         // 0: decode rows split across workgroups (partials + combine list);
                       // W > 0: one workgroup per row item, its W waves split the keys and
                       // merge in LDS (partials only where a context is cut into parts)
  H_OVERLAP,           // 1: planned for tiles and rows on two streams (tiles shared), 0: one
  H_SLOTS,             // S > 0: the row requests' partials sit in S slots per (token, q head)
                       // (rows cut into parts); 0: nsplit slots per (token, q head)
};
// Waves a workgroup-split row item may use (the kernel's LDS merge is sized for this many).
constexpr int kMaxRowWaves = 16;
enum Item { I_REQ = 0, I_HEAD, I_QBEGIN, I_QCOUNT, I_KVBEGIN, I_KVEND, I_SPLIT, I_PAD };
static_assert(kItemWords == 8 && I_KVBEGIN == 4 && I_PAD == 7,
              "the decode kernel reads an item as two int4 words");
// R_PSTRIDE: partial slots per (token, q head): nsplit, or H_SLOTS for slotted row requests,
// whose splits past nsplit hold empty records (m = -inf). Partial (t, hq, s) of request r sits at
// R_PARTOFF + ((t - q0) * n_q_heads + hq) * R_PSTRIDE + s.
enum Req { R_NSPLIT = 0, R_SPLITLEN, R_PARTOFF, R_PSTRIDE };
// Combine-list entry: everything one merge needs in a single 32-byte load.
enum Combine { C_TOK = 0, C_Q0, C_C, C_L, C_NSPLIT, C_SPLITLEN, C_PARTOFF, C_PSTRIDE };
// Largest slot count of a slotted plan (the slotted merge launch reads every slot of a row).
constexpr int kMaxPartSlots = 32;

}  // namespace plan

// Everything a kernel launch needs; built once per edgerag_paged_attention call.
struct AttnLaunch {
  hipStream_t s;
  const void* q;
  int64_t q_st, q_sh;
  const void *kp, *vp;
  const int32_t* bt;
  int64_t bt_stride;
  const int32_t *qsl, *ctx, *plan;
  int32_t hq, hkv, nb, bs;
  float scale_log2;
  void* out;
  int64_t o_st, o_sh;
  float2* ml;
  float* pacc;
  // Append fused into the decode rows (nk == NULL: off): the step's new K/V rows, [tokens,
  // n_kv_heads, head_dim] at nk + t * n_st + h * n_sh, written to the pools at slots[t].
  const void *nk, *nv;
  int64_t n_st, n_sh;
  const int32_t* slots;
};

// Prefill tiles on MFMA (attention_prefill.hip): fp16, head_dim 64.
#ifndef EDGERAG_TILE_ROWS
#define EDGERAG_TILE_ROWS 128
#endif
// Virtual query rows (token x head-in-group) per MFMA tile workgroup: 32 per wave.
constexpr int kMfmaTileRows = EDGERAG_TILE_ROWS;
constexpr int kMaxTileBlocks = 512;  // block ids one tile item stages in LDS (caps its split)
// shared: one workgroup per CU (the rest of each CU is left to concurrently running rows).
void launch_prefill_tiles_f16_d64(const AttnLaunch& a, int item_base, int count, bool shared);
// Whether a pool of this size can use the MFMA tile kernel (buffer-resource addressing).
bool prefill_tiles_supported(int32_t num_blocks, int32_t block_size);

}  // namespace edgerag
