// Launchers of the MFMA weight-only linear kernels (quant_mfma.hip), called by
// edgerag_quant_linear for fp16 activations.
#pragma once

#include "common.h"

namespace edgerag {

// Whether the MFMA kernels take this shape: K a whole number of 16-byte lane loads per row
// (64 k for INT8, 128 k for INT4), one scale per lane load (group_size % 16 for INT8, % 32 for
// INT4), 16-byte aligned weights and activations.
bool qlinear_mfma_supported(int32_t k, int32_t bits, int32_t g, const void* x, int64_t x_stride,
                            const void* packed);

// y[M, N] = x[M, K] . W^T (+ bias) with W = fp16(code) * fp16(scale) rounded once, like the
// reference's dequantize_groupwise; fp32 accumulation on v_mfma_f32_*_f16. Enqueues on `s`.
void launch_qlinear_mfma(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                         const f16* scales, const f16* bias, int32_t n, int32_t bits, int32_t g,
                         f16* y, int64_t ys, hipStream_t s);

// Operands of the fused RoPE + KV-append epilogue (unused by the other epilogues).
struct EpiArgs {
  const f16* cos_tok;    // [m, head_dim]: cos table row at each token's position
  const f16* sin_tok;    // [m, head_dim]
  const int32_t* slots;  // [m]: pool slot of each token's K/V (out of range: not written)
  f16* q_out;            // [m, n_q_heads, head_dim] at q_out + t q_st + h head_dim
  int64_t q_st;
  f16* kpool;  // head-major [n_kv_heads, num_blocks, block_size, head_dim]
  f16* vpool;
  int32_t num_blocks, block_size, n_q_heads, n_kv_heads, head_dim;
};

// RoPE + KV-append form for decode batches: W is the fused [q heads | k heads | v heads]
// projection (N = heads * head_dim rows, INT8 per-channel); q heads are rotated into q_out, k
// heads rotated and v heads copied into the pools at the token's slot. The projection values are
// the fp16 outputs launch_qlinear_mfma would write for the same shape. Covered: M <= 64, K a
// multiple of 64 (at least 256, at most 8 waves' worth), head_dim a multiple of 32, and shapes
// the plain launch runs with one k-slice.
bool qlinear_rope_supported(int32_t m, int32_t k, int32_t n, int32_t bits, int32_t g,
                            int32_t heads, int32_t head_dim, const void* x, int64_t x_stride,
                            const void* packed);
void launch_qlinear_rope(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                         const f16* scales, const f16* bias, int32_t n, const EpiArgs& ea,
                         hipStream_t s);

// SwiGLU form for decode batches: W = [gate; up] (N = 2 I rows, INT8 per-channel), y[M, I] =
// fp16(fp16(silu(g)) * u) with g, u the fp16 outputs launch_qlinear_mfma would write for the same
// shape. Covered: M <= 64, K a multiple of 64 (at least 256), N at least 8192 (two 16-row tiles
// per workgroup).
bool qlinear_swiglu_supported(int32_t m, int32_t k, int32_t n, int32_t bits, int32_t g,
                              const void* x, int64_t x_stride, const void* packed);
void launch_qlinear_swiglu(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                           const f16* scales, const f16* bias, int32_t n, f16* y, int64_t ys,
                           hipStream_t s);

}  // namespace edgerag
