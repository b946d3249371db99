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

// Workspace route of the tiled GEMM for (M, K, N, bits, group_size): `splits` = 0 when the
// plain launch is used, 1 for 64x64 tiles without a split, else the number of k ranges; `bytes`
// is the workspace a split needs (its fp32 partial tiles: at most 8 MiB).
struct SplitPlan {
  int splits;
  int64_t bytes;
};
SplitPlan qlinear_split_plan(int32_t m, int32_t k, int32_t n, int32_t bits, int32_t g);

// Runs the workspace route when the plan takes the shape (a split: two launches, the k ranges'
// partial tiles into the workspace, then their sum in split order and the epilogue) and the
// workspace holds `bytes`; returns false, enqueuing nothing, otherwise.
bool launch_qlinear_split(const f16* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                          const f16* scales, const f16* bias, int32_t n, int32_t bits, int32_t g,
                          f16* y, int64_t ys, void* ws, int64_t ws_bytes, hipStream_t s);

// Operands of the fused epilogues and of normed inputs (zero when unused).
struct EpiArgs {
  const f16* cos_tok;    // [m, head_dim]: cos table row at each token's position
  const f16* sin_tok;    // [m, head_dim]
  const int32_t* slots;  // [m]: pool slot of each token's K/V (out of range: not written)
  f16* q_out;            // [m, n_q_heads, head_dim] at q_out + t q_st + h head_dim
  int64_t q_st;
  f16* kpool;  // head-major [n_kv_heads, num_blocks, block_size, head_dim]
  f16* vpool;
  int32_t num_blocks, block_size, n_q_heads, n_kv_heads, head_dim;
  // Residual epilogue (the projection feeding a residual add + RMSNorm): hidden[t][n] =
  // fp16(hidden[t][n] + y[t][n]) in place, part[t * grid + workgroup] = the sum of the new values
  // squared over the workgroup's rows (fp32, a fixed order), and, when xw != NULL,
  // xw[t][n] = fp16(next_w[n] * hidden[t][n]): the next RMSNorm's weight applied, its 1 / rms not.
  f16* hidden;
  int64_t hid_st;
  float* part;
  const f16* next_w;
  f16* xw;
  int64_t xw_st;
  // Normed input (a projection after RMSNorm, x = a residual producer's xw): r_t =
  // rsqrt(sum of norm_part[t][0, norm_parts) / K + eps) multiplies token t's fp32 sums.
  const float* norm_part;
  int32_t norm_parts;
  float eps;
};

// Partial sums per token a normed launch can read (norm_parts).
constexpr int kNormMaxParts = 256;

// RoPE + KV-append form for decode batches: W is the fused [q heads | k heads | v heads]
// projection (N = heads * head_dim rows, INT8 per-channel); q heads are rotated into q_out, k
// heads rotated and v heads copied into the pools at the token's slot. The projection values are
// the fp16 outputs launch_qlinear_mfma would write for the same shape. Covered: M <= 64, K a
// multiple of 64 (at least 256, at most 8 waves' worth), head_dim a multiple of 32, and shapes
// the plain launch runs with one k-slice.
bool qlinear_rope_supported(int32_t m, int32_t k, int32_t n, int32_t bits, int32_t g,
                            int32_t heads, int32_t head_dim, const void* x, int64_t x_stride,
                            const void* packed);
// True when launch_qlinear_rope takes the shape on the streaming GEMV alone; otherwise the tiled
// GEMM's epilogue reads cos / sin in 8-byte runs, so their rows must be 8-byte aligned.
bool stream_rope_shape(int32_t m, int32_t k, int32_t n, int32_t heads, int32_t head_dim);
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
                           const EpiArgs& ea, hipStream_t s);

// Residual form for decode batches (M <= 16, INT8 per-channel): the plain launch's y is added to
// ea.hidden in place and per-(token, workgroup) sums of squares go to ea.part. Returns the number
// of partial sums per token (workgroups) for the shape, 0 when it is not covered.
int qlinear_residual_parts(int32_t m, int32_t k, int32_t n, int32_t bits, int32_t g,
                           const void* x, int64_t x_stride, const void* packed);
void launch_qlinear_residual(const f16* x, int64_t xs, int32_t m, int32_t k,
                             const uint8_t* packed, const f16* scales, const f16* bias, int32_t n,
                             const EpiArgs& ea, hipStream_t s);

}  // namespace edgerag
