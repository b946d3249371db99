// Weight-only INT8 / INT4 quantisation and linear layers.
//
// Storage follows the reference exactly (edgerag/core/quant.py:60-138, linear.py:152-196):
//   packed  uint8 [N, K] (int8 codes, two's complement) or [N, K/2] (int4, byte j = (c[2j]+8) |
//           (c[2j+1]+8) << 4), scales fp16 [N, K/group_size], optional fp16 bias [N].
// The linear never materialises the fp16 weight: each wave streams its output rows' packed bytes
// from HBM once, rebuilds w = fp16(code) * scale in registers (one fp16 rounding, the same value
// the reference's dequantize_groupwise produces) and accumulates x . w in fp32 with
// v_dot2_f32_f16. Weight bytes dominate traffic for M <= 64, so the kernel is HBM-bound there.
#include <cmath>

#include "common.h"
#include "quant_mfma.h"

namespace edgerag {
namespace {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// ---- quantize ---------------------------------------------------------------------------------
// One wavefront per (row, group). amax over the group, scale = amax / qmax in fp32 (1.0 for an
// all-zero group), codes = clamp(rint(w / scale)) with rint = round-half-even like torch.round.
template <typename T, int BITS>
__global__ __launch_bounds__(256) void quantize_kernel(const T* __restrict__ w, int32_t n,
                                                       int32_t k, int32_t g,
                                                       uint8_t* __restrict__ packed,
                                                       f16* __restrict__ scales) {
  const int wave = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int lane = threadIdx.x % kWave;
  const int groups = k / g;
  if (wave >= n * groups) return;
  const int row = wave / groups, grp = wave % groups;
  const T* src = w + int64_t(row) * k + int64_t(grp) * g;
  float amax = 0.f;
  for (int i = lane; i < g; i += kWave) amax = fmaxf(amax, fabsf(to_f32<T>(src[i])));
  amax = xor_max<0, 6>(amax);
  constexpr float qmax = BITS == 4 ? 7.f : 127.f;
  const float scale = amax > 0.f ? amax / qmax : 1.f;
  if (lane == 0) scales[int64_t(row) * groups + grp] = __float2half_rn(scale);
  if constexpr (BITS == 8) {
    uint8_t* dst = packed + int64_t(row) * k + int64_t(grp) * g;
    for (int i = lane; i < g; i += kWave) {
      const float c = fminf(fmaxf(rintf(to_f32<T>(src[i]) / scale), -qmax), qmax);
      dst[i] = uint8_t(int8_t(c));
    }
  } else {
    uint8_t* dst = packed + int64_t(row) * (k / 2) + int64_t(grp) * (g / 2);
    for (int i = lane; i < g / 2; i += kWave) {
      const float c0 = fminf(fmaxf(rintf(to_f32<T>(src[2 * i]) / scale), -qmax), qmax);
      const float c1 = fminf(fmaxf(rintf(to_f32<T>(src[2 * i + 1]) / scale), -qmax), qmax);
      dst[i] = uint8_t((int(c0) + 8) | ((int(c1) + 8) << 4));
    }
  }
}

template <int BITS>
__device__ __forceinline__ int code_at(const uint8_t* __restrict__ row, int kk) {
  if constexpr (BITS == 8) {
    return int(int8_t(row[kk]));
  } else {
    const uint8_t b = row[kk >> 1];
    return int((kk & 1) ? (b >> 4) : (b & 15)) - 8;
  }
}

// ---- dequantize -------------------------------------------------------------------------------
template <int BITS>
__global__ __launch_bounds__(256) void dequantize_kernel(const uint8_t* __restrict__ packed,
                                                         const f16* __restrict__ scales, int32_t n,
                                                         int32_t k, int32_t g,
                                                         f16* __restrict__ out) {
  const int64_t total = int64_t(n) * k;
  const int64_t row_bytes = BITS == 8 ? k : k / 2;
  const int groups = k / g;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * blockDim.x) {
    const int row = int(i / k), kk = int(i % k);
    const int code = code_at<BITS>(packed + row * row_bytes, kk);
    const float sc = __half2float(scales[int64_t(row) * groups + kk / g]);
    out[i] = __float2half_rn(float(code) * sc);  // exact product, one rounding (= fp16 mul)
  }
}

// ---- linear: vector path ------------------------------------------------------------------------
// Each wave owns ROWS consecutive output rows and MB activation rows. Per iteration a lane takes
// 16 consecutive k: 16 bytes of an INT8 row or 8 bytes of an INT4 row, so a wave covers 1024 k.
// Requires K % 16 == 0 and group_size % 16 == 0 (all 16 k of a lane share one scale).
constexpr int kLinThreads = 256;
constexpr int kKPerLane = 16;

template <int BITS>
__device__ __forceinline__ void dequant16(const uint8_t* __restrict__ wrow, int k0, f16 scale,
                                          half2_t (&w)[8]) {
  int codes[16];
  if constexpr (BITS == 8) {
    const Vec16 raw = *reinterpret_cast<const Vec16*>(wrow + k0);
#pragma unroll
    for (int i = 0; i < 16; ++i) codes[i] = int(int8_t((raw.w[i / 4] >> (8 * (i % 4))) & 0xff));
  } else {
    const uint2 raw = *reinterpret_cast<const uint2*>(wrow + k0 / 2);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t word = i < 8 ? raw.x : raw.y;
      codes[i] = int((word >> (4 * (i % 8))) & 15) - 8;
    }
  }
  const _Float16 s = *reinterpret_cast<const _Float16*>(&scale);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // fp16(code) is exact for |code| <= 127; the product rounds once, like codes.half() * scales.
    w[i] = half2_t{_Float16(codes[2 * i]) * s, _Float16(codes[2 * i + 1]) * s};
  }
}

template <int BITS, int ROWS, int MB, typename XT>
__global__ __launch_bounds__(kLinThreads) void qlinear_vec_kernel(
    const XT* __restrict__ x, int64_t x_stride, int32_t m, int32_t k,
    const uint8_t* __restrict__ packed, const f16* __restrict__ scales,
    const f16* __restrict__ bias, int32_t n, int32_t g, XT* __restrict__ y, int64_t y_stride) {
  const int wave = (blockIdx.x * kLinThreads + threadIdx.x) / kWave;
  const int lane = threadIdx.x % kWave;
  const int n0 = wave * ROWS;
  if (n0 >= n) return;
  const int64_t row_bytes = BITS == 8 ? k : k / 2;
  const int groups = k / g;
  for (int mb = 0; mb < m; mb += MB) {
    float acc[ROWS][MB];
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
      for (int j = 0; j < MB; ++j) acc[r][j] = 0.f;
    for (int k0 = lane * kKPerLane; k0 < k; k0 += kWave * kKPerLane) {
      // Activations for this k slice, per activation row.
      half2_t xh[MB][8];
      float xf[MB][16];
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        const int mm = mb + j < m ? mb + j : m - 1;  // clamp: padded rows are never written
        const XT* xp = x + int64_t(mm) * x_stride + k0;
        if constexpr (__is_same(XT, f16)) {
          const Vec16 a = load16(xp), b = load16(xp + 8);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            xh[j][i] = *reinterpret_cast<const half2_t*>(&a.w[i]);
            xh[j][4 + i] = *reinterpret_cast<const half2_t*>(&b.w[i]);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) xf[j][i] = to_f32<XT>(xp[i]);
        }
      }
#pragma unroll
      for (int r = 0; r < ROWS; ++r) {
        const int row = n0 + r < n ? n0 + r : n - 1;
        half2_t w[8];
        dequant16<BITS>(packed + row * row_bytes, k0, scales[int64_t(row) * groups + k0 / g], w);
#pragma unroll
        for (int j = 0; j < MB; ++j) {
          if constexpr (__is_same(XT, f16)) {
#pragma unroll
            for (int i = 0; i < 8; ++i)
              acc[r][j] = __builtin_amdgcn_fdot2(w[i], xh[j][i], acc[r][j], false);
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              acc[r][j] = fmaf(float(w[i].x), xf[j][2 * i], acc[r][j]);
              acc[r][j] = fmaf(float(w[i].y), xf[j][2 * i + 1], acc[r][j]);
            }
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        const float v = xor_sum<0, 6>(acc[r][j]);
        if (lane == 0 && n0 + r < n && mb + j < m) {
          const float b = bias != nullptr ? __half2float(bias[n0 + r]) : 0.f;
          y[int64_t(mb + j) * y_stride + n0 + r] = from_f32<XT>(v + b);
        }
      }
    }
  }
}

// ---- linear: generic path (any K, any group size) ----------------------------------------------
template <int BITS, typename XT>
__global__ __launch_bounds__(kLinThreads) void qlinear_generic_kernel(
    const XT* __restrict__ x, int64_t x_stride, int32_t m, int32_t k,
    const uint8_t* __restrict__ packed, const f16* __restrict__ scales,
    const f16* __restrict__ bias, int32_t n, int32_t g, XT* __restrict__ y, int64_t y_stride) {
  const int wave = (blockIdx.x * kLinThreads + threadIdx.x) / kWave;
  const int lane = threadIdx.x % kWave;
  if (wave >= int64_t(m) * n) return;
  const int mm = wave / n, row = wave % n;
  const int64_t row_bytes = BITS == 8 ? k : k / 2;
  const int groups = k / g;
  float acc = 0.f;
  for (int kk = lane; kk < k; kk += kWave) {
    const f16 w = __float2half_rn(float(code_at<BITS>(packed + row * row_bytes, kk)) *
                                  __half2float(scales[int64_t(row) * groups + kk / g]));
    acc = fmaf(__half2float(w), to_f32<XT>(x[int64_t(mm) * x_stride + kk]), acc);
  }
  acc = xor_sum<0, 6>(acc);
  if (lane == 0) {
    const float b = bias != nullptr ? __half2float(bias[row]) : 0.f;
    y[int64_t(mm) * y_stride + row] = from_f32<XT>(acc + b);
  }
}

unsigned waves_to_blocks(int64_t waves) {
  return unsigned((waves * kWave + kLinThreads - 1) / kLinThreads);
}

int check_quant_shape(const char* fn, int32_t n, int32_t k, int32_t bits, int32_t g) {
  if (bits != 4 && bits != 8)
    return fail(EDGERAG_EINVAL, "%s: only 4- and 8-bit are supported, got %d", fn, bits);
  if (n <= 0 || k <= 0) return fail(EDGERAG_EINVAL, "%s: N=%d K=%d must be positive", fn, n, k);
  if (g <= 0) return fail(EDGERAG_EINVAL, "%s: group_size must be positive, got %d", fn, g);
  if (k % g != 0)
    return fail(EDGERAG_EINVAL, "%s: in_features=%d is not divisible by group_size=%d", fn, k, g);
  if (bits == 4 && k % 2 != 0)
    return fail(EDGERAG_EINVAL, "%s: input dimension %d must be even to pack two per byte", fn, k);
  return EDGERAG_OK;
}

template <int BITS, typename XT>
int launch_linear(const void* x, int64_t xs, int32_t m, int32_t k, const uint8_t* packed,
                  const void* scales, const void* bias, int32_t n, int32_t g, void* y, int64_t ys,
                  hipStream_t s) {
  const auto* xp = static_cast<const XT*>(x);
  const auto* sp = static_cast<const f16*>(scales);
  const auto* bp = static_cast<const f16*>(bias);
  auto* yp = static_cast<XT*>(y);
  const bool vec = k % kKPerLane == 0 && g % kKPerLane == 0 && aligned16(packed) &&
                   aligned16(x) && (xs * int64_t(sizeof(XT))) % 16 == 0 &&
                   (BITS == 4 || (k % 16 == 0));
  if (vec) {
    constexpr int kRows = 4;
    const int64_t waves = (n + kRows - 1) / kRows;
    if (m == 1) {
      hipLaunchKernelGGL((qlinear_vec_kernel<BITS, kRows, 1, XT>), dim3(waves_to_blocks(waves)),
                         dim3(kLinThreads), 0, s, xp, xs, m, k, packed, sp, bp, n, g, yp, ys);
    } else if (m == 2) {
      hipLaunchKernelGGL((qlinear_vec_kernel<BITS, kRows, 2, XT>), dim3(waves_to_blocks(waves)),
                         dim3(kLinThreads), 0, s, xp, xs, m, k, packed, sp, bp, n, g, yp, ys);
    } else {
      hipLaunchKernelGGL((qlinear_vec_kernel<BITS, kRows, 4, XT>), dim3(waves_to_blocks(waves)),
                         dim3(kLinThreads), 0, s, xp, xs, m, k, packed, sp, bp, n, g, yp, ys);
    }
  } else {
    hipLaunchKernelGGL((qlinear_generic_kernel<BITS, XT>), dim3(waves_to_blocks(int64_t(m) * n)),
                       dim3(kLinThreads), 0, s, xp, xs, m, k, packed, sp, bp, n, g, yp, ys);
  }
  return check_launch("edgerag_quant_linear");
}

}  // namespace
}  // namespace edgerag

using namespace edgerag;

extern "C" int edgerag_quantize(const void* weight, int32_t w_dtype, int32_t n, int32_t k,
                                int32_t bits, int32_t group_size, uint8_t* packed,
                                void* scales_f16, void* stream) {
  clear_error();
  if (int rc = check_quant_shape("edgerag_quantize", n, k, bits, group_size)) return rc;
  if (bits == 4 && group_size % 2 != 0)
    return fail(EDGERAG_EUNSUPPORTED,
                "edgerag_quantize: an odd group_size (%d) would split INT4 bytes across groups",
                group_size);
  if (weight == nullptr || packed == nullptr || scales_f16 == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_quantize: NULL pointer");
  auto s = static_cast<hipStream_t>(stream);
  const int64_t waves = int64_t(n) * (k / group_size);
  const dim3 grid(unsigned((waves * kWave + 255) / 256)), block(256);
  auto* sc = static_cast<f16*>(scales_f16);
#define EDGERAG_Q(TYPE)                                                                        \
  if (bits == 8)                                                                               \
    hipLaunchKernelGGL((quantize_kernel<TYPE, 8>), grid, block, 0, s,                          \
                       static_cast<const TYPE*>(weight), n, k, group_size, packed, sc);        \
  else                                                                                         \
    hipLaunchKernelGGL((quantize_kernel<TYPE, 4>), grid, block, 0, s,                          \
                       static_cast<const TYPE*>(weight), n, k, group_size, packed, sc);
  switch (w_dtype) {
    case EDGERAG_F32: EDGERAG_Q(float); break;
    case EDGERAG_F16: EDGERAG_Q(f16); break;
    case EDGERAG_BF16: EDGERAG_Q(bf16); break;
    default: return fail(EDGERAG_EINVAL, "edgerag_quantize: dtype %d", w_dtype);
  }
#undef EDGERAG_Q
  return check_launch("edgerag_quantize");
}

extern "C" int edgerag_dequantize(const uint8_t* packed, const void* scales_f16, int32_t n,
                                  int32_t k, int32_t bits, int32_t group_size, void* weight_f16,
                                  void* stream) {
  clear_error();
  if (int rc = check_quant_shape("edgerag_dequantize", n, k, bits, group_size)) return rc;
  if (packed == nullptr || scales_f16 == nullptr || weight_f16 == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_dequantize: NULL pointer");
  auto s = static_cast<hipStream_t>(stream);
  const int64_t total = int64_t(n) * k;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65535LL * 16) blocks = 65535LL * 16;
  if (bits == 8)
    hipLaunchKernelGGL((dequantize_kernel<8>), dim3(unsigned(blocks)), dim3(256), 0, s, packed,
                       static_cast<const f16*>(scales_f16), n, k, group_size,
                       static_cast<f16*>(weight_f16));
  else
    hipLaunchKernelGGL((dequantize_kernel<4>), dim3(unsigned(blocks)), dim3(256), 0, s, packed,
                       static_cast<const f16*>(scales_f16), n, k, group_size,
                       static_cast<f16*>(weight_f16));
  return check_launch("edgerag_dequantize");
}

extern "C" int64_t edgerag_quant_linear_workspace_bytes(int32_t m, int32_t k, int32_t n,
                                                        int32_t bits, int32_t group_size) {
  return qlinear_split_plan(m, k, n, bits, group_size).bytes;
}

extern "C" int edgerag_quant_linear_ws(const void* x, int32_t x_dtype, int64_t x_stride, int32_t m,
                                       int32_t k, const uint8_t* packed, const void* scales_f16,
                                       const void* bias_f16, int32_t n, int32_t bits,
                                       int32_t group_size, void* y, int64_t y_stride,
                                       void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  if (workspace_bytes < 0 || (workspace_bytes > 0 && workspace == nullptr))
    return fail(EDGERAG_EINVAL, "edgerag_quant_linear_ws: workspace of %lld bytes at NULL",
                (long long)workspace_bytes);
  if (x_dtype == EDGERAG_F16 && m > 0 && x != nullptr && packed != nullptr &&
      scales_f16 != nullptr && y != nullptr && x_stride >= k && y_stride >= n &&
      check_quant_shape("edgerag_quant_linear_ws", n, k, bits, group_size) == EDGERAG_OK &&
      qlinear_mfma_supported(k, bits, group_size, x, x_stride, packed) &&
      launch_qlinear_split(static_cast<const f16*>(x), x_stride, m, k, packed,
                           static_cast<const f16*>(scales_f16), static_cast<const f16*>(bias_f16),
                           n, bits, group_size, static_cast<f16*>(y), y_stride, workspace,
                           workspace_bytes, static_cast<hipStream_t>(stream)))
    return check_launch("edgerag_quant_linear_ws");
  return edgerag_quant_linear(x, x_dtype, x_stride, m, k, packed, scales_f16, bias_f16, n, bits,
                              group_size, y, y_stride, stream);
}

extern "C" int edgerag_quant_linear(const void* x, int32_t x_dtype, int64_t x_stride, int32_t m,
                                    int32_t k, const uint8_t* packed, const void* scales_f16,
                                    const void* bias_f16, int32_t n, int32_t bits,
                                    int32_t group_size, void* y, int64_t y_stride, void* stream) {
  clear_error();
  if (int rc = check_quant_shape("edgerag_quant_linear", n, k, bits, group_size)) return rc;
  if (m < 0) return fail(EDGERAG_EINVAL, "edgerag_quant_linear: M < 0");
  if (m == 0) return EDGERAG_OK;
  if (x == nullptr || packed == nullptr || scales_f16 == nullptr || y == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_quant_linear: NULL pointer");
  if (x_stride < k || y_stride < n)
    return fail(EDGERAG_EINVAL, "edgerag_quant_linear: row strides (%lld, %lld) below K/N",
                (long long)x_stride, (long long)y_stride);
  auto s = static_cast<hipStream_t>(stream);
  if (x_dtype == EDGERAG_F16) {
    if (qlinear_mfma_supported(k, bits, group_size, x, x_stride, packed)) {
      launch_qlinear_mfma(static_cast<const f16*>(x), x_stride, m, k, packed,
                          static_cast<const f16*>(scales_f16), static_cast<const f16*>(bias_f16),
                          n, bits, group_size, static_cast<f16*>(y), y_stride, s);
      return check_launch("edgerag_quant_linear");
    }
    return bits == 8 ? launch_linear<8, f16>(x, x_stride, m, k, packed, scales_f16, bias_f16, n,
                                             group_size, y, y_stride, s)
                     : launch_linear<4, f16>(x, x_stride, m, k, packed, scales_f16, bias_f16, n,
                                             group_size, y, y_stride, s);
  }
  if (x_dtype == EDGERAG_F32) {
    return bits == 8 ? launch_linear<8, float>(x, x_stride, m, k, packed, scales_f16, bias_f16, n,
                                               group_size, y, y_stride, s)
                     : launch_linear<4, float>(x, x_stride, m, k, packed, scales_f16, bias_f16, n,
                                               group_size, y, y_stride, s);
  }
  return fail(EDGERAG_EUNSUPPORTED, "edgerag_quant_linear: activation dtype %d", x_dtype);
}

namespace edgerag {
namespace {

// The optional RMSNorm operands of the fused entry points: NULL norm_partials means a plain input.
// Returns EDGERAG_OK or an error code (with the message set).
int set_norm(const char* fn, int32_t m, const float* norm_partials, int32_t norm_parts, float eps,
             EpiArgs& ea) {
  if (norm_partials == nullptr) return EDGERAG_OK;
  if (norm_parts <= 0 || norm_parts > kNormMaxParts || m > 16 || !(eps >= 0.f) ||
      !std::isfinite(eps))
    return fail(EDGERAG_EUNSUPPORTED,
                "%s: normed input needs M <= 16 (got %d), 1..%d partial sums per token (got %d) "
                "and a finite eps >= 0",
                fn, m, kNormMaxParts, norm_parts);
  ea.norm_part = norm_partials;
  ea.norm_parts = norm_parts;
  ea.eps = eps;
  return EDGERAG_OK;
}

const void* aligned_stand_in() { return reinterpret_cast<const void*>(uintptr_t(256)); }

}  // namespace
}  // namespace edgerag

extern "C" int edgerag_quant_linear_swiglu_supported(int32_t x_dtype, int32_t m, int32_t k,
                                                     int32_t n, int32_t bits, int32_t group_size,
                                                     int32_t normed) {
  // Alignment is the caller's part of the contract; a 16-byte aligned stand-in checks the rest.
  const void* aligned = aligned_stand_in();
  return x_dtype == EDGERAG_F16 && n > 0 && k > 0 && group_size == k && (!normed || m <= 16) &&
                 qlinear_swiglu_supported(m, k, n, bits, group_size, aligned, k, aligned)
             ? 1
             : 0;
}

extern "C" int edgerag_quant_linear_swiglu(const void* x, int32_t x_dtype, int64_t x_stride,
                                           int32_t m, int32_t k, const uint8_t* packed,
                                           const void* scales_f16, const void* bias_f16, int32_t n,
                                           int32_t bits, int32_t group_size, void* y,
                                           int64_t y_stride, const float* norm_partials,
                                           int32_t norm_parts, float eps, void* stream) {
  clear_error();
  if (int rc = check_quant_shape("edgerag_quant_linear_swiglu", n, k, bits, group_size)) return rc;
  if (m < 0) return fail(EDGERAG_EINVAL, "edgerag_quant_linear_swiglu: M < 0");
  if (m == 0) return EDGERAG_OK;
  if (x == nullptr || packed == nullptr || scales_f16 == nullptr || y == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_quant_linear_swiglu: NULL pointer");
  if (x_stride < k || y_stride < n / 2)
    return fail(EDGERAG_EINVAL, "edgerag_quant_linear_swiglu: row strides (%lld, %lld) below K/I",
                (long long)x_stride, (long long)y_stride);
  if (x_dtype != EDGERAG_F16 ||
      !qlinear_swiglu_supported(m, k, n, bits, group_size, x, x_stride, packed))
    return fail(EDGERAG_EUNSUPPORTED,
                "edgerag_quant_linear_swiglu: shape not covered (dtype %d, M %d, K %d, N %d, "
                "bits %d, group %d); use edgerag_quant_linear + edgerag_silu_mul",
                x_dtype, m, k, n, bits, group_size);
  EpiArgs ea{};
  if (int rc = set_norm("edgerag_quant_linear_swiglu", m, norm_partials, norm_parts, eps, ea))
    return rc;
  launch_qlinear_swiglu(static_cast<const f16*>(x), x_stride, m, k, packed,
                        static_cast<const f16*>(scales_f16), static_cast<const f16*>(bias_f16), n,
                        static_cast<f16*>(y), y_stride, ea, static_cast<hipStream_t>(stream));
  return check_launch("edgerag_quant_linear_swiglu");
}

extern "C" int edgerag_quant_linear_rope_append_supported(int32_t x_dtype, int32_t m, int32_t k,
                                                         int32_t bits, int32_t group_size,
                                                         int32_t n_q_heads, int32_t n_kv_heads,
                                                         int32_t head_dim, int32_t normed) {
  if (x_dtype != EDGERAG_F16 || n_q_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || k <= 0 ||
      group_size != k || (normed && m > 16))
    return 0;
  const int64_t heads = int64_t(n_q_heads) + 2 * int64_t(n_kv_heads);
  if (heads * head_dim > INT32_MAX) return 0;
  const void* aligned = aligned_stand_in();
  return qlinear_rope_supported(m, k, int32_t(heads * head_dim), bits, group_size, int32_t(heads),
                                head_dim, aligned, k, aligned)
             ? 1
             : 0;
}

extern "C" int edgerag_quant_linear_rope_append(
    const void* x, int32_t x_dtype, int64_t x_stride, int32_t m, int32_t k, const uint8_t* packed,
    const void* scales_f16, const void* bias_f16, int32_t bits, int32_t group_size,
    const void* cos_tok, const void* sin_tok, int32_t n_q_heads, int32_t n_kv_heads,
    int32_t head_dim, void* q_out, int64_t q_stride_tok, const int32_t* slots, void* key_pool,
    void* value_pool, int32_t num_blocks, int32_t block_size, const float* norm_partials,
    int32_t norm_parts, float eps, void* stream) {
  clear_error();
  if (m < 0 || n_q_heads <= 0 || n_kv_heads <= 0 || head_dim <= 0 || head_dim % 2 ||
      num_blocks <= 0 || block_size <= 0)
    return fail(EDGERAG_EINVAL, "edgerag_quant_linear_rope_append: bad shape");
  const int64_t heads = int64_t(n_q_heads) + 2 * int64_t(n_kv_heads);
  if (heads * head_dim > INT32_MAX)
    return fail(EDGERAG_EINVAL, "edgerag_quant_linear_rope_append: projection too wide");
  const int32_t n = int32_t(heads * head_dim);
  if (int rc = check_quant_shape("edgerag_quant_linear_rope_append", n, k, bits, group_size))
    return rc;
  if (m == 0) return EDGERAG_OK;
  if (x == nullptr || packed == nullptr || scales_f16 == nullptr || cos_tok == nullptr ||
      sin_tok == nullptr || q_out == nullptr || slots == nullptr || key_pool == nullptr ||
      value_pool == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_quant_linear_rope_append: NULL pointer");
  if (x_stride < k || q_stride_tok < int64_t(n_q_heads) * head_dim)
    return fail(EDGERAG_EINVAL, "edgerag_quant_linear_rope_append: row strides (%lld, %lld) too small",
                (long long)x_stride, (long long)q_stride_tok);
  if (x_dtype != EDGERAG_F16 ||
      !qlinear_rope_supported(m, k, n, bits, group_size, int32_t(heads), head_dim, x, x_stride,
                              packed))
    return fail(EDGERAG_EUNSUPPORTED,
                "edgerag_quant_linear_rope_append: shape not covered (dtype %d, M %d, K %d, N %d, "
                "bits %d, group %d, head_dim %d); use edgerag_quant_linear + edgerag_rope_append",
                x_dtype, m, k, n, bits, group_size, head_dim);
  if (!stream_rope_shape(m, k, n, int32_t(heads), head_dim) &&
      ((reinterpret_cast<uintptr_t>(cos_tok) | reinterpret_cast<uintptr_t>(sin_tok)) & 7) != 0)
    return fail(EDGERAG_EINVAL,
                "edgerag_quant_linear_rope_append: cos_tok / sin_tok must be 8-byte aligned for "
                "M %d (the tiled GEMM reads them in 8-byte runs)", m);
  EpiArgs ea{};
  if (int rc = set_norm("edgerag_quant_linear_rope_append", m, norm_partials, norm_parts, eps,
                        ea))
    return rc;
  ea.cos_tok = static_cast<const f16*>(cos_tok);
  ea.sin_tok = static_cast<const f16*>(sin_tok);
  ea.slots = slots;
  ea.q_out = static_cast<f16*>(q_out);
  ea.q_st = q_stride_tok;
  ea.kpool = static_cast<f16*>(key_pool);
  ea.vpool = static_cast<f16*>(value_pool);
  ea.num_blocks = num_blocks;
  ea.block_size = block_size;
  ea.n_q_heads = n_q_heads;
  ea.n_kv_heads = n_kv_heads;
  ea.head_dim = head_dim;
  launch_qlinear_rope(static_cast<const f16*>(x), x_stride, m, k, packed,
                      static_cast<const f16*>(scales_f16), static_cast<const f16*>(bias_f16), n, ea,
                      static_cast<hipStream_t>(stream));
  return check_launch("edgerag_quant_linear_rope_append");
}

extern "C" int edgerag_quant_linear_residual_parts(int32_t x_dtype, int32_t m, int32_t k, int32_t n,
                                                   int32_t bits, int32_t group_size) {
  if (x_dtype != EDGERAG_F16 || m < 1 || k <= 0 || n <= 0) return 0;
  const void* aligned = aligned_stand_in();
  return qlinear_residual_parts(m, k, n, bits, group_size, aligned, k, aligned);
}

extern "C" int edgerag_quant_linear_residual(const void* x, int32_t x_dtype, int64_t x_stride,
                                             int32_t m, int32_t k, const uint8_t* packed,
                                             const void* scales_f16, const void* bias_f16,
                                             int32_t n, int32_t bits, int32_t group_size,
                                             void* hidden, int64_t hidden_stride, float* partials,
                                             int64_t partials_capacity, int32_t* n_parts,
                                             const void* next_norm_weight, void* xw,
                                             int64_t xw_stride, void* stream) {
  clear_error();
  if (int rc = check_quant_shape("edgerag_quant_linear_residual", n, k, bits, group_size))
    return rc;
  if (m < 0) return fail(EDGERAG_EINVAL, "edgerag_quant_linear_residual: M < 0");
  if (n_parts != nullptr) *n_parts = 0;
  if (m == 0) return EDGERAG_OK;
  if (x == nullptr || packed == nullptr || scales_f16 == nullptr || hidden == nullptr ||
      partials == nullptr)
    return fail(EDGERAG_EINVAL, "edgerag_quant_linear_residual: NULL pointer");
  if (x_stride < k || hidden_stride < n)
    return fail(EDGERAG_EINVAL, "edgerag_quant_linear_residual: row strides (%lld, %lld) below K/N",
                (long long)x_stride, (long long)hidden_stride);
  const int parts = x_dtype == EDGERAG_F16
                        ? qlinear_residual_parts(m, k, n, bits, group_size, x, x_stride, packed)
                        : 0;
  if (parts == 0)
    return fail(EDGERAG_EUNSUPPORTED,
                "edgerag_quant_linear_residual: shape not covered (dtype %d, M %d, K %d, N %d, "
                "bits %d, group %d); use edgerag_quant_linear + edgerag_rmsnorm",
                x_dtype, m, k, n, bits, group_size);
  if (partials_capacity < int64_t(m) * parts)
    return fail(EDGERAG_EWORKSPACE, "edgerag_quant_linear_residual: partials hold %lld floats, need %lld",
                (long long)partials_capacity, (long long)(int64_t(m) * parts));
  if ((next_norm_weight == nullptr) != (xw == nullptr) || (xw != nullptr && xw_stride < n))
    return fail(EDGERAG_EINVAL,
                "edgerag_quant_linear_residual: next_norm_weight and xw go together (xw row stride "
                ">= N)");
  EpiArgs ea{};
  ea.hidden = static_cast<f16*>(hidden);
  ea.hid_st = hidden_stride;
  ea.part = partials;
  ea.next_w = static_cast<const f16*>(next_norm_weight);
  ea.xw = static_cast<f16*>(xw);
  ea.xw_st = xw_stride;
  launch_qlinear_residual(static_cast<const f16*>(x), x_stride, m, k, packed,
                          static_cast<const f16*>(scales_f16), static_cast<const f16*>(bias_f16), n,
                          ea, static_cast<hipStream_t>(stream));
  if (n_parts != nullptr) *n_parts = parts;
  return check_launch("edgerag_quant_linear_residual");
}
