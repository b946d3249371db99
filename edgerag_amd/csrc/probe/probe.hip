// Measurement probes for the rooflines bench.py reports next to each kernel: the HBM ceilings
// that an access pattern can reach on this GPU, so a kernel's rate can be read against what is
// achievable for the same bytes, not only against the 8 TB/s datasheet figure.
//
// * probe_read_kernel: a plain streaming read. Each workgroup reads one contiguous slice of the
//   buffer with 16-byte loads, U loads in flight per thread -- the best case for a weight
//   stream of the same size.
// * probe_gather_kernel: one wavefront per list of chunk ids; each chunk (a multiple of 1 KiB,
//   read with 1 KiB wave-wide loads) sits at a random chunk-aligned offset -- the access pattern
//   of the paged KV pool (one 2 KiB (head, block) row of K or V per 16 tokens). With NT the loads
//   are non-temporal, as the decode rows read the pools.
// Neither kernel writes anything but a sentinel that no real data produces.
#include "../common.h"
#include "edgerag_probe.h"

namespace edgerag {
namespace {

constexpr int kProbeThreads = 256;

template <int U>
__global__ __launch_bounds__(kProbeThreads) void probe_read_kernel(const uint4* __restrict__ p,
                                                                   int64_t n16,
                                                                   uint32_t* __restrict__ sink) {
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t b = int64_t(blockIdx.x) * per, e = min(b + per, n16);
  uint32_t acc = 0;
  for (int64_t i = b + threadIdx.x; i < e; i += int64_t(kProbeThreads) * U) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = i + int64_t(u) * kProbeThreads;
      v[u] = j < e ? p[j] : uint4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

template <int LOADS, bool NT>
__global__ __launch_bounds__(kWave) void probe_gather_kernel(const uint8_t* __restrict__ base,
                                                             const int32_t* __restrict__ ids,
                                                             int32_t per_wave,
                                                             uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x;
  const int32_t* my = ids + int64_t(blockIdx.x) * per_wave;
  uint32_t acc = 0;
  for (int i = 0; i < per_wave; i += 2) {
    uint4 v[2][LOADS];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t c = my[min(i + u, per_wave - 1)];
#pragma unroll
      for (int l = 0; l < LOADS; ++l)
      {
        const uint8_t* a = base + c * (LOADS * 1024) + l * 1024 + lane * 16;
        if constexpr (NT) {
          const Vec16 w = load16_stream(a);
          v[u][l] = uint4{w.w[0], w.w[1], w.w[2], w.w[3]};
        } else {
          v[u][l] = *reinterpret_cast<const uint4*>(a);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int l = 0; l < LOADS; ++l) acc ^= v[u][l].x ^ v[u][l].y ^ v[u][l].z ^ v[u][l].w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace
}  // namespace edgerag

using namespace edgerag;

extern "C" int edgerag_probe_read(const void* src, int64_t bytes, int32_t workgroups,
                                  int32_t unroll, void* sink, void* stream) {
  clear_error();
  if (src == nullptr || sink == nullptr || bytes <= 0 || bytes % 16 != 0 || workgroups <= 0 ||
      !aligned16(src))
    return fail(EDGERAG_EINVAL, "edgerag_probe_read: bad arguments");
  auto s = static_cast<hipStream_t>(stream);
  const auto* p = static_cast<const uint4*>(src);
  auto* out = static_cast<uint32_t*>(sink);
  switch (unroll) {
    case 1: hipLaunchKernelGGL(probe_read_kernel<1>, dim3(workgroups), dim3(kProbeThreads), 0, s, p, bytes / 16, out); break;
    case 2: hipLaunchKernelGGL(probe_read_kernel<2>, dim3(workgroups), dim3(kProbeThreads), 0, s, p, bytes / 16, out); break;
    case 4: hipLaunchKernelGGL(probe_read_kernel<4>, dim3(workgroups), dim3(kProbeThreads), 0, s, p, bytes / 16, out); break;
    default: return fail(EDGERAG_EINVAL, "edgerag_probe_read: unroll %d (1, 2 or 4)", unroll);
  }
  return check_launch("edgerag_probe_read");
}

extern "C" int edgerag_probe_gather(const void* base, const int32_t* chunk_ids, int32_t waves,
                                    int32_t per_wave, int32_t chunk_bytes, int32_t nontemporal,
                                    void* sink, void* stream) {
  clear_error();
  if (base == nullptr || chunk_ids == nullptr || sink == nullptr || waves <= 0 || per_wave <= 0 ||
      !aligned16(base))
    return fail(EDGERAG_EINVAL, "edgerag_probe_gather: bad arguments");
  auto s = static_cast<hipStream_t>(stream);
  const auto* b = static_cast<const uint8_t*>(base);
  auto* out = static_cast<uint32_t*>(sink);
#define EDGERAG_GATHER(L)                                                                       \
  do {                                                                                         \
    if (nontemporal)                                                                           \
      hipLaunchKernelGGL((probe_gather_kernel<L, true>), dim3(waves), dim3(kWave), 0, s, b,    \
                         chunk_ids, per_wave, out);                                            \
    else                                                                                       \
      hipLaunchKernelGGL((probe_gather_kernel<L, false>), dim3(waves), dim3(kWave), 0, s, b,   \
                         chunk_ids, per_wave, out);                                            \
  } while (0)
  switch (chunk_bytes) {
    case 1024: EDGERAG_GATHER(1); break;
    case 2048: EDGERAG_GATHER(2); break;
    case 4096: EDGERAG_GATHER(4); break;
    default: return fail(EDGERAG_EINVAL, "edgerag_probe_gather: chunk_bytes %d (1, 2 or 4 KiB)", chunk_bytes);
  }
#undef EDGERAG_GATHER
  return check_launch("edgerag_probe_gather");
}
