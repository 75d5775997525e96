// Read-only HBM streaming probe (include/wr_probe.h): the achievable read
// bandwidth for a given set of byte ranges, measured with the access pattern
// a streaming kernel can reach at best -- each wave reads 1 KB contiguous per
// load instruction, U loads in flight per lane, non-temporal -- and the rate
// of two gate/up read orders over the same experts' bytes.
#include <hip/hip_runtime.h>

#include <stdint.h>

#include "wr_probe.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct Ranges {
  const u32x4* p[WR_PROBE_MAX_RANGES];
  int64_t n[WR_PROBE_MAX_RANGES];  // 16-byte vectors
  int count;
};

template <int U>
__global__ __launch_bounds__(256) void k_probe_read(Ranges r, uint32_t* sink) {
  u32x4 acc = {0u, 0u, 0u, 0u};
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int i = 0; i < r.count; ++i) {
    const u32x4* p = r.p[i];
    const int64_t n = r.n[i];
    int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    for (; j + (U - 1) * stride < n; j += U * stride) {
      u32x4 v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(p + j + u * stride);
#pragma unroll
      for (int u = 0; u < U; ++u) acc ^= v[u];
    }
    for (; j < n; j += stride) acc ^= __builtin_nontemporal_load(p + j);
  }
  if (acc[0] == 0x9e3779b9u && acc[1] == 0x7f4a7c15u && acc[2] == 0x85ebca6bu &&
      acc[3] == 0xc2b2ae35u)
    sink[0] = acc[0] ^ acc[3];
}

// An opaque zero that depends on v, so that a round's load addresses wait
// for the previous round's data, as a kernel's next round waits for its
// arithmetic.
__device__ __forceinline__ int dep_zero(uint32_t v) {
  int z;
  asm volatile("v_and_b32 %0, 0, %1" : "=v"(z) : "v"(v));
  return z;
}

struct Experts {
  const unsigned char* p[WR_PROBE_MAX_EXPERTS];
};

__device__ __forceinline__ u32x4 ld16(const unsigned char* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Pattern 0: the single-token kernel's gate/up slots (8 rows, wave w rows
// 2w and 2w + 1 of gate and up), NR rounds of four 1 KB loads per row.
template <int NR>
__global__ __launch_bounds__(256) void k_probe_slots(Experts ex, int64_t rowb, int I, int nslots,
                                                     uint32_t* sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int spe = I / 8;
  u32x4 acc = {0u, 0u, 0u, 0u};
  int z = 0;
  for (int v = blockIdx.x; v < nslots; v += gridDim.x) {
    const int e = v / spe;
    const unsigned char* G = ex.p[e] + (int64_t)((v - e * spe) * 8 + 2 * wave) * rowb;
    const unsigned char* U = G + (int64_t)I * rowb;
    for (int rd = 0; rd < NR; ++rd) {
      u32x4 a[16];
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int64_t o = j * rowb + (rd * 4 + u) * 1024 + lane * 16 + z;
          a[8 * j + u] = ld16(G + o);
          a[8 * j + 4 + u] = ld16(U + o);
        }
#pragma unroll
      for (int i = 0; i < 16; ++i) acc ^= a[i];
      z = dep_zero(acc[0]);
    }
  }
  if (acc[0] == 0x9e3779b9u && acc[1] == 0x7f4a7c15u && acc[2] == 0x85ebca6bu &&
      acc[3] == 0xc2b2ae35u)
    sink[0] = acc[0] ^ acc[3] ^ (uint32_t)z;
}

// Pattern 1: workgroup-level grid stride over 4-row groups of gate and up;
// wave w reads the w-th quarter of each row (CW 1 KB loads), one round per
// group.
template <int CW>
__global__ __launch_bounds__(256) void k_probe_rows(Experts ex, int64_t rowb, int I, int nrows,
                                                    uint32_t* sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  u32x4 acc = {0u, 0u, 0u, 0u};
  int z = 0;
  for (int r0 = blockIdx.x * 4; r0 < nrows; r0 += gridDim.x * 4) {
    u32x4 a[8 * CW];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = r0 + j, e = r / I;
      const unsigned char* G = ex.p[e] + (int64_t)(r - e * I) * rowb;
      const unsigned char* U = G + (int64_t)I * rowb;
#pragma unroll
      for (int u = 0; u < CW; ++u) {
        const int64_t o = (wave * CW + u) * 1024 + lane * 16 + z;
        a[2 * CW * j + u] = ld16(G + o);
        a[2 * CW * j + CW + u] = ld16(U + o);
      }
    }
#pragma unroll
    for (int i = 0; i < 8 * CW; ++i) acc ^= a[i];
    z = dep_zero(acc[0]);
  }
  if (acc[0] == 0x9e3779b9u && acc[1] == 0x7f4a7c15u && acc[2] == 0x85ebca6bu &&
      acc[3] == 0xc2b2ae35u)
    sink[0] = acc[0] ^ acc[3] ^ (uint32_t)z;
}

// Down, pattern 0: the single-token kernel's order (see wr_probe_down).
__global__ __launch_bounds__(256) void k_probe_down_kernel(Experts ex, int nexp, int64_t rowb, int h,
                                                           uint32_t* sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = (int)((rowb + 1023) / 1024), C = nexp * nch;
  u32x4 acc = {0u, 0u, 0u, 0u};
  int z = 0;
  for (int r0 = blockIdx.x * 4; r0 < h; r0 += gridDim.x * 4) {
    for (int q0 = wave; q0 < C; q0 += 16) {
      u32x4 a[16];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int q = q0 + 4 * u;
        const int e = q < C ? q / nch : 0;
        const int col = (q - e * nch) * 1024 + lane * 16;  // byte in the row
        const bool ok = q < C && col < rowb;
        const unsigned char* D = ex.p[e] + (int64_t)r0 * rowb + col + z;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          a[4 * u + j] = ok ? ld16(D + j * rowb) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) acc ^= a[i];
      z = dep_zero(acc[0]);
    }
  }
  if (acc[0] == 0x9e3779b9u && acc[1] == 0x7f4a7c15u && acc[2] == 0x85ebca6bu &&
      acc[3] == 0xc2b2ae35u)
    sink[0] = acc[0] ^ acc[3] ^ (uint32_t)z;
}

// Down, pattern 1: wave w reads row w of the group, 16 consecutive 1 KB loads
// per round over the concatenation of the experts' rows.
__global__ __launch_bounds__(256) void k_probe_down_rows(Experts ex, int nexp, int64_t rowb, int h,
                                                         uint32_t* sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = (int)((rowb + 1023) / 1024), C = nexp * nch;
  u32x4 acc = {0u, 0u, 0u, 0u};
  int z = 0;
  for (int r0 = blockIdx.x * 4; r0 < h; r0 += gridDim.x * 4) {
    for (int q0 = 0; q0 < C; q0 += 16) {
      u32x4 a[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int q = q0 + u;
        const int e = q < C ? q / nch : 0;
        const int col = (q - e * nch) * 1024 + lane * 16;
        a[u] = (q < C && col < rowb) ? ld16(ex.p[e] + (int64_t)(r0 + wave) * rowb + col + z)
                                     : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) acc ^= a[i];
      z = dep_zero(acc[0]);
    }
  }
  if (acc[0] == 0x9e3779b9u && acc[1] == 0x7f4a7c15u && acc[2] == 0x85ebca6bu &&
      acc[3] == 0xc2b2ae35u)
    sink[0] = acc[0] ^ acc[3] ^ (uint32_t)z;
}

int cu_count() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    return 256;
  return n;
}

}  // namespace

extern "C" WR_PROBE_API int wr_probe_read(const void* const* ptrs, const int64_t* bytes,
                                          int n_ranges, int blocks_per_cu, int unroll,
                                          uint32_t* sink, void* stream) {
  if (ptrs == nullptr || bytes == nullptr || sink == nullptr) return -1;
  if (n_ranges < 1 || n_ranges > WR_PROBE_MAX_RANGES) return -1;
  if (blocks_per_cu < 1 || blocks_per_cu > 64) return -1;
  if (unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8) return -1;
  Ranges r{};
  r.count = n_ranges;
  for (int i = 0; i < n_ranges; ++i) {
    if (ptrs[i] == nullptr || bytes[i] < 0 || bytes[i] % 16 != 0 ||
        reinterpret_cast<uintptr_t>(ptrs[i]) % 16 != 0)
      return -1;
    r.p[i] = static_cast<const u32x4*>(ptrs[i]);
    r.n[i] = bytes[i] / 16;
  }
  const dim3 grid(blocks_per_cu * cu_count());
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (unroll) {
    case 1: hipLaunchKernelGGL(k_probe_read<1>, grid, dim3(256), 0, s, r, sink); break;
    case 2: hipLaunchKernelGGL(k_probe_read<2>, grid, dim3(256), 0, s, r, sink); break;
    case 4: hipLaunchKernelGGL(k_probe_read<4>, grid, dim3(256), 0, s, r, sink); break;
    default: hipLaunchKernelGGL(k_probe_read<8>, grid, dim3(256), 0, s, r, sink); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

extern "C" WR_PROBE_API int wr_probe_gateup(const void* const* experts, int n_experts,
                                            int64_t row_bytes, int I, int pattern, int blocks,
                                            uint32_t* sink, void* stream) {
  if (experts == nullptr || sink == nullptr) return -1;
  if (n_experts < 1 || n_experts > WR_PROBE_MAX_EXPERTS) return -1;
  if ((row_bytes != 4096 && row_bytes != 8192) || I < 8 || I % 8 != 0) return -1;
  if ((pattern != 0 && pattern != 1) || blocks < 1) return -1;
  Experts ex{};
  for (int i = 0; i < n_experts; ++i) {
    if (experts[i] == nullptr || reinterpret_cast<uintptr_t>(experts[i]) % 16 != 0) return -1;
    ex.p[i] = static_cast<const unsigned char*>(experts[i]);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(blocks), block(256);
  if (pattern == 0) {
    const int nslots = n_experts * (I / 8);
    if (row_bytes == 4096)
      hipLaunchKernelGGL(k_probe_slots<1>, grid, block, 0, s, ex, row_bytes, I, nslots, sink);
    else
      hipLaunchKernelGGL(k_probe_slots<2>, grid, block, 0, s, ex, row_bytes, I, nslots, sink);
  } else {
    const int nrows = n_experts * I;
    if (row_bytes == 4096)
      hipLaunchKernelGGL(k_probe_rows<1>, grid, block, 0, s, ex, row_bytes, I, nrows, sink);
    else
      hipLaunchKernelGGL(k_probe_rows<2>, grid, block, 0, s, ex, row_bytes, I, nrows, sink);
  }
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

extern "C" WR_PROBE_API int wr_probe_down(const void* const* down, int n_experts, int64_t row_bytes,
                                          int h, int pattern, int blocks, uint32_t* sink,
                                          void* stream) {
  if (down == nullptr || sink == nullptr) return -1;
  if (n_experts < 1 || n_experts > WR_PROBE_MAX_EXPERTS) return -1;
  if (row_bytes < 16 || row_bytes > 65536 || row_bytes % 16 != 0) return -1;
  if (h < 4 || h % 4 != 0 || (pattern != 0 && pattern != 1) || blocks < 1) return -1;
  Experts ex{};
  for (int i = 0; i < n_experts; ++i) {
    if (down[i] == nullptr || reinterpret_cast<uintptr_t>(down[i]) % 16 != 0) return -1;
    ex.p[i] = static_cast<const unsigned char*>(down[i]);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (pattern == 0)
    hipLaunchKernelGGL(k_probe_down_kernel, dim3(blocks), dim3(256), 0, s, ex, n_experts, row_bytes,
                       h, sink);
  else
    hipLaunchKernelGGL(k_probe_down_rows, dim3(blocks), dim3(256), 0, s, ex, n_experts, row_bytes,
                       h, sink);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}
