// Measurement helpers: a cache-eviction sweep run on the timed stream before
// each measured launch, the gfx950 counterpart of the reference's L2 eviction
// (benchmarks/cache.py:13-92, benchmarks/cache_sweep.py:15-32). MI355X has a
// 4 MiB L2 per XCD and a 256 MiB Infinity Cache, so callers pass a buffer of
// at least 1 GiB. And a shader-clock probe, so that a benchmark can state the
// clock its kernels ran at.
#include "common.h"
#include "../../include/ascendflow_amd.h"

namespace afa {

__global__ __launch_bounds__(256) void cache_flush_kernel(const u32x4* buf, uint64_t n16,
                                                          uint32_t* sink) {
  uint32_t acc = 0;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
    const u32x4 v = buf[i];  // cached load: displaces what the caches held
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  // Never true for the zero-filled buffers callers use; keeps the reads live.
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

// Every thread runs `spins` dependent FMAs (all SIMDs busy, so the clock is
// the one a loaded GPU runs at); thread 0 of workgroup 0 reads the
// shader-cycle counter and the 100 MHz real-time counter before and after.
__global__ __launch_bounds__(256) void clock_probe_kernel(uint64_t* out, int spins) {
  const uint64_t c0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  float x = (float)threadIdx.x;
  for (int i = 0; i < spins; ++i) x = __builtin_fmaf(x, 1.0000001f, 0.5f);
  const uint64_t c1 = __builtin_amdgcn_s_memtime();
  const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    out[0] = c0;
    out[1] = c1;
    out[2] = r0;
    out[3] = r1;
  }
  if (x == -1.0f) out[4] = 0;  // never true; keeps the chain live
}

}  // namespace afa

extern "C" int launch_clock_probe(void* stream, uint64_t* out, int32_t spins) {
  if (!out) return AFA_E_NULL;
  if (spins <= 0) return AFA_E_SHAPE;
  hipLaunchKernelGGL(afa::clock_probe_kernel, dim3(1024), dim3(256), 0, (hipStream_t)stream, out, (int)spins);
  return (int)hipGetLastError();
}

extern "C" int launch_cache_flush(void* stream, void* buffer, uint64_t bytes) {
  if (!buffer) return AFA_E_NULL;
  const uint64_t n16 = bytes / 16;
  if (n16 == 0) return AFA_OK;
  hipLaunchKernelGGL(afa::cache_flush_kernel, dim3(4096), dim3(256), 0, (hipStream_t)stream,
                     (const afa::u32x4*)buffer, n16, (uint32_t*)buffer);
  return (int)hipGetLastError();
}

extern "C" const char* ascendflow_amd_version(void) { return "ascendflow_amd 0.1 gfx950"; }
