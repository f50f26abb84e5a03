// Memory-system probes of libmuspace_probes.so (bench.py --gather-probe,
// --atomic-probe, --lds-atomic-probe). They measure the ceilings the MSDA
// kernels are priced against on MI355X and are not part of the MSDA library:
//
//   gather      random 128-byte line reads, 16 bytes per lane (8 lanes per
//               line), the rate of the forward's corner-row gathers;
//   atomic      line-wide fp32 atomic adds (32 lanes on one 128-byte line),
//               the rate of a reference-style atomic grad_value scatter;
//   lds atomic  fp32 (ds_add_f32) and u32 (ds_add_u32) atomic adds to LDS,
//               bank-conflict-free or scattered addresses, the rate an
//               LDS-accumulated grad_value would run at;
//   scatter     a 4-byte and an 8-byte store per record to random records of
//               two arrays, the tile backward's direct location and weight
//               gradient writes.
//
// Each workgroup works in the region of the XCD it runs on (hardware
// register XCC_ID), so `lines` per XCD sets the footprint one L2 sees.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kProbeBlock = 256;

__device__ __forceinline__ uint32_t mix(uint32_t x) {
  x *= 0x9E3779B1u;
  x ^= x >> 15;
  x *= 0x85EBCA77u;
  x ^= x >> 13;
  return x;
}

__device__ __forceinline__ uint32_t xcd_id() {
  // s_getreg of HW_REG_XCC_ID (register 20), bits [3:0]
  return static_cast<uint32_t>(__builtin_amdgcn_s_getreg((3 << 11) | 20)) & 7u;
}

__global__ void __launch_bounds__(kProbeBlock)
    probe_gather(const float *__restrict__ buf, uint32_t lines, int iters,
                 float *__restrict__ sink) {
  const float *region = buf + static_cast<size_t>(xcd_id()) * lines * 32;
  const uint32_t lane = threadIdx.x & 63u, group = lane >> 3, part = (lane & 7u) * 4;
  const uint32_t wave = blockIdx.x * (kProbeBlock / 64) + threadIdx.x / 64;
  // kInFlight independent loads per step, so the rate is a throughput and
  // not one load's round-trip latency
  constexpr int kInFlight = 8;
  float acc = 0.0f;
  for (int it = 0; it < iters; it += kInFlight) {
    float4 v[kInFlight];
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) {
      const uint32_t step = static_cast<uint32_t>(it + u);
      const uint32_t line = mix(wave * 8u + group + 0x632BE5ABu * step) % lines;
      v[u] = *reinterpret_cast<const float4 *>(region + static_cast<size_t>(line) * 32 + part);
    }
#pragma unroll
    for (int u = 0; u < kInFlight; ++u) acc += (v[u].x + v[u].y) + (v[u].z + v[u].w);
  }
  sink[blockIdx.x * kProbeBlock + threadIdx.x] = acc;
}

__global__ void __launch_bounds__(kProbeBlock)
    probe_atomic(float *__restrict__ buf, uint32_t lines, int iters) {
  float *region = buf + static_cast<size_t>(xcd_id()) * lines * 32;
  const uint32_t lane = threadIdx.x & 63u, half = lane >> 5, c = lane & 31u;
  const uint32_t wave = blockIdx.x * (kProbeBlock / 64) + threadIdx.x / 64;
  for (int it = 0; it < iters; ++it) {
    const uint32_t line = mix(wave * 2u + half + 0x632BE5ABu * static_cast<uint32_t>(it)) % lines;
    __hip_atomic_fetch_add(region + static_cast<size_t>(line) * 32 + c, 1.0f, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Scattered records: every lane stores a 4-byte and an 8-byte value to a
// random record of its XCD's region (`records` records of each array) per
// step, so the footprint one L2 sees is records * 12 bytes.
__global__ void __launch_bounds__(kProbeBlock)
    probe_scatter12(float *__restrict__ ga, float2 *__restrict__ gl, uint32_t records, int iters) {
  const size_t x = xcd_id();
  float *ra = ga + x * records;
  float2 *rl = gl + x * records;
  const uint32_t t = blockIdx.x * kProbeBlock + threadIdx.x;
  for (int it = 0; it < iters; ++it) {
    const uint32_t r = mix(t + 0x632BE5ABu * static_cast<uint32_t>(it)) % records;
    ra[r] = 1.0f;
    rl[r] = make_float2(2.0f, 3.0f);
  }
}

// kind bit 0: u32 (else fp32) adds; bit 1: scattered (else consecutive,
// bank-conflict-free) addresses. Every index is masked into the 8192-word
// array; out[] gets one word per thread.
template <typename T>
__device__ __forceinline__ void lds_atomic_body(T *out, int iters, bool scattered) {
  __shared__ T s[8192];
  for (int i = threadIdx.x; i < 8192; i += blockDim.x) s[i] = T(0);
  __syncthreads();
  const uint32_t t = threadIdx.x;
  for (int it = 0; it < iters; ++it) {
    const uint32_t a = scattered ? mix(t * 8191u + static_cast<uint32_t>(it)) & 8191u
                                 : (t + 97u * static_cast<uint32_t>(it)) & 8191u;
    atomicAdd(&s[a], T(1));
  }
  __syncthreads();
  out[blockIdx.x * blockDim.x + threadIdx.x] = s[t];
}

// 64-bit integer adds (ds_add_u64) into an 8192-entry array (64 KB); out[]
// gets the low word of one entry per thread.
__global__ void __launch_bounds__(1024)
    probe_lds_atomic64(uint32_t *out, int iters, bool scattered) {
  __shared__ unsigned long long s[8192];
  for (int i = threadIdx.x; i < 8192; i += blockDim.x) s[i] = 0ull;
  __syncthreads();
  const uint32_t t = threadIdx.x;
  for (int it = 0; it < iters; ++it) {
    const uint32_t a = scattered ? mix(t * 8191u + static_cast<uint32_t>(it)) & 8191u
                                 : (t + 97u * static_cast<uint32_t>(it)) & 8191u;
    atomicAdd(&s[a], 1ull);
  }
  __syncthreads();
  out[blockIdx.x * blockDim.x + threadIdx.x] = static_cast<uint32_t>(s[t]);
}

__global__ void __launch_bounds__(1024) probe_lds_atomic(uint32_t *out, int iters, int kind) {
  if (kind & 1) {
    lds_atomic_body<uint32_t>(out, iters, (kind & 2) != 0);
  } else {
    lds_atomic_body<float>(reinterpret_cast<float *>(out), iters, (kind & 2) != 0);
  }
}

bool bad_args(const void *buf, uint64_t lines, int blocks, int iters) {
  return buf == nullptr || lines == 0 || lines > (uint64_t{1} << 26) || blocks <= 0 ||
         iters <= 0;
}

}  // namespace

extern "C" {

// buf: 8 * lines * 128 bytes; sink: blocks * 256 floats; iters a multiple of
// 8 (each lane reads iters 16-byte pieces). Returns a hipError_t.
__attribute__((visibility("default"))) int muspace_probe_gather(const float *buf, uint64_t lines,
                                                                int blocks, int iters, float *sink,
                                                                void *stream) {
  if (bad_args(buf, lines, blocks, iters) || sink == nullptr || iters % 8 != 0) {
    return hipErrorInvalidValue;
  }
  probe_gather<<<blocks, kProbeBlock, 0, static_cast<hipStream_t>(stream)>>>(
      buf, static_cast<uint32_t>(lines), iters, sink);
  return hipGetLastError();
}

// buf: 8 * lines * 128 bytes (each element gains blocks*256*iters / (8*lines*32)
// on average). Returns a hipError_t.
__attribute__((visibility("default"))) int muspace_probe_atomic(float *buf, uint64_t lines,
                                                                int blocks, int iters,
                                                                void *stream) {
  if (bad_args(buf, lines, blocks, iters)) return hipErrorInvalidValue;
  probe_atomic<<<blocks, kProbeBlock, 0, static_cast<hipStream_t>(stream)>>>(
      buf, static_cast<uint32_t>(lines), iters);
  return hipGetLastError();
}

// blocks workgroups of 1024 threads, each thread `iters` LDS atomic adds
// (kind 0-3 as probe_lds_atomic; 5 and 7: 64-bit integer adds, consecutive
// and scattered); out: blocks * 1024 words. Returns a hipError_t.
__attribute__((visibility("default"))) int muspace_probe_lds_atomic(uint32_t *out, int blocks,
                                                                    int iters, int kind,
                                                                    void *stream) {
  if (out == nullptr || blocks <= 0 || iters <= 0 || kind < 0 || kind > 7 || kind == 4 ||
      kind == 6) {
    return hipErrorInvalidValue;
  }
  if (kind & 4) {
    probe_lds_atomic64<<<blocks, 1024, 0, static_cast<hipStream_t>(stream)>>>(out, iters,
                                                                              (kind & 2) != 0);
  } else {
    probe_lds_atomic<<<blocks, 1024, 0, static_cast<hipStream_t>(stream)>>>(out, iters, kind);
  }
  return hipGetLastError();
}

// ga: 8 * records floats, gl: 8 * records float2; each lane stores iters
// records. Returns a hipError_t.
__attribute__((visibility("default"))) int muspace_probe_scatter(float *ga, void *gl,
                                                                 uint64_t records, int blocks,
                                                                 int iters, void *stream) {
  if (ga == nullptr || gl == nullptr || records == 0 || records > (1u << 28) || blocks <= 0 ||
      iters <= 0) {
    return hipErrorInvalidValue;
  }
  probe_scatter12<<<blocks, kProbeBlock, 0, static_cast<hipStream_t>(stream)>>>(
      ga, static_cast<float2 *>(gl), static_cast<uint32_t>(records), iters);
  return hipGetLastError();
}

}  // extern "C"
