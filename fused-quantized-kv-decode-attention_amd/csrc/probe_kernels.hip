// Streaming-read probe: the ceiling the decode kernels are measured against.
//
// A decode call at batch 1 reads its KV cache once and writes almost
// nothing, so the fastest it could possibly run is a kernel that only reads
// the same number of bytes. stream_read_kernel gives each workgroup one
// contiguous span of the source (the way the decode kernels give each
// workgroup one contiguous KV tile) and reads it with 16-byte non-temporal
// loads, 8 in flight per lane, folding them into one word that is stored
// only if it equals an impossible value (so the loads cannot be optimised
// away). bench.py times it on the same number of bytes per call as the
// headline workload.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "launch.h"

namespace fqkv {

typedef uint32_t p4_t __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256) stream_read_kernel(const p4_t* __restrict__ src, size_t n16, size_t span,
                                                          uint32_t* sink) {
  constexpr int U = 8, T = 256;
  const size_t begin = (size_t)blockIdx.x * span;
  const size_t end = begin + span < n16 ? begin + span : n16;
  uint32_t acc = 0;
  size_t i = begin + threadIdx.x;
  for (; i + (U - 1) * T < end; i += U * T) {
    p4_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(src + i + u * T);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < end; i += T) {
    const p4_t v = __builtin_nontemporal_load(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9E3779B9u && sink) sink[blockIdx.x] = acc;
}

// Range-check probe: what a raw buffer load returns past its descriptor's
// num_records, depending on which part of the offset points there. The
// kernels rely on zeros for offsets past the end carried in the VGPR offset
// or the instruction's immediate offset; the probe records those cases, the
// SGPR offset, and a 16-byte load that straddles the end. The descriptor
// covers the first `records` bytes of a buffer at least records + 64 bytes
// long, so every access stays inside the allocation whatever the answer.
// out[0]: offset records - 4 (in range); out[1]: VGPR offset records;
// out[2]: VGPR records - 4 + SGPR 16; out[3]: VGPR 0 + SGPR records;
// out[4]: VGPR records - 4 + immediate 16; out[5..8]: 16 bytes at
// records - 8.
__global__ void buffer_range_kernel(const uint32_t* buf, int records, uint32_t* out, int zero) {
  if (threadIdx.x != 0) return;
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(buf), (short)0, records, 0x00020000);
  const int last = records - 4;
  out[0] = __builtin_amdgcn_raw_buffer_load_b32(r, last, zero, 0);
  out[1] = __builtin_amdgcn_raw_buffer_load_b32(r, records, zero, 0);
  out[2] = __builtin_amdgcn_raw_buffer_load_b32(r, last, zero + 16, 0);
  out[3] = __builtin_amdgcn_raw_buffer_load_b32(r, zero, records, 0);
  out[4] = __builtin_amdgcn_raw_buffer_load_b32(r, last + 16, zero, 0);  // the 16 goes to the immediate field
  const p4_t v = __builtin_bit_cast(p4_t, __builtin_amdgcn_raw_buffer_load_b128(r, records - 8, zero, 0));
  out[5] = v.x;
  out[6] = v.y;
  out[7] = v.z;
  out[8] = v.w;
}

hipError_t launch_buffer_range(const void* buf, int records, uint32_t* out, hipStream_t st) {
  hipLaunchKernelGGL(buffer_range_kernel, dim3(1), dim3(64), 0, st, (const uint32_t*)buf, records, out, 0);
  return hipGetLastError();
}

hipError_t launch_stream_read(const void* src, size_t bytes, uint32_t* sink, int blocks, hipStream_t st) {
  if (!src || bytes % 16 || blocks < 1) return hipErrorInvalidValue;
  const size_t n16 = bytes / 16, span = (n16 + blocks - 1) / blocks;
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, st, (const p4_t*)src, n16, span, sink);
  return hipGetLastError();
}

}  // namespace fqkv
