// llmk_read_probe.hip — the box's achievable streaming-read bandwidth, for
// the benchmark's report: every lane reads 128-bit words with non-temporal
// loads (the access pattern of the sampler's tile loads) and sums them, one
// atomic add per workgroup.  Not part of the sampler's interface.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f4v __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(1024) void read_probe_kernel(const f4v* __restrict__ x, uint64_t n4,
                                                          float* __restrict__ out) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  float acc = 0.0f;
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n4; i += 4 * stride) {
    const f4v a = __builtin_nontemporal_load(x + i);
    const f4v b = __builtin_nontemporal_load(x + i + stride);
    const f4v c = __builtin_nontemporal_load(x + i + 2 * stride);
    const f4v d = __builtin_nontemporal_load(x + i + 3 * stride);
    acc += ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w)) +
           ((c.x + c.y) + (c.z + c.w)) + ((d.x + d.y) + (d.z + d.w));
  }
  for (; i < n4; i += stride) {
    const f4v a = __builtin_nontemporal_load(x + i);
    acc += (a.x + a.y) + (a.z + a.w);
  }
  __shared__ float red[16];
  for (int o = 32; o > 0; o >>= 1) acc += __shfl_down(acc, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float s = 0.0f;
    for (int k = 0; k < (int)(blockDim.x >> 6); ++k) s += red[k];
    atomicAdd(out, s);
  }
}

// Reads nbytes (a multiple of 16) at x once; out: one float, accumulated.
// Returns 0, or the HIP error code.
extern "C" int llmk_read_probe(const void* x, uint64_t nbytes, float* out, uint32_t blocks,
                               void* stream) {
  hipLaunchKernelGGL(read_probe_kernel, dim3(blocks), dim3(1024), 0, (hipStream_t)stream,
                     (const f4v*)x, nbytes / 16, out);
  return (int)hipGetLastError();
}
