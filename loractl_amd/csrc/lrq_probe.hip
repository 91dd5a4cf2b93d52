// A streaming read of device memory, the measured ceiling against which the
// few-token kernels' HBM rates are read: every byte of a buffer is loaded
// once with 16-byte loads, eight in flight per lane, and folded into one
// value per workgroup so the loads stay live. It has no counterpart in the
// reference; it is measurement infrastructure (lrq_probe_stream_read).

#include "lrq_common.h"
#include "lrq_kernels.h"

namespace {

constexpr int PR_NT = 256;   // threads per workgroup
constexpr int PR_UNROLL = 8; // 16-byte loads in flight per lane

// Workgroup b reads the 16-byte words [b * per, min((b + 1) * per, n16)),
// lane-interleaved so each load instruction covers 4 KiB of contiguous
// memory, and writes the XOR of everything it read to out[b].
__global__ void __launch_bounds__(PR_NT) k_stream_read(const u32x4* __restrict__ p, int64_t n16, int64_t per,
                                                        uint32_t* __restrict__ out) {
  const int64_t b0 = (int64_t)blockIdx.x * per;
  const int64_t end = b0 + per < n16 ? b0 + per : n16;
  uint32_t acc = 0;
  for (int64_t i = b0 + threadIdx.x; i < end; i += (int64_t)PR_NT * PR_UNROLL) {
    u32x4 v[PR_UNROLL];
#pragma unroll
    for (int u = 0; u < PR_UNROLL; ++u) {
      const int64_t j = i + (int64_t)u * PR_NT;
      v[u] = j < end ? __builtin_nontemporal_load(p + j) : zero4();
    }
#pragma unroll
    for (int u = 0; u < PR_UNROLL; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  // one value per workgroup: the lanes' values folded through LDS
  __shared__ uint32_t red[PR_NT];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int s = PR_NT / 2; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) red[threadIdx.x] ^= red[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) out[blockIdx.x] = red[0];
}

}  // namespace

// One full round of loads per lane at least (2048 words per workgroup), at
// most eight workgroups per CU.
int probe_read_grid(int64_t bytes) {
  const int64_t n16 = bytes / 16, cap = 8 * (int64_t)get_num_cus();
  const int64_t g = (n16 + PR_NT * PR_UNROLL - 1) / (PR_NT * PR_UNROLL);
  return (int)(g < 1 ? 1 : (g > cap ? cap : g));
}

hipError_t launch_stream_read(hipStream_t st, const void* data, int64_t bytes, uint32_t* out) {
  const int64_t n16 = bytes / 16;
  if (n16 <= 0) return hipSuccess;
  const int grid = probe_read_grid(bytes);
  const int64_t per = (n16 + grid - 1) / grid;
  hipLaunchKernelGGL(k_stream_read, dim3(grid), dim3(PR_NT), 0, st, reinterpret_cast<const u32x4*>(data), n16, per,
                     out);
  return hipGetLastError();
}
