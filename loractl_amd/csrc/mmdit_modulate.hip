// Modulated RMSNorm, gated residual and the MLP's GELU of a double-stream
// MMDiT block, the elementwise glue around its fused linears:
//
//   h = (scale + 1) * x / sqrt(mean(x^2) + eps) + shift      (per row of x)
//   y = x + gate * o
//   g = gelu_tanh(u) = u / (1 + exp(-2 c (u + 0.044715 u^3))), c = sqrt(2/pi)
//
// with scale, shift and gate one [h] vector per block (the modulation
// linear's output). Forwards and gradients are HIP kernels here. The
// residual's forward and GELU are flat streams of 16-byte chunks (y: 6
// bytes per element; GELU 4, its gradient 6).
//
// A row is one wavefront: lane l takes the 16-byte chunks l, l + 64, ... of
// the row, so the row's sum is a 64-lane reduction and every load and store
// is 16 bytes. The vector gradients (d scale, d shift, d gate) are column
// sums over all rows: each workgroup sums its own rows (its four wavefronts
// meet in LDS in a fixed order) into one f32 partial row, and a second
// launch sums the partial rows in order, so the results are bitwise
// reproducible. HBM-bound: norm forward reads and writes the row once (4h
// bytes per row), its gradient reads dh and x and writes dx (6h), the
// residual's gradient reads dy and o and writes do (6h).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "loractl_mmdit.h"

extern __attribute__((visibility("hidden"))) thread_local std::string lmd_err_msg;  // lmd_last_error's message (mmdit_attn_prep.hip)

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

#define LMD_DEV __device__ __forceinline__

constexpr int MAX_CPL = 8;  // 16-byte chunks per lane: h <= 4096
constexpr int GROUPS = 256; // partial rows of a column sum, at most (one wavefront per SIMD)

LMD_DEV uint32_t pack2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
LMD_DEV void unpack8(const u32x4& w, float f[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __builtin_bit_cast(float, w[i] << 16);
    f[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xffff0000u);
  }
}
LMD_DEV u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
LMD_DEV void st16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }
LMD_DEV float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

struct ModArgs {
  int64_t rows;
  int h;
  int rpw;  // rows per workgroup (gradients)
  float eps;
  const uint16_t* x;      // norm input / residual branch o
  const uint16_t* vec0;   // scale / gate [h]
  const uint16_t* vec1;   // shift [h]
  const uint16_t* grad;   // dh / dy
  const float* rstd_in;
  uint16_t* out;          // h / dx / do
  float* rstd_out;
  float* part;            // [groups][nsum][h]
  uint16_t* vout0;        // d scale / d gate [h]
  uint16_t* vout1;        // d shift [h]
};

template <int CPL>
__global__ __launch_bounds__(256) void k_modnorm_fwd(ModArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;  // whole wavefronts leave
  const int C = a.h / 8;
  const uint16_t* xr = a.x + row * a.h;
  u32x4 xv[CPL];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    xv[j] = c < C ? ld16(xr + c * 8) : (u32x4){0u, 0u, 0u, 0u};
    float f[8];
    unpack8(xv[j], f);
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(f[e], f[e], ss);
  }
  const float r = rsqrtf(wave_sum(ss) / (float)a.h + a.eps);
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = lane + 64 * j;
    if (c >= C) continue;
    float f[8], s[8], t[8];
    unpack8(xv[j], f);
    unpack8(ld16(a.vec0 + c * 8), s);
    unpack8(ld16(a.vec1 + c * 8), t);
    u32x4 y;
#pragma unroll
    for (int p = 0; p < 4; ++p)
      y[p] = pack2(__builtin_fmaf(f[2 * p] * r, s[2 * p] + 1.0f, t[2 * p]),
                   __builtin_fmaf(f[2 * p + 1] * r, s[2 * p + 1] + 1.0f, t[2 * p + 1]));
    st16(a.out + row * a.h + c * 8, y);
  }
  if (lane == 0) a.rstd_out[row] = r;
}

// The workgroup's partial column sums acc[k] (NS sums) -> part[blockIdx][k][h],
// the four wavefronts added in order through LDS.
template <int CPL, int NS>
LMD_DEV void group_partials(const ModArgs& a, float (&acc)[NS][CPL][8], float* red) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int C = a.h / 8;
  for (int w = 0; w < 4; ++w) {
    if (wv == w) {
#pragma unroll
      for (int k = 0; k < NS; ++k)
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          const int c = lane + 64 * j;
          if (c >= C) continue;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float& dst = red[k * a.h + c * 8 + e];
            dst = w == 0 ? acc[k][j][e] : dst + acc[k][j][e];
          }
        }
    }
    __syncthreads();
  }
  float* dst = a.part + (int64_t)blockIdx.x * NS * a.h;
  for (int i = threadIdx.x; i < NS * a.h; i += 256) dst[i] = red[i];
}

template <int CPL>
__global__ __launch_bounds__(256) void k_modnorm_bwd(ModArgs a) {
  extern __shared__ float red[];  // [2][h]
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int C = a.h / 8;
  float acc[2][CPL][8];  // d scale = sum dh * n, d shift = sum dh
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[0][j][e] = acc[1][j][e] = 0.0f;
  const int64_t r0 = (int64_t)blockIdx.x * a.rpw;
  const int64_t r1 = r0 + a.rpw < a.rows ? r0 + a.rpw : a.rows;
  for (int64_t row = r0 + wv; row < r1; row += 4) {
    const float r = a.rstd_in[row];
    u32x4 gv[CPL], xv[CPL];
    float dot = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      const bool ok = c < C;
      gv[j] = ok ? ld16(a.grad + row * a.h + c * 8) : (u32x4){0u, 0u, 0u, 0u};
      xv[j] = ok ? ld16(a.x + row * a.h + c * 8) : (u32x4){0u, 0u, 0u, 0u};
      const u32x4 sv = ok ? ld16(a.vec0 + c * 8) : (u32x4){0u, 0u, 0u, 0u};
      float g[8], f[8], s[8];
      unpack8(gv[j], g);
      unpack8(xv[j], f);
      unpack8(sv, s);
#pragma unroll
      for (int e = 0; e < 8; ++e) dot = __builtin_fmaf(g[e] * (s[e] + 1.0f), f[e] * r, dot);
    }
    dot = wave_sum(dot) / (float)a.h;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      if (c >= C) continue;
      float g[8], f[8], s[8];
      unpack8(gv[j], g);
      unpack8(xv[j], f);
      unpack8(ld16(a.vec0 + c * 8), s);
      u32x4 y;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        float d[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int e = 2 * p + q;
          const float n = f[e] * r;
          d[q] = r * (g[e] * (s[e] + 1.0f) - n * dot);
          acc[0][j][e] = __builtin_fmaf(g[e], n, acc[0][j][e]);
          acc[1][j][e] += g[e];
        }
        y[p] = pack2(d[0], d[1]);
      }
      st16(a.out + row * a.h + c * 8, y);
    }
  }
  group_partials<CPL, 2>(a, acc, red);
}

template <int CPL>
__global__ __launch_bounds__(256) void k_gated_res_bwd(ModArgs a) {
  extern __shared__ float red[];  // [h]
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int C = a.h / 8;
  float acc[1][CPL][8];  // d gate = sum dy * o
#pragma unroll
  for (int j = 0; j < CPL; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[0][j][e] = 0.0f;
  const int64_t r0 = (int64_t)blockIdx.x * a.rpw;
  const int64_t r1 = r0 + a.rpw < a.rows ? r0 + a.rpw : a.rows;
  for (int64_t row = r0 + wv; row < r1; row += 4) {
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = lane + 64 * j;
      if (c >= C) continue;
      float g[8], o[8], s[8];
      unpack8(ld16(a.grad + row * a.h + c * 8), g);
      unpack8(ld16(a.x + row * a.h + c * 8), o);
      unpack8(ld16(a.vec0 + c * 8), s);
      u32x4 y;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        y[p] = pack2(g[2 * p] * s[2 * p], g[2 * p + 1] * s[2 * p + 1]);
        acc[0][j][2 * p] = __builtin_fmaf(g[2 * p], o[2 * p], acc[0][j][2 * p]);
        acc[0][j][2 * p + 1] = __builtin_fmaf(g[2 * p + 1], o[2 * p + 1], acc[0][j][2 * p + 1]);
      }
      st16(a.out + row * a.h + c * 8, y);
    }
  }
  group_partials<CPL, 1>(a, acc, red);
}

// out_k[c] = bf16(sum over groups of part[g][k][c]), in a fixed order: a
// workgroup owns 64 four-column quads of the nsum * h sums; thread (quarter
// u, quad q) sums groups u * gq .. in order, loads issued 16 at a time, and
// the four quarters are added in order through LDS.
__global__ __launch_bounds__(256) void k_colsum(ModArgs a, int groups, int nsum) {
  __shared__ float4 lds[4][64];
  const int q = threadIdx.x & 63, u = threadIdx.x >> 6;
  const int quad = blockIdx.x * 64 + q, nq = nsum * a.h / 4;
  const int gq = (groups + 3) / 4, g0 = u * gq, g1 = g0 + gq < groups ? g0 + gq : groups;
  const float4* part = reinterpret_cast<const float4*>(a.part);
  float4 s = {0.0f, 0.0f, 0.0f, 0.0f};
  if (quad < nq) {
    for (int g = g0; g < g1; g += 16) {
      float4 v[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) v[i] = g + i < g1 ? part[(int64_t)(g + i) * nq + quad] : (float4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        s.x += v[i].x;
        s.y += v[i].y;
        s.z += v[i].z;
        s.w += v[i].w;
      }
    }
  }
  lds[u][q] = s;
  __syncthreads();
  if (u != 0 || quad >= nq) return;
  float t[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    t[0] += lds[w][q].x;
    t[1] += lds[w][q].y;
    t[2] += lds[w][q].z;
    t[3] += lds[w][q].w;
  }
  const int i = quad * 4, k = i / a.h, c = i - k * a.h;  // h % 8 == 0: the quad stays in one sum
  uint16_t* out = (k == 0 ? a.vout0 : a.vout1) + c;
#pragma unroll
  for (int e = 0; e < 4; ++e) out[e] = __builtin_bit_cast(uint16_t, (__bf16)t[e]);
}

// y = x + gate * o over rows x h, one thread per 16-byte chunk
__global__ __launch_bounds__(256) void k_gated_res_fwd(const uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ o,
                                                       const uint16_t* __restrict__ gate, int64_t chunks, int cpr,
                                                       uint16_t* __restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= chunks) return;
  const int c = (int)(i % cpr);
  float xv[8], ov[8], gv[8];
  unpack8(ld16(x + i * 8), xv);
  unpack8(ld16(o + i * 8), ov);
  unpack8(ld16(gate + c * 8), gv);
  u32x4 r;
#pragma unroll
  for (int p = 0; p < 4; ++p)
    r[p] = pack2(__builtin_fmaf(gv[2 * p], ov[2 * p], xv[2 * p]), __builtin_fmaf(gv[2 * p + 1], ov[2 * p + 1], xv[2 * p + 1]));
  st16(y + i * 8, r);
}

constexpr float GELU_C = 0.7978845608028654f;  // sqrt(2 / pi)
constexpr float GELU_K = 0.044715f;

// sigmoid(2 c (u + k u^3)) = (1 + tanh(c (u + k u^3))) / 2, and its argument's
// derivative in u
LMD_DEV float gelu_gate(float u, float* dz) {
  const float u2 = fminf(u * u, 1e30f);  // |u| past 1e15: z and z' stay ordered, no inf * 0 below
  const float z = GELU_C * __builtin_fmaf(GELU_K * u2, u, u);
  if (dz) *dz = GELU_C * __builtin_fmaf(3.0f * GELU_K, u2, 1.0f);
  return __builtin_amdgcn_rcpf(1.0f + __expf(-2.0f * z));
}

// g = u * sigmoid(2z), one thread per 16-byte chunk
__global__ __launch_bounds__(256) void k_gelu_fwd(const uint16_t* __restrict__ u, int64_t chunks,
                                                  uint16_t* __restrict__ g) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= chunks) return;
  float f[8];
  unpack8(ld16(u + i * 8), f);
  u32x4 r;
#pragma unroll
  for (int p = 0; p < 4; ++p)
    r[p] = pack2(f[2 * p] * gelu_gate(f[2 * p], nullptr), f[2 * p + 1] * gelu_gate(f[2 * p + 1], nullptr));
  st16(g + i * 8, r);
}

// du = dg * (s + 2 u s (1 - s) z'), s = sigmoid(2z): the derivative of
// u * (1 + tanh z) / 2 with 1 - tanh^2 z = 4 s (1 - s)
__global__ __launch_bounds__(256) void k_gelu_bwd(const uint16_t* __restrict__ dg, const uint16_t* __restrict__ u,
                                                  int64_t chunks, uint16_t* __restrict__ du) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= chunks) return;
  float f[8], d[8], o[8];
  unpack8(ld16(u + i * 8), f);
  unpack8(ld16(dg + i * 8), d);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float dz;
    const float sg = gelu_gate(f[e], &dz);
    const float w = sg * (1.0f - sg);  // 0 once the sigmoid saturates, before u scales it
    o[e] = d[e] * __builtin_fmaf(2.0f * (w * f[e]), dz, sg);
  }
  u32x4 r;
#pragma unroll
  for (int p = 0; p < 4; ++p) r[p] = pack2(o[2 * p], o[2 * p + 1]);
  st16(du + i * 8, r);
}

int fail(int code, const char* what) {
  lmd_err_msg = what;
  return code;
}

bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int rows_per_group(int64_t rows) {
  int64_t rpw = (rows + GROUPS - 1) / GROUPS;
  rpw = (rpw + 3) / 4 * 4;
  return (int)(rpw < 4 ? 4 : rpw);
}

int check_common(int64_t rows, int h, const void* x, const void* vec0) {
  if (rows <= 0) return fail(-1, "rows must be positive");
  if (h <= 0 || h % 8 || h > 64 * 8 * MAX_CPL) return fail(-1, "h must be a positive multiple of 8, at most 4096");
  if (!x || !vec0) return fail(-1, "null input pointer");
  if (!al16(x) || !al16(vec0)) return fail(-1, "inputs must be 16-byte aligned");
  return 0;
}

#define LMD_CPL_SWITCH(KERN, grid, lds)                                                               \
  switch ((a.h / 8 + 63) / 64) {                                                                      \
    case 1: hipLaunchKernelGGL(KERN<1>, grid, dim3(256), lds, (hipStream_t)stream, a); break;         \
    case 2: hipLaunchKernelGGL(KERN<2>, grid, dim3(256), lds, (hipStream_t)stream, a); break;         \
    case 3: hipLaunchKernelGGL(KERN<3>, grid, dim3(256), lds, (hipStream_t)stream, a); break;         \
    case 4: hipLaunchKernelGGL(KERN<4>, grid, dim3(256), lds, (hipStream_t)stream, a); break;         \
    case 5: hipLaunchKernelGGL(KERN<5>, grid, dim3(256), lds, (hipStream_t)stream, a); break;         \
    case 6: hipLaunchKernelGGL(KERN<6>, grid, dim3(256), lds, (hipStream_t)stream, a); break;         \
    case 7: hipLaunchKernelGGL(KERN<7>, grid, dim3(256), lds, (hipStream_t)stream, a); break;         \
    default: hipLaunchKernelGGL(KERN<8>, grid, dim3(256), lds, (hipStream_t)stream, a); break;        \
  }

int launched() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : fail(-3, hipGetErrorString(e));
}

}  // namespace

extern "C" int64_t lmd_colsum_groups(int64_t rows) {
  if (rows <= 0) return 0;
  const int rpw = rows_per_group(rows);
  return (rows + rpw - 1) / rpw;
}

extern "C" int lmd_modnorm_fwd(const uint16_t* x, int64_t rows, int h, const uint16_t* scale, const uint16_t* shift,
                               float eps, uint16_t* out, float* rstd, void* stream) {
  if (int rc = check_common(rows, h, x, scale)) return rc;
  if (!shift || !out || !rstd) return fail(-1, "null pointer");
  if (!al16(shift) || !al16(out)) return fail(-1, "shift and out must be 16-byte aligned");
  if (!(eps > 0.0f)) return fail(-1, "eps must be positive");
  ModArgs a{};
  a.rows = rows;
  a.h = h;
  a.eps = eps;
  a.x = x;
  a.vec0 = scale;
  a.vec1 = shift;
  a.out = out;
  a.rstd_out = rstd;
  lmd_err_msg.clear();
  const dim3 grid((unsigned)((rows + 3) / 4));
  LMD_CPL_SWITCH(k_modnorm_fwd, grid, 0)
  return launched();
}

extern "C" int lmd_modnorm_bwd(const uint16_t* dh, const uint16_t* x, int64_t rows, int h, const uint16_t* scale,
                               const float* rstd, uint16_t* dx, uint16_t* dscale, uint16_t* dshift, float* part,
                               void* stream) {
  if (int rc = check_common(rows, h, x, scale)) return rc;
  if (!dh || !rstd || !dx || !dscale || !dshift || !part) return fail(-1, "null pointer");
  if (!al16(dh) || !al16(dx)) return fail(-1, "dh and dx must be 16-byte aligned");
  ModArgs a{};
  a.rows = rows;
  a.h = h;
  a.rpw = rows_per_group(rows);
  a.x = x;
  a.vec0 = scale;
  a.grad = dh;
  a.rstd_in = rstd;
  a.out = dx;
  a.part = part;
  a.vout0 = dscale;
  a.vout1 = dshift;
  lmd_err_msg.clear();
  const int groups = (int)lmd_colsum_groups(rows);
  LMD_CPL_SWITCH(k_modnorm_bwd, dim3(groups), 2 * h * sizeof(float))
  if (int rc = launched()) return rc;
  hipLaunchKernelGGL(k_colsum, dim3((2 * h / 4 + 63) / 64), dim3(256), 0, (hipStream_t)stream, a, groups, 2);
  return launched();
}

extern "C" int lmd_gated_residual_bwd(const uint16_t* dy, const uint16_t* o, int64_t rows, int h, const uint16_t* gate,
                                      uint16_t* d_o, uint16_t* dgate, float* part, void* stream) {
  if (int rc = check_common(rows, h, o, gate)) return rc;
  if (!dy || !d_o || !dgate || !part) return fail(-1, "null pointer");
  if (!al16(dy) || !al16(d_o)) return fail(-1, "dy and do must be 16-byte aligned");
  ModArgs a{};
  a.rows = rows;
  a.h = h;
  a.rpw = rows_per_group(rows);
  a.x = o;
  a.vec0 = gate;
  a.grad = dy;
  a.out = d_o;
  a.part = part;
  a.vout0 = dgate;
  lmd_err_msg.clear();
  const int groups = (int)lmd_colsum_groups(rows);
  LMD_CPL_SWITCH(k_gated_res_bwd, dim3(groups), h * sizeof(float))
  if (int rc = launched()) return rc;
  hipLaunchKernelGGL(k_colsum, dim3((h / 4 + 63) / 64), dim3(256), 0, (hipStream_t)stream, a, groups, 1);
  return launched();
}

extern "C" int lmd_gated_residual_fwd(const uint16_t* x, const uint16_t* o, int64_t rows, int h, const uint16_t* gate,
                                      uint16_t* y, void* stream) {
  if (int rc = check_common(rows, h, o, gate)) return rc;
  if (!x || !y) return fail(-1, "null pointer");
  if (!al16(x) || !al16(y)) return fail(-1, "x and y must be 16-byte aligned");
  const int64_t chunks = rows * (h / 8);
  if ((chunks + 255) / 256 > 0x7fffffff) return fail(-1, "too many rows");
  lmd_err_msg.clear();
  hipLaunchKernelGGL(k_gated_res_fwd, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x, o,
                     gate, chunks, h / 8, y);
  return launched();
}

extern "C" int lmd_gelu_tanh_fwd(const uint16_t* u, int64_t n, uint16_t* g, void* stream) {
  if (n <= 0 || n % 8) return fail(-1, "n must be a positive multiple of 8");
  if (!u || !g) return fail(-1, "null pointer");
  if (!al16(u) || !al16(g)) return fail(-1, "u and g must be 16-byte aligned");
  const int64_t chunks = n / 8;
  if ((chunks + 255) / 256 > 0x7fffffff) return fail(-1, "too many elements");
  lmd_err_msg.clear();
  hipLaunchKernelGGL(k_gelu_fwd, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, (hipStream_t)stream, u, chunks,
                     g);
  return launched();
}

extern "C" int lmd_gelu_tanh_bwd(const uint16_t* dg, const uint16_t* u, int64_t n, uint16_t* du, void* stream) {
  if (n <= 0 || n % 8) return fail(-1, "n must be a positive multiple of 8");
  if (!dg || !u || !du) return fail(-1, "null pointer");
  if (!al16(dg) || !al16(u) || !al16(du)) return fail(-1, "dg, u and du must be 16-byte aligned");
  const int64_t chunks = n / 8;
  if ((chunks + 255) / 256 > 0x7fffffff) return fail(-1, "too many elements");
  lmd_err_msg.clear();
  hipLaunchKernelGGL(k_gelu_bwd, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, (hipStream_t)stream, dg, u,
                     chunks, du);
  return launched();
}
