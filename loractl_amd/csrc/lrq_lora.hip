// The low-rank (LoRA) side products of the fused linear, as matrix-core
// kernels with a deterministic two-stage reduction (no atomics):
//
//   t  = s . x  . A      [m, r]  (src/lora.rs:199-203, A-linear then scale)
//   u  = s . dy . B^T    [m, r]  (autodiff of the B-linear, input side)
//   dA = x^T . u         [k, r]  (weight grad of the A-linear)
//   dB = t^T . dy        [r, n]  (weight grad of the B-linear)
//
// "nt" kernels reduce along a contiguous dimension (t, u); "tn" kernels
// reduce along the token dimension m, which is strided in memory, so the
// token tile is transposed into LDS before it feeds the matrix cores.
// Stage 1 writes f32 partial sums per split of the reduction; stage 2 sums
// the splits in a fixed order.
#include "lrq_common.h"
#include "lrq_kernels.h"

namespace {

constexpr int NT = 256;
constexpr int TARGET_WG = 768;

// ------------------------------------------------------------------ nt
// partial[s][m][j] = sum_{c in split s} p[m][c] * q[j][c]; 64 rows per
// workgroup (16 per wavefront), c in steps of 32 (one 16x16x32 MFMA per
// 16-wide j tile).
__global__ void __launch_bounds__(NT) k_skinny_nt(const uint16_t* __restrict__ p,
                                                  const uint16_t* __restrict__ q, int64_t M,
                                                  int64_t C, int R, int rp, int64_t c_per,
                                                  float* __restrict__ partial) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t m0 = (int64_t)blockIdx.x * 64 + wave * 16;
  const int split = blockIdx.y;
  const int64_t c_lo = split * c_per;
  const int64_t c_hi = min(C, c_lo + c_per);
  const int64_t mrow = m0 + (lane & 15);
  const bool mok = mrow < M;
  const int koff = (lane >> 4) * 8;
  const int jt_n = rp / 16;

  f32x4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  const uint16_t* prow = p + (mok ? mrow : 0) * C;
  for (int64_t c = c_lo; c < c_hi; c += 32) {
    const int64_t cc = c + koff;
    const bool cok = cc < c_hi;
    const bf16x8 fa = as_bf16x8(ld16_pred(prow + cc, mok && cok));
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (t < jt_n) {
        const int j = t * 16 + (lane & 15);
        const bf16x8 fb = as_bf16x8(ld16_pred(q + (int64_t)(j < R ? j : 0) * C + cc, cok && j < R));
        acc[t] = mfma16(fa, fb, acc[t]);
      }
    }
  }
  float* out = partial + (int64_t)split * M * rp;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (t < jt_n) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t m = m0 + 4 * (lane >> 4) + v;
        if (m < M) out[m * rp + t * 16 + (lane & 15)] = acc[t][v];
      }
    }
  }
}

__global__ void __launch_bounds__(NT) k_nt_reduce(const float* __restrict__ partial, int splits,
                                                  int64_t M, int64_t ldT, int rp, int R, float s,
                                                  uint16_t* __restrict__ out,
                                                  uint16_t* __restrict__ outT,
                                                  uint16_t* __restrict__ out_user, int r_user) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= ldT * rp) return;
  // j fastest for the [m, rp] outputs
  const int64_t m = idx / rp;
  const int j = (int)(idx % rp);
  if (m >= M) {  // zero the padding columns of the transposed copy
    if (outT) outT[(int64_t)j * ldT + m] = 0;
    return;
  }
  float v = 0.0f;
  for (int sp = 0; sp < splits; ++sp) v += partial[(int64_t)sp * M * rp + idx];
  v = (j < R) ? v * s : 0.0f;
  const uint16_t h = f32_to_bf16_bits(v);
  if (out) out[idx] = h;
  if (outT) outT[(int64_t)j * ldT + m] = h;
  if (out_user && j < r_user) out_user[m * r_user + j] = h;
}

// ------------------------------------------------------------------ tn
// partial[s][c][j] = sum_{m in split s} p[m][c] * qT[j][m]; 64 c per
// workgroup (16 per wavefront). The p tile [64 m][64 c] is transposed into
// LDS as [c][m] so the A-role fragment (8 consecutive m) is one 16-byte read.
constexpr int TLD = 64 + 8;

__global__ void __launch_bounds__(NT) k_skinny_tn(const uint16_t* __restrict__ p,
                                                  const uint16_t* __restrict__ qT, int64_t ldq,
                                                  int64_t M, int64_t C, int rp, int64_t m_per,
                                                  float* __restrict__ partial) {
  __shared__ __attribute__((aligned(16))) uint16_t sT[64 * TLD];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t c0 = (int64_t)blockIdx.x * 64;
  const int split = blockIdx.y;
  const int64_t m_lo = split * m_per;
  const int64_t m_hi = min(M, m_lo + m_per);
  const int jt_n = rp / 16;
  const int koff = (lane >> 4) * 8;

  f32x4 acc[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  // loader: 2 chunks per thread, chunk id -> row id/8, columns (id%8)*8
  u32x4 pr[2];
  auto gload = [&](int64_t mb) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int id = tid + NT * h;
      const int row = id >> 3, cc = (id & 7) * 8;
      const int64_t m = mb + row;
      const bool ok = (m < m_hi) && (c0 + cc < C);
      pr[h] = ld16_pred(p + (ok ? m : 0) * C + c0 + cc, ok);
    }
  };

  gload(m_lo);
  for (int64_t mb = m_lo; mb < m_hi; mb += 64) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int id = tid + NT * h;
      const int row = id >> 3, cc = (id & 7) * 8;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sT[(cc + 2 * e) * TLD + row] = (uint16_t)(pr[h][e] & 0xffffu);
        sT[(cc + 2 * e + 1) * TLD + row] = (uint16_t)(pr[h][e] >> 16);
      }
    }
    __syncthreads();
    if (mb + 64 < m_hi) gload(mb + 64);
#pragma unroll
    for (int ms = 0; ms < 2; ++ms) {
      const bf16x8 fa = as_bf16x8(ld16(sT + (wave * 16 + (lane & 15)) * TLD + ms * 32 + koff));
      const int64_t mm = mb + ms * 32 + koff;
      const bool mok = mm < m_hi;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (t < jt_n) {
          const int j = t * 16 + (lane & 15);
          const bf16x8 fb = as_bf16x8(ld16_pred(qT + (int64_t)j * ldq + (mok ? mm : 0), mok));
          acc[t] = mfma16(fa, fb, acc[t]);
        }
      }
    }
    __syncthreads();
  }
  float* out = partial + (int64_t)split * C * rp;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (t < jt_n) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t c = c0 + wave * 16 + 4 * (lane >> 4) + v;
        if (c < C) out[c * rp + t * 16 + (lane & 15)] = acc[t][v];
      }
    }
  }
}

__global__ void __launch_bounds__(NT) k_tn_reduce(const float* __restrict__ partial, int splits,
                                                  int64_t C, int rp, int R, float* __restrict__ out,
                                                  int64_t sc, int64_t sj) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= C * rp) return;
  const int64_t c = idx / rp;
  const int j = (int)(idx % rp);
  if (j >= R) return;
  float v = 0.0f;
  for (int sp = 0; sp < splits; ++sp) v += partial[(int64_t)sp * C * rp + idx];
  out[c * sc + (int64_t)j * sj] = v;
}

// ------------------------------------------------------------------ layout
__global__ void __launch_bounds__(NT) k_pad_transpose(const uint16_t* __restrict__ src, int64_t rows,
                                                      int64_t cols, int64_t ld_src,
                                                      uint16_t* __restrict__ dst, int64_t dst_rows,
                                                      int64_t dst_cols, int transpose) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= dst_rows * dst_cols) return;
  const int64_t dr = idx / dst_cols, dc = idx % dst_cols;
  // dst[dr][dc] = transpose ? src[dc][dr] : src[dr][dc]
  const int64_t sr = transpose ? dc : dr, sc = transpose ? dr : dc;
  dst[idx] = (sr < rows && sc < cols) ? src[sr * ld_src + sc] : (uint16_t)0;
}

inline unsigned nblocks(int64_t items) { return (unsigned)((items + NT - 1) / NT); }

}  // namespace

int skinny_nt_splits(int64_t M, int64_t C) {
  const int64_t tiles = (M + 63) / 64;
  int64_t s = (TARGET_WG + tiles - 1) / tiles;
  const int64_t smax = (C + 255) / 256;  // keep >= 256 columns per split
  if (s > smax) s = smax;
  if (s < 1) s = 1;
  return (int)s;
}

int skinny_tn_splits(int64_t M, int64_t C) {
  const int64_t tiles = (C + 63) / 64;
  int64_t s = (TARGET_WG + tiles - 1) / tiles;
  const int64_t smax = (M + 127) / 128;  // keep >= 128 tokens per split
  if (s > smax) s = smax;
  if (s < 1) s = 1;
  return (int)s;
}

hipError_t launch_skinny_nt(hipStream_t st, const uint16_t* p, const uint16_t* q, int64_t M,
                            int64_t C, int R, int rp, float s, float* partial, int splits,
                            uint16_t* out, uint16_t* outT, int64_t ldT, uint16_t* out_user,
                            int r_user) {
  if (M == 0) return hipSuccess;
  const int64_t c_per = ((C + splits - 1) / splits + 31) / 32 * 32;
  const int used = (int)((C + c_per - 1) / c_per);
  hipLaunchKernelGGL(k_skinny_nt, dim3((unsigned)((M + 63) / 64), (unsigned)used), dim3(NT), 0, st,
                     p, q, M, C, R, rp, c_per, partial);
  const int64_t ld = outT ? ldT : M;  // without a transposed copy only the M real rows exist
  hipLaunchKernelGGL(k_nt_reduce, dim3(nblocks(ld * rp)), dim3(NT), 0, st, partial, used, M, ld,
                     rp, R, s, out, outT, out_user, r_user);
  return hipGetLastError();
}

hipError_t launch_skinny_tn(hipStream_t st, const uint16_t* p, const uint16_t* qT, int64_t ldq,
                            int64_t M, int64_t C, int R, int rp, float* partial, int splits,
                            float* out, int64_t sc, int64_t sj) {
  if (C == 0) return hipSuccess;
  const int64_t m_per = ((M + splits - 1) / splits + 63) / 64 * 64;
  const int used = M == 0 ? 1 : (int)((M + m_per - 1) / m_per);
  hipLaunchKernelGGL(k_skinny_tn, dim3((unsigned)((C + 63) / 64), (unsigned)used), dim3(NT), 0, st,
                     p, qT, ldq, M, C, rp, m_per, partial);
  hipLaunchKernelGGL(k_tn_reduce, dim3(nblocks(C * rp)), dim3(NT), 0, st, partial, used, C, rp, R,
                     out, sc, sj);
  return hipGetLastError();
}

hipError_t launch_pad_transpose(hipStream_t st, const uint16_t* src, int64_t rows, int64_t cols,
                                int64_t ld_src, uint16_t* dst, int64_t dst_rows, int64_t dst_cols,
                                bool transpose) {
  if (dst_rows * dst_cols == 0) return hipSuccess;
  hipLaunchKernelGGL(k_pad_transpose, dim3(nblocks(dst_rows * dst_cols)), dim3(NT), 0, st, src, rows,
                     cols, ld_src, dst, dst_rows, dst_cols, transpose ? 1 : 0);
  return hipGetLastError();
}
