// Weight-format kernels: int4 and int8 block quantization (src/quant.rs:74-82
// closed form), fp8 e4m3fn repack (reference/fp8_reference.py:83-91), and the
// dequantize kernels that expose the f32 values (src/quant.rs:232,
// src/fp8.rs:306-318) and the bf16 matrix-core operands.
//
// All of these are HBM-bound byte/integer work: one thread per 8-value run,
// 16-byte stores where the layout allows it, no LDS.
#include "lrq_common.h"
#include "lrq_kernels.h"

// ------------------------------------------------------------------ int4 / int8 quantize
// QMAX 7: Q4S, packed nibbles q + 8; QMAX 127: Q8S, int8 bytes (src/quant.rs:156-162).
// One thread per (row, 32-value half-block); a block of `group` values is
// covered by group/32 consecutive threads that reduce absmax with lane
// shuffles (group/32 <= 64 lanes, a power of two or not: a plain loop over
// the partner lanes keeps it exact).
// FP8: the input is e4m3fn bytes [n, k] with a scalar or per-row f32 scale,
// and each value is LUT[byte] * scale in f32 first (src/fp8.rs:306-318), the
// reference's f32 snapshot of an fp8 checkpoint tensor, which its load pass
// then quantizes (src/diffusion_trainer.rs:1143-1169); no f32 copy is kept.
template <bool FP8, int QMAX>
__global__ void __launch_bounds__(256) k_quantize(const void* __restrict__ wv, const float* __restrict__ fsc,
                                                       int per_channel, int64_t n, int64_t k, int g,
                                                       uint8_t* __restrict__ packed, float* __restrict__ scales) {
  const int64_t runs_per_row = k / 32;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= n * runs_per_row) return;
  const int64_t row = tid / runs_per_row;
  const int64_t run = tid % runs_per_row;
  float v[32];
  float amax = 0.0f;
  if constexpr (FP8) {
    const uint8_t* src = static_cast<const uint8_t*>(wv) + row * k + run * 32;
    const float sc = fsc[per_channel ? row : 0];
#pragma unroll
    for (int i = 0; i < 32; i += 16) {
      const u32x4 b = ld16(src + i);
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        float f[4];
        fp8x4_to_f32(b[d], f);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[i + 4 * d + e] = f[e] * sc;
      }
    }
  } else {
    const float* src = static_cast<const float*>(wv) + row * k + run * 32;
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
      f32x4 t = *reinterpret_cast<const f32x4*>(src + i);
      v[i] = t[0]; v[i + 1] = t[1]; v[i + 2] = t[2]; v[i + 3] = t[3];
    }
  }
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  // absmax over the whole block: the block's runs are consecutive tids,
  // hence consecutive lanes of one wavefront (g/32 divides... g is a multiple
  // of 32 and rows start at run 0, but a block may straddle two wavefronts
  // when g/32 does not divide 64; the host restricts g/32 to a divisor of 64).
  const int rpb = g / 32;
  if (rpb > 1) {
    const int lane = threadIdx.x & 63;
    const int first = lane - (int)(run % rpb);
    float m = 0.0f;
    for (int j = 0; j < rpb; ++j) m = fmaxf(m, __shfl(amax, first + j, 64));
    amax = m;
  }
  const float s = amax / (float)QMAX;  // correctly rounded f32 division
  if (run % rpb == 0) scales[row * (k / g) + run / rpb] = s;
  // q = clamp(round_half_away(RN(v / s))). The quotient RN(v / s) is formed
  // without a division per value: with y = RN(1 / s), q0 = RN(v y) and the
  // exact remainder r = v - q0 s (one fma), RN(q0 + r y) == RN(v / s)
  // (Markstein: y within half an ulp of 1/s and q0 within one ulp of v/s,
  // no underflow). r stays normal for s >= 2^-80; smaller scales divide.
  int q[32];
  auto to_int = [](float t) {
    const float r = fminf(fmaxf(roundf(t), -(float)QMAX), (float)QMAX);  // half away from zero
    return (int)r;
  };
  if (s >= 0x1p-80f) {
    const float y = 1.0f / s;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float q0 = v[i] * y;
      const float rem = __builtin_fmaf(-q0, s, v[i]);
      q[i] = to_int(__builtin_fmaf(rem, y, q0));
    }
  } else if (s != 0.0f) {
#pragma unroll
    for (int i = 0; i < 32; ++i) q[i] = to_int(v[i] / s);
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) q[i] = 0;
  }
  if constexpr (QMAX == 7) {
    u32x4 o = zero4();
#pragma unroll
    for (int i = 0; i < 32; ++i) o[i >> 3] |= (uint32_t)(q[i] + 8) << (4 * (i & 7));
    st16(packed + row * (k / 2) + run * 16, o);
  } else {
    u32x4 o[2] = {zero4(), zero4()};
#pragma unroll
    for (int i = 0; i < 32; ++i) o[i >> 4][(i >> 2) & 3] |= ((uint32_t)q[i] & 0xffu) << (8 * (i & 3));
    st16(packed + row * k + run * 32, o[0]);
    st16(packed + row * k + run * 32 + 16, o[1]);
  }
}

// ------------------------------------------------------------------ fp8 quantize
// Exact RNE e4m3fn encode of an f32 that is already divided by the scale.
__device__ __forceinline__ uint32_t fp8_encode_rne(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;     // NaN
  if (a >= 0x43e00000u) return sign | 0x7eu;    // |x| >= 448: saturate
  if (a < 0x3c800000u) {                        // |x| < 2^-6: subnormal grid 2^-9
    const float ax = __builtin_bit_cast(float, a) * 512.0f;  // exact
    const float r = __builtin_rintf(ax);                      // RNE
    return sign | (uint32_t)r;                                // 8 rolls into 0x08
  }
  // normal: keep 3 mantissa bits with RNE on the f32 bit pattern
  const uint32_t lsb = (a >> 20) & 1u;
  const uint32_t rounded = a + 0x7ffffu + lsb;
  const uint32_t e = (rounded >> 23) - 120u;  // fp8 exponent field
  const uint32_t m = (rounded >> 20) & 7u;
  uint32_t code = (e << 3) | m;
  if (code > 0x7eu) code = 0x7eu;
  return sign | code;
}

// Per-row (or whole-tensor) amax -> scale. One block per row for per-channel;
// for a scalar scale a first pass writes per-row amax and a second block folds.
__global__ void __launch_bounds__(256) k_rowabsmax(const float* __restrict__ w, int64_t k,
                                                   float* __restrict__ out) {
  const int64_t row = blockIdx.x;
  const float* src = w + row * k;
  float m = 0.0f;
  for (int64_t i = threadIdx.x; i < k; i += blockDim.x) m = fmaxf(m, fabsf(src[i]));
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) out[row] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__global__ void __launch_bounds__(256) k_fp8_scales(float* __restrict__ amax, int64_t n,
                                                    int per_channel, float* __restrict__ scales) {
  if (per_channel) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
      float s = amax[i] / 448.0f;
      scales[i] = s < 1e-12f ? 1e-12f : s;
    }
  } else if (blockIdx.x == 0) {
    float m = 0.0f;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) m = fmaxf(m, amax[i]);
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    __shared__ float red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
      float s = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])) / 448.0f;
      scales[0] = s < 1e-12f ? 1e-12f : s;
    }
  }
}

__global__ void __launch_bounds__(256) k_fp8_encode(const float* __restrict__ w, int64_t n, int64_t k,
                                                    int per_channel, const float* __restrict__ scales,
                                                    uint8_t* __restrict__ out) {
  // one thread per 4 consecutive values (k % 32 == 0 so rows hold whole runs)
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = n * k / 4;
  if (tid >= total) return;
  const int64_t row = (tid * 4) / k;
  const float s = per_channel ? scales[row] : scales[0];
  f32x4 v = *reinterpret_cast<const f32x4*>(w + tid * 4);
  uint32_t word = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) word |= fp8_encode_rne(v[j] / s) << (8 * j);
  reinterpret_cast<uint32_t*>(out)[tid] = word;
}

// ------------------------------------------------------------------ blocked layout
// The fused GEMMs read the frozen weight in 64 (n) x 64 (k) blocks that are
// contiguous in memory (int4: 64 rows x 32 bytes; fp8, int8: 64 rows x 64
// bytes), block (nb, kb) at (nb * KB + kb) * block bytes, KB = ceil(k / 64);
// int4 and int8 scales as [NB][Gp][64] (Gp = 64*KB / group). Rows past n and
// columns past k are padding: int4 nibbles 8 (q = 0) with scale 0, int8 and
// fp8 bytes 0 (int8 with scale 0). A second,
// transposed section of the same size follows (k_block_data_t).
LRQ_DEV int64_t blk_data_off(int fmt, int64_t n, int64_t k, int64_t KB) {
  const int64_t rb = (fmt == LRQ_FMT_INT4) ? 32 : 64;  // bytes per block row
  const int64_t kb = k >> 6, kin = k & 63;
  return (((n >> 6) * KB + kb) * 64 + (n & 63)) * rb + ((fmt == LRQ_FMT_INT4) ? (kin >> 1) : kin);
}

// one thread per 16 output bytes of the blocked data
__global__ void __launch_bounds__(256) k_block_data(const uint8_t* __restrict__ src, int64_t n, int64_t k,
                                                    int fmt, int64_t NB, int64_t KB, uint8_t* __restrict__ dst) {
  const int64_t rb = (fmt == LRQ_FMT_INT4) ? 32 : 64;
  const int64_t chunks = NB * KB * 64 * (rb / 16);
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= chunks) return;
  const int64_t per_row = rb / 16, per_blk = 64 * per_row;
  const int64_t blk = tid / per_blk, inb = tid % per_blk;
  const int64_t nb = blk / KB, kb = blk % KB;
  const int64_t row = nb * 64 + inb / per_row;
  const int64_t kcol = kb * 64 + (inb % per_row) * ((fmt == LRQ_FMT_INT4) ? 32 : 16);
  u32x4 v;
  const uint32_t fill = (fmt == LRQ_FMT_INT4) ? 0x88888888u : 0u;
  v[0] = v[1] = v[2] = v[3] = fill;
  if (row < n && kcol < k) {
    const int64_t rowb = (fmt == LRQ_FMT_INT4) ? k / 2 : k;
    v = ld16(src + row * rowb + ((fmt == LRQ_FMT_INT4) ? kcol / 2 : kcol));
  }
  st16(dst + tid * 16, v);
}

__global__ void __launch_bounds__(256) k_block_scales(const float* __restrict__ src, int64_t n, int64_t G,
                                                      int64_t NB, int64_t Gp, float* __restrict__ dst) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= NB * Gp * 64) return;
  const int64_t r = tid & 63, j = (tid >> 6) % Gp, nb = (tid >> 6) / Gp;
  const int64_t row = nb * 64 + r;
  dst[tid] = (row < n && j < G) ? src[row * G + j] : 0.0f;
}

// Transposed section, read by the input-gradient GEMM (its reduction runs
// along n): the blocked layout of W^T [k, n], i.e. 64 (k) x 64 (n) blocks,
// block (kb, nb) at (kb * NB + nb) * block bytes, block row r = k. int4: 32
// bytes per row, byte c holding n = 2c in its low nibble and 2c+1 in its high
// nibble, each nibble q in two's complement (the kernel sign-extends it);
// fp8 and int8: 64 bytes per row, bytes as in the row layout. Padding is
// q = 0 (int4) or byte 0 (fp8, int8). One thread
// per 16 output bytes (32 or 16 values of one k row, gathered from as many
// rows of the row layout).
__global__ void __launch_bounds__(256) k_block_data_t(const uint8_t* __restrict__ src, int64_t n, int64_t k,
                                                      int fmt, int64_t NB, int64_t KB, uint8_t* __restrict__ dst) {
  const bool i4 = fmt == LRQ_FMT_INT4;
  const int64_t per_row = i4 ? 2 : 4;  // 16-byte chunks per block row
  const int64_t chunks = KB * NB * 64 * per_row;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= chunks) return;
  const int64_t per_blk = 64 * per_row;
  const int64_t blk = tid / per_blk, inb = tid % per_blk;
  const int64_t kb = blk / NB, nb = blk % NB;
  const int64_t kk = kb * 64 + inb / per_row;
  const int64_t n0 = nb * 64 + (inb % per_row) * (i4 ? 32 : 16);
  u32x4 v = zero4();
  if (kk < k) {
    if (i4) {
      for (int e = 0; e < 32; ++e) {
        if (n0 + e >= n) break;
        const uint32_t byte = src[(n0 + e) * (k / 2) + kk / 2];
        const uint32_t u = (kk & 1) ? (byte >> 4) : (byte & 15u);  // q + 8
        v[e >> 3] |= ((u - 8u) & 15u) << (4 * (e & 7));
      }
    } else {
      for (int e = 0; e < 16; ++e) {
        if (n0 + e >= n) break;
        v[e >> 2] |= (uint32_t)src[(n0 + e) * k + kk] << (8 * (e & 3));
      }
    }
  }
  st16(dst + tid * 16, v);
}

// int4 and int8 scales of the transposed section: ST [KGt][NB*64], ST[kg][n] = scale
// of row n, group kg (zero for padding rows and groups).
__global__ void __launch_bounds__(256) k_block_scales_t(const float* __restrict__ src, int64_t n, int64_t G,
                                                        int64_t KGt, int64_t NP, float* __restrict__ dst) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= KGt * NP) return;
  const int64_t kg = tid / NP, row = tid % NP;
  dst[tid] = (row < n && kg < G) ? src[row * G + kg] : 0.0f;
}

// ------------------------------------------------------------------ dequantize
// int4 -> f32 (bit-exact q*s) or bf16 operand; one thread per 8-value run.
template <bool BF16>
__global__ void __launch_bounds__(256) k_dequant_int4(const uint8_t* __restrict__ packed,
                                                      const float* __restrict__ scales, int64_t n,
                                                      int64_t k, int g, int blocked, void* __restrict__ out) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t runs = n * (k / 8);
  if (tid >= runs) return;
  const int64_t row = tid / (k / 8);
  const int64_t kk = (tid % (k / 8)) * 8;
  const int64_t KB = (k + 63) / 64;
  const int64_t Gp = KB * 64 / g;
  const int64_t doff = blocked ? blk_data_off(LRQ_FMT_INT4, row, kk, KB) : row * (k / 2) + kk / 2;
  const int64_t soff = blocked ? (((row >> 6) * Gp + kk / g) * 64 + (row & 63)) : row * (k / g) + kk / g;
  const uint32_t word = *reinterpret_cast<const uint32_t*>(packed + doff);
  const float s = scales[soff];
  if (BF16) {
    st16(reinterpret_cast<uint16_t*>(out) + row * k + kk, dequant8_int4_bf16(word, s));
  } else {
    float f[8];
    dequant8_int4_f32(word, s, f);
    float* o = reinterpret_cast<float*>(out) + row * k + kk;
    f32x4 a = {f[0], f[1], f[2], f[3]};
    f32x4 b = {f[4], f[5], f[6], f[7]};
    *reinterpret_cast<f32x4*>(o) = a;
    *reinterpret_cast<f32x4*>(o + 4) = b;
  }
}

// int8 -> f32 (bit-exact q*s) or bf16 operand; one thread per 8-value run.
template <bool BF16>
__global__ void __launch_bounds__(256) k_dequant_int8(const uint8_t* __restrict__ data,
                                                      const float* __restrict__ scales, int64_t n,
                                                      int64_t k, int g, int blocked, void* __restrict__ out) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t runs = n * (k / 8);
  if (tid >= runs) return;
  const int64_t row = tid / (k / 8);
  const int64_t kk = (tid % (k / 8)) * 8;
  const int64_t KB = (k + 63) / 64;
  const int64_t Gp = KB * 64 / g;
  const int64_t doff = blocked ? blk_data_off(LRQ_FMT_INT8, row, kk, KB) : row * k + kk;
  const int64_t soff = blocked ? (((row >> 6) * Gp + kk / g) * 64 + (row & 63)) : row * (k / g) + kk / g;
  const u32x2 word = *reinterpret_cast<const u32x2*>(data + doff);
  const float s = scales[soff];
  if (BF16) {
    st16(reinterpret_cast<uint16_t*>(out) + row * k + kk, dequant8_int8_bf16(word, s));
  } else {
    float f[8];
    dequant8_int8_f32(word, s, f);
    float* o = reinterpret_cast<float*>(out) + row * k + kk;
    *reinterpret_cast<f32x4*>(o) = (f32x4){f[0], f[1], f[2], f[3]};
    *reinterpret_cast<f32x4*>(o + 4) = (f32x4){f[4], f[5], f[6], f[7]};
  }
}

// fp8 -> f32 (LUT value * scale, one f32 rounding) or the unscaled bf16 operand.
template <bool BF16>
__global__ void __launch_bounds__(256) k_dequant_fp8(const uint8_t* __restrict__ bytes,
                                                     const float* __restrict__ scales, int64_t n,
                                                     int64_t k, int per_channel, int blocked,
                                                     void* __restrict__ out) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t quads = n * k / 4;
  if (tid >= quads) return;
  const int64_t row = (tid * 4) / k, kk = (tid * 4) % k;
  const int64_t doff = blocked ? blk_data_off(LRQ_FMT_FP8, row, kk, (k + 63) / 64) : tid * 4;
  const uint32_t word = *reinterpret_cast<const uint32_t*>(bytes + doff);
  if (BF16) {
    reinterpret_cast<u32x2*>(out)[tid] = fp8x4_to_bf16(word);
  } else {
    const float s = per_channel ? scales[row] : scales[0];
    f32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = fp8_e4m3fn_to_f32((word >> (8 * j)) & 0xffu) * s;
    reinterpret_cast<f32x4*>(out)[tid] = o;
  }
}

// ------------------------------------------------------------------ launchers
static inline unsigned blocks_for(int64_t items, int per_block) {
  return (unsigned)((items + per_block - 1) / per_block);
}

hipError_t launch_quantize_int4(hipStream_t st, const float* w, int64_t n, int64_t k, int g,
                                uint8_t* packed, float* scales) {
  const int64_t items = n * (k / 32);
  if (items == 0) return hipSuccess;
  hipLaunchKernelGGL((k_quantize<false, 7>), dim3(blocks_for(items, 256)), dim3(256), 0, st, w, nullptr, 0, n, k,
                     g, packed, scales);
  return hipGetLastError();
}

hipError_t launch_quantize_int8(hipStream_t st, const float* w, int64_t n, int64_t k, int g, int8_t* q,
                                float* scales) {
  const int64_t items = n * (k / 32);
  if (items == 0) return hipSuccess;
  hipLaunchKernelGGL((k_quantize<false, 127>), dim3(blocks_for(items, 256)), dim3(256), 0, st, w, nullptr, 0, n, k,
                     g, reinterpret_cast<uint8_t*>(q), scales);
  return hipGetLastError();
}

hipError_t launch_requantize_fp8_int4(hipStream_t st, const uint8_t* bytes, const float* scale, int per_channel,
                                      int64_t n, int64_t k, int g, uint8_t* packed, float* scales) {
  const int64_t items = n * (k / 32);
  if (items == 0) return hipSuccess;
  hipLaunchKernelGGL((k_quantize<true, 7>), dim3(blocks_for(items, 256)), dim3(256), 0, st, bytes, scale,
                     per_channel, n, k, g, packed, scales);
  return hipGetLastError();
}

hipError_t launch_quantize_fp8(hipStream_t st, const float* w, int64_t n, int64_t k,
                               int per_channel, uint8_t* bytes, float* scales, float* amax_ws) {
  if (n == 0 || k == 0) return hipSuccess;
  hipLaunchKernelGGL(k_rowabsmax, dim3((unsigned)n), dim3(256), 0, st, w, k, amax_ws);
  hipLaunchKernelGGL(k_fp8_scales, dim3(per_channel ? blocks_for(n, 256) : 1), dim3(256), 0, st,
                     amax_ws, n, per_channel, scales);
  hipLaunchKernelGGL(k_fp8_encode, dim3(blocks_for(n * k / 4, 256)), dim3(256), 0, st, w, n, k,
                     per_channel, scales, bytes);
  return hipGetLastError();
}

hipError_t launch_dequant(hipStream_t st, const lrq_weight* w, void* out, bool bf16) {
  const int64_t n = w->n, k = w->k;
  if (n == 0 || k == 0) return hipSuccess;
  const uint8_t* d = reinterpret_cast<const uint8_t*>(w->data);
  const int blocked = w->layout == LRQ_LAYOUT_BLOCKED;
  if (w->format == LRQ_FMT_INT4) {
    const int64_t runs = n * (k / 8);
    if (bf16)
      hipLaunchKernelGGL(k_dequant_int4<true>, dim3(blocks_for(runs, 256)), dim3(256), 0, st, d,
                         w->scales, n, k, w->group, blocked, out);
    else
      hipLaunchKernelGGL(k_dequant_int4<false>, dim3(blocks_for(runs, 256)), dim3(256), 0, st, d,
                         w->scales, n, k, w->group, blocked, out);
  } else if (w->format == LRQ_FMT_INT8) {
    const int64_t runs = n * (k / 8);
    if (bf16)
      hipLaunchKernelGGL(k_dequant_int8<true>, dim3(blocks_for(runs, 256)), dim3(256), 0, st, d,
                         w->scales, n, k, w->group, blocked, out);
    else
      hipLaunchKernelGGL(k_dequant_int8<false>, dim3(blocks_for(runs, 256)), dim3(256), 0, st, d,
                         w->scales, n, k, w->group, blocked, out);
  } else {
    const int64_t quads = n * k / 4;
    if (bf16)
      hipLaunchKernelGGL(k_dequant_fp8<true>, dim3(blocks_for(quads, 256)), dim3(256), 0, st, d,
                         w->scales, n, k, w->per_channel, blocked, out);
    else
      hipLaunchKernelGGL(k_dequant_fp8<false>, dim3(blocks_for(quads, 256)), dim3(256), 0, st, d,
                         w->scales, n, k, w->per_channel, blocked, out);
  }
  return hipGetLastError();
}

void blocked_sections(int fmt, int64_t n, int64_t k, int64_t group, int64_t* data_bytes, int64_t* scale_count) {
  const int64_t NB = (n + 63) / 64, KB = (k + 63) / 64;
  *data_bytes = NB * KB * 64 * (fmt == LRQ_FMT_INT4 ? 32 : 64);
  *scale_count = (fmt != LRQ_FMT_FP8) ? NB * (KB * 64 / group) * 64 : 0;
}

int64_t blocked_t_scale_count(int fmt, int64_t n, int64_t k, int64_t group) {
  if (fmt == LRQ_FMT_FP8) return 0;
  const int64_t NB = (n + 63) / 64, KB = (k + 63) / 64;
  return (KB * 64 + group - 1) / group * NB * 64;
}

void blocked_sizes(int fmt, int64_t n, int64_t k, int64_t group, int64_t* data_bytes, int64_t* scale_count) {
  int64_t db = 0, sc = 0;
  blocked_sections(fmt, n, k, group, &db, &sc);
  *data_bytes = 2 * db;
  *scale_count = sc + blocked_t_scale_count(fmt, n, k, group);
}

hipError_t launch_block(hipStream_t st, const lrq_weight* w, uint8_t* data, float* scales) {
  const int64_t n = w->n, k = w->k;
  const int64_t NB = (n + 63) / 64, KB = (k + 63) / 64;
  int64_t db = 0, sc = 0;
  blocked_sections(w->format, n, k, w->group, &db, &sc);
  if (db == 0) return hipSuccess;
  const uint8_t* src = reinterpret_cast<const uint8_t*>(w->data);
  hipLaunchKernelGGL(k_block_data, dim3(blocks_for(db / 16, 256)), dim3(256), 0, st, src, n, k, w->format, NB, KB,
                     data);
  hipLaunchKernelGGL(k_block_data_t, dim3(blocks_for(db / 16, 256)), dim3(256), 0, st, src, n, k, w->format, NB,
                     KB, data + db);
  if (w->format != LRQ_FMT_FP8 && sc > 0) {
    hipLaunchKernelGGL(k_block_scales, dim3(blocks_for(sc, 256)), dim3(256), 0, st, w->scales, n,
                       k / w->group, NB, KB * 64 / w->group, scales);
    const int64_t st_count = blocked_t_scale_count(w->format, n, k, w->group);
    hipLaunchKernelGGL(k_block_scales_t, dim3(blocks_for(st_count, 256)), dim3(256), 0, st, w->scales, n,
                       k / w->group, st_count / (NB * 64), NB * 64, scales + sc);
  }
  return hipGetLastError();
}
