// Internal launcher declarations shared by the kernel files and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "loractl_rocm.h"

// lrq_quant.hip
hipError_t launch_quantize_int4(hipStream_t st, const float* w, int64_t n, int64_t k, int g,
                                uint8_t* packed, float* scales);
hipError_t launch_quantize_fp8(hipStream_t st, const float* w, int64_t n, int64_t k,
                               int per_channel, uint8_t* bytes, float* scales, float* amax_ws);
hipError_t launch_dequant(hipStream_t st, const lrq_weight* w, void* out, bool bf16);
void blocked_sizes(int fmt, int64_t n, int64_t k, int64_t group, int64_t* data_bytes, int64_t* scale_count);
hipError_t launch_block(hipStream_t st, const lrq_weight* w, uint8_t* data, float* scales);

// Arguments of the fused GEMM (lrq_gemm.hip), one struct for both passes:
//   forward  : act = x  [m, k], l = k, e = n; lact = t [m, rp]; lw = B [r, n]
//   backward : act = dy [m, n], l = n, e = k; lact = u [m, rp]; lw = A [k, r]
// The weight is always the file-layout [n, k] packed tensor (wk = k).
struct GemmArgs {
  const uint16_t* act;
  int64_t m, l, e, wk;
  const uint8_t* wdata;
  const float* wscale;
  int group;
  int gshift;            // log2(group) (int4 blocks are powers of two)
  uint32_t nib;          // 0x0f0f0f0f, passed opaquely (see dequant8_int4_f32)
  int per_channel;
  const float* bias;     // forward only, [n] or null
  const uint16_t* lact;  // [m, rp] pre-scaled LoRA activation, or null
  const uint16_t* lw;    // the weight-side LoRA factor (user layout)
  int r, rp;             // rank and rank padded to 16 (rp == 0: no LoRA)
  uint16_t* out;         // [m, e]
};

hipError_t launch_gemm(hipStream_t st, bool bwd, int fmt, const GemmArgs& a);

// lrq_lora.hip
// out[m, j] = s * sum_c p[m, c] * q[j, c] over c < C, for j < R (rows j >= R
// of q read as zero); written as bf16 [m, rp], optionally as bf16 [rp, ldT]
// (columns m >= M zeroed) and as bf16 [m, r_user].
hipError_t launch_skinny_nt(hipStream_t st, const uint16_t* p, const uint16_t* q, int64_t M,
                            int64_t C, int R, int rp, float s, float* partial, int splits,
                            uint16_t* out, uint16_t* outT, int64_t ldT, uint16_t* out_user,
                            int r_user);
// out(c, j) = sum_m p[m, c] * qT[j, m] (qT has leading dimension ldq >= M
// rounded up to 64, zero past M); written as f32 at out[c*sc + j*sj], j < R.
hipError_t launch_skinny_tn(hipStream_t st, const uint16_t* p, const uint16_t* qT, int64_t ldq,
                            int64_t M, int64_t C, int R, int rp, float* partial, int splits,
                            float* out, int64_t sc, int64_t sj);
// Small layout kernels for the LoRA factors.
hipError_t launch_pad_transpose(hipStream_t st, const uint16_t* src, int64_t rows, int64_t cols,
                                int64_t ld_src, uint16_t* dst, int64_t dst_rows, int64_t dst_cols,
                                bool transpose);

int skinny_nt_splits(int64_t M, int64_t C);
int skinny_tn_splits(int64_t M, int64_t C);

// kernel ids for the profiler (lrq_profile_*)
enum {
  KID_QUANT_INT4 = 0,
  KID_QUANT_FP8,
  KID_DEQUANT,
  KID_FWD_MAIN,
  KID_BWD_DX,
  KID_LORA_PREP,
  KID_LORA_T,
  KID_LORA_U,
  KID_LORA_DA,
  KID_LORA_DB,
  KID_BLOCK,
  KID_COUNT
};
