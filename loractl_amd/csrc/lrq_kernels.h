// Internal launcher declarations shared by the kernel files and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/loractl_rocm.h"

// lrq_quant.hip
hipError_t launch_quantize_int4(hipStream_t st, const float* w, int64_t n, int64_t k, int g,
                                uint8_t* packed, float* scales);
hipError_t launch_quantize_fp8(hipStream_t st, const float* w, int64_t n, int64_t k,
                               int per_channel, uint8_t* bytes, float* scales, float* amax_ws);
hipError_t launch_dequant(hipStream_t st, const lrq_weight* w, void* out, bool bf16);

// Arguments of the fused forward: y = x . dq(w)^T (+bias) + t . bt^T
struct FwdArgs {
  const uint16_t* x;  // [m, k]
  int64_t m, n, k;
  const uint8_t* wdata;
  const float* wscale;
  int group;
  int per_channel;
  const float* bias;   // [n] or null
  const uint16_t* t;   // [m, rp] (already scaled), null when no LoRA
  const uint16_t* bt;  // [n, rp]
  int rp;              // padded rank, multiple of 16, 0 = no LoRA
  uint16_t* y;         // [m, n]
};

// Arguments of the fused backward dx: dx = dy . dq(w) + u . ap^T
struct BwdArgs {
  const uint16_t* dy;  // [m, n]
  int64_t m, n, k;
  const uint8_t* wdata;
  const float* wscale;
  int group;
  int per_channel;
  const uint16_t* u;   // [m, rp] (already scaled) or null
  const uint16_t* ap;  // [k, rp]
  int rp;
  uint16_t* dx;        // [m, k]
};

// lrq_gemm.hip
hipError_t launch_fwd_main(hipStream_t st, int fmt, const FwdArgs& a, int* kid);
hipError_t launch_bwd_dx(hipStream_t st, int fmt, const BwdArgs& a, int* kid);

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
  KID_COUNT
};
