// Internal launcher declarations shared by the kernel files and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "loractl_rocm.h"

// lrq_quant.hip
hipError_t launch_quantize_int4(hipStream_t st, const float* w, int64_t n, int64_t k, int g,
                                uint8_t* packed, float* scales);
// Q8S: int8 q [n, k] + scales [n, k/g]
hipError_t launch_quantize_int8(hipStream_t st, const float* w, int64_t n, int64_t k, int g, int8_t* q,
                                float* scales);
// the same from e4m3fn bytes [n, k] and their scalar (per_channel 0) or
// per-row f32 scale: int4 of the f32 values LUT[byte] * scale
hipError_t launch_requantize_fp8_int4(hipStream_t st, const uint8_t* bytes, const float* scale, int per_channel,
                                      int64_t n, int64_t k, int g, uint8_t* packed, float* scales);
hipError_t launch_quantize_fp8(hipStream_t st, const float* w, int64_t n, int64_t k,
                               int per_channel, uint8_t* bytes, float* scales, float* amax_ws);
hipError_t launch_dequant(hipStream_t st, const lrq_weight* w, void* out, bool bf16);
// whole blocked layout (both sections)
void blocked_sizes(int fmt, int64_t n, int64_t k, int64_t group, int64_t* data_bytes, int64_t* scale_count);
// the row-blocked section alone (the transposed section starts at these offsets)
void blocked_sections(int fmt, int64_t n, int64_t k, int64_t group, int64_t* data_bytes, int64_t* scale_count);
hipError_t launch_block(hipStream_t st, const lrq_weight* w, uint8_t* data, float* scales);

// Arguments of the fused GEMMs, one struct for both passes:
//   forward  (lrq_gemm.hip, lrq_skinny.hip): act = x [m, k], l = k, e = n;
//            lact = t [m, rp]; lw = B^T [n, rp] (lrq_gemm.hip) or
//            B [r, n] (lrq_skinny.hip)
//   backward (lrq_gemm.hip): act = dy [m, n], l = n, e = k; lact = u [m, rp];
//            lw = A [k, rp]
// The weight is a section of the blocked layout (wk = k).
// One tn job as its workgroups see it (lrq_tn.h): TN_WAVES wavefronts per
// workgroup, 128 columns x a token slice each.
constexpr int TN_WAVES = 4;
struct TnArgs {
  const uint16_t* p;   // [M, C] bf16
  const uint16_t* q;   // [M, ldq] bf16, columns j < R
  int64_t M, C, ldq;
  int R;
  int64_t m_per;       // tokens per slice (multiple of 128)
  float* partial;      // [splits][C][rp]
  int tiles, blocks;   // column tiles of 128, tiles x slices
  float* out;          // the result out[c * sc + j * sj] (j < R)
  int64_t sc, sj;
  int splits;          // token slices; one slice writes out directly
  uint32_t* cnt;       // [tiles][TN_WAVES] arrival counters, zero on entry and exit
};

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
  float* part;           // lrq_gemm.hip split-depth partials [S][m][e] (gemm_split_floats), or null
  int splits, spl;       // set by lrq_gemm.hip: depth ranges and steps per range
  // lrq_gemm_mid.hip with the token-side LoRA factor formed in the same
  // launch (fold != 0, rank 8 to 32, a multiple of 8): the first fold_wgs workgroups (a
  // multiple of 8) form bf16(fscale . act . F) for 64-token groups over
  // fold_slices depth slices of MID_FOLD_KT (F = lact: forward A [l, r],
  // backward B [r, l]), sum the slices in order, store it to fout
  // [m][fout_ld] and publish a stamped ready flag per group; the tiles read
  // it after the flag. lw is then the raw weight-side factor (forward B
  // [r, e], backward A [e, r]). fpart holds the slices' f32 partials
  // [fold_slices][round_up(m, 64)][rp]; fcnt is the counter area (zero on
  // entry and exit; the epoch only grows).
  int fold, fold_wgs, fold_slices;
  float fscale;
  uint16_t* fout;
  int fout_ld;
  float* fpart;
  uint32_t* fcnt;
  // The backward with the fold also runs the weight gradients' token
  // reductions (dB = t^T dy, dA = x^T u; lrq_tn.h) in tn_blocks workgroups
  // after the tiles: job tj[0]'s blocks, then tj[1]'s. Job tn_da (or none,
  // -1) is dA: its blocks wait for the ready flags of their token slice's
  // groups and read u at device scope. Plans from mid_tn_plan; counters in
  // the counter area past the fold's [0, 2 G).
  TnArgs tj[2];
  int tn_blocks, tn_da;
  // lrq_gemm_mid.hip with depth ranges (msplit in 2 .. MID_MAX_SPLIT): each
  // tile's depth in msplit ranges of mspl stages (a multiple of 4; the last
  // range to the end), one workgroup each; their f32 accumulators go to
  // `part` (msplit x tiles x tokens x 64), mcnt holds one arrival counter per
  // tile (zero on entry and exit). Set by lrq_gemm.hip's planner.
  int msplit, mspl;
  uint32_t* mcnt;
};

// lrq_gemm.hip: the forward for m > 16 and the input gradient, weight
// dequantized into registers. a.lw is the weight-side LoRA rows [e, rp]
// (B^T forward, A backward; zero-padded columns), a.lact is t or u [m, rp].
// The backward's a.wdata / a.wscale point at the transposed section.
// With fewer output tiles than CUs the depth is split into S ranges whose
// f32 partials a.part must hold: gemm_split_floats(m, e, depth) floats (0
// when the shape is not split).
hipError_t launch_fwd(hipStream_t st, int fmt, const GemmArgs& a);
hipError_t launch_bwd(hipStream_t st, int fmt, const GemmArgs& a);
int64_t gemm_split_floats(int64_t m, int64_t e, int64_t depth);
int get_num_cus();
// lrq_gemm_mid.hip: the same products on 64-row tiles of 64 or 128 tokens
// over the whole depth or a few depth ranges finished in the launch, 16
// rows per wavefront (MID_64, MID_128); lrq_gemm.hip's launchers take one
// when it is modelled faster (gemm_mid_tokens: its tile's tokens, or 0).
// With depth ranges the caller provides a.part (gemm_split_floats) and
// a.mcnt (mid_split_plan(...).tiles counters).
enum { MID_NONE = 0, MID_64 = 1, MID_128 = 2 };
constexpr int MID_MAX_SPLIT = 4;
constexpr int MID_MST = 4;  // the mid kernel's pipeline stages (a range is whole rounds of them)
// The mid-size tiles' depth ranges for a product (m tokens, e outputs,
// `depth`): S = 1 (whole depth) when the large tiles or one range per tile
// are modelled faster; tiles and the partial floats the ranges need.
struct MidSplit {
  int S, spl;
  int64_t tiles, floats;
};
MidSplit mid_split_plan(int64_t m, int64_t e, int64_t depth);
hipError_t launch_mid(hipStream_t st, int fmt, bool bwd, const GemmArgs& a, int variant);
int gemm_mid_tokens(int64_t m, int64_t e, int64_t depth);
// depth per slice of the folded factor's workgroups (GemmArgs.fold)
constexpr int MID_FOLD_KT = 384;
// the token slices of a weight-gradient job run inside the mid-size
// backward: the factor slice takes at most 16 KiB of LDS (ranks padded to 16 or 32)
constexpr int MID_TN_LDS = 16384;
// tuning and test hook (lrq_debug_gemm_path): 0 planned, 1 large tiles,
// 2 MID_64, 3 MID_128
void set_gemm_path(int path);

// lrq_skinny.hip: the forward for m <= 16 in one launch. Split workgroups
// stream the packed weight once and write f32 partials of x . W^T per
// reduction split ([S][m][n]) and, when a.rp > 0, workgroups over k slices
// write the partials of x . A ([TS][16][rp], from the down factor A [k, r]).
// The last workgroup to arrive at a block row of 64 outputs sums them in a
// fixed order and writes y = bf16(sc * base + t . B + bias) with
// t = bf16(scaling * x . A), and t itself ([m, r]) when t_out is set. a.lw
// is B [r, n]. `cnt` holds ceil(n / 64) <= LRQ_CNT_WORDS arrival counters,
// zero on entry; the kernel leaves them zero.
// With bwd, the same launch gives the input gradient for m <= 16 from the
// transposed section (GemmArgs of the backward, a plan of
// skinny_plan(k, n, rp, .)): dx = bf16(sum of partials + u . A^T) with
// u = bf16(scaling * dy . B^T) from the partials of dy . B^T (`A` is then
// B [r, n]), written to t_out as [m, rp]; a.lw is A [k, r].
struct SkinnyPlan {
  int S, KS;  // reduction splits of the base, 64-wide blocks per split
  int TS;     // k slices of t (0 without LoRA)
  int64_t KT; // k per t slice (a multiple of 32)
  int full;   // a forward may run whole-depth workgroups (k_skf) instead of splits
};
// arrival counters at the start of every workspace (zeroed when allocated):
// block rows at [0, SK_MAX_NB), then, one 128-byte line each, the count of
// finished t slices, the launch epoch (t is published stamped with it), the
// epilogue count and the failure flag (set when an epilogue gave up waiting
// for t; lrq_sync reports it)
constexpr int64_t LRQ_CNT_WORDS = 16384;
constexpr size_t LRQ_CNT_BYTES = (size_t)LRQ_CNT_WORDS * 4;
constexpr int64_t SK_MAX_NB = LRQ_CNT_WORDS - 160;
constexpr int64_t SK_TCNT = LRQ_CNT_WORDS - 128, SK_EPOCH = LRQ_CNT_WORDS - 96, SK_DCNT = LRQ_CNT_WORDS - 64,
                  SK_FAIL = LRQ_CNT_WORDS - 32;
static_assert(LRQ_MAX_LORA_TOKENS <= (SK_MAX_NB - 8) * 16,
              "the t and u kernels keep one arrival counter per 16 tokens");
SkinnyPlan skinny_plan(int64_t n, int64_t k, int rp, int num_cus);
// test hook (lrq_debug_force_wait_timeout): later launches wait for a stamp
// that is never published, 16 polls at most
void set_force_wait_timeout(bool on);
bool force_wait_timeout();
size_t skinny_ws_bytes(const SkinnyPlan& p, int64_t m, int64_t n, int rp);
// The backward's LoRA factor gradients, folded into its launch (null: not
// formed): dA = x^T . u (f32 [k, r]) from the forward input x [m, k] and
// dB = t^T . dy (f32 [r, n]) from the forward's t [m, r].
struct SkGrads {
  const uint16_t* x;
  const uint16_t* t;
  float* da;
  float* db;
};
hipError_t launch_skinny(hipStream_t st, int fmt, bool bwd, const GemmArgs& a, const uint16_t* A,
                         const SkinnyPlan& p, float* part, float* tpart, uint32_t* cnt, float scaling,
                         uint16_t* t_out, const SkGrads& gr = SkGrads{});

// lrq_lora.hip
// A split of a LoRA reduction: `tiles` output tiles x `splits` slices of
// `per` columns (nt) or tokens (tn).
struct LoraPlan {
  int64_t tiles;
  int64_t per;
  int splits;
  int lw;  // nt: wavefronts (16 tokens each) per workgroup, 4 or 8
};
LoraPlan lora_plan_nt(int64_t M, int64_t C, int rp);
LoraPlan lora_plan_tn(int64_t M, int64_t C, int rp, int64_t other_c = 0);
// tn slices that fit the mid-size backward's LDS (MID_TN_LDS for the factor
// slice): as few token slices as that allows
LoraPlan mid_tn_plan(int64_t M, int64_t C, int rp);
// out = bf16(s * sum over slices of p[m, c] * q(j, c)) as [M, rp] (columns
// >= r zero) and/or [M, r], with q(j, c) = q[j * ldq + c] when qrow (B [r, n]),
// else q[c * ldq + j] (A [k, r]); entries j >= R read as zero. One launch:
// the slices write f32 partials (plan.splits * round_up(M, 128) * rp floats)
// and the last slice to finish each 16-token group sums them in slice order;
// cnt holds 8 * plan.tiles <= SK_MAX_NB counters, zero on entry and exit.
// With fr set,
// the launch also writes the fused GEMM's weight-side LoRA rows fr [N, rp]
// (columns >= r zero): B^T from B [r, N], or (b_rows) A [N, r] itself,
// divided by bdiv[n] (bdiv_rows) or bdiv[0] when bdiv is set (an fp8 weight
// scale).
struct NtFinish {
  uint32_t* cnt;
  float s;
  int r;
  uint16_t* out;       // [M, rp] or null
  uint16_t* out_user;  // [M, r] or null
  const uint16_t* B;
  int64_t N;
  int b_rows;
  uint16_t* fr;        // or null
  const float* bdiv;
  int bdiv_rows;
};
hipError_t launch_lora_nt(hipStream_t st, const uint16_t* p, const uint16_t* q, bool qrow, int64_t ldq,
                          int R, int64_t M, int64_t C, int rp, const LoraPlan& plan, float* partial,
                          const NtFinish& fin);
// out[c * sc + j * sj] = sum over tokens of p[m, c] * q[m * ldq + j] (f32)
// for c < C, j < R (columns j >= R of q read as zero). One or two such jobs
// per launch (the first job's workgroups are dispatched first). Token slices
// write f32 partials (plan.splits * C * rp floats; a single slice writes out
// directly) and the last slice to finish each 32-column group sums them in
// slice order; cnt holds 4 counters per 128-column tile of the jobs together
// (<= SK_MAX_NB), zero on entry and exit.
struct TnSpec {
  const uint16_t* p;
  const uint16_t* q;
  int64_t ldq, M, C;
  int R;
  LoraPlan plan;
  float* partial;
  float* out;
  int64_t sc, sj;
};
hipError_t launch_lora_tn(hipStream_t st, const TnSpec* jobs, int njobs, int rp, uint32_t* cnt);
// The job's workgroup arguments, its counters at cnt.
TnArgs tn_args(const TnSpec& j, uint32_t* cnt);

// lrq_probe.hip: a streaming read of `bytes` (a multiple of 16) with one
// 32-bit value per workgroup to out (probe_read_grid(bytes) of them)
int probe_read_grid(int64_t bytes);
hipError_t launch_stream_read(hipStream_t st, const void* data, int64_t bytes, uint32_t* out);

// kernel ids for the profiler (lrq_profile_*)
enum {
  KID_QUANT_INT4 = 0,
  KID_QUANT_FP8,
  KID_DEQUANT,
  KID_FWD_MAIN,
  KID_BWD_DX,
  KID_LORA_T,
  KID_LORA_U,
  KID_LORA_DA,
  KID_LORA_DB,
  KID_BLOCK,
  KID_LORA_DADB,
  KID_QUANT_INT8,
  KID_COUNT
};
