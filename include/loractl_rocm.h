/*
 * loractl_rocm.h — C ABI of libloractl_rocm.so, the MI355X (gfx950) kernels
 * for loractl's quantized frozen-base LoRA linear.
 *
 * Reference interfaces replaced (laurigates/loractl, crates/loractl-core):
 *   - QuantBackend::quant_matmul_t (src/quant.rs:172-178) and its Autodiff
 *     override QuantMatmulT (src/quant.rs:210-263)
 *       -> lrq_quant_matmul_t / lrq_quant_matmul_t_bwd
 *   - site() = BaseLinear::forward + LoraAdapters::apply
 *     (src/mmdit.rs:483-536, src/adapters.rs:75-85, src/lora.rs:199-203)
 *       -> lrq_lora_fwd / lrq_lora_bwd (the fused drop-in: base + delta)
 *   - quantize_linear_weight (src/quant.rs:74-82) -> lrq_quantize_int4 (Q4S)
 *     and lrq_quantize_int8 (Q8S, the Quant::Int8 knob, src/quant.rs:156-162)
 *   - dequantize to f32 (src/quant.rs:232, :250) -> lrq_dequant
 *   - e4m3fn LUT decode * scale (src/fp8.rs:39-56, :279-329) -> lrq_dequant
 *     on an LRQ_FMT_FP8 weight
 *   - fp8 repack encoder (reference/fp8_reference.py:83-91; no counterpart in
 *     the crate) -> lrq_quantize_fp8
 *
 * Conventions
 *   - Every tensor pointer is a DEVICE pointer owned by the caller; the
 *     library never frees it. Row-major, densely packed, 16-byte aligned.
 *   - bf16 tensors are passed as uint16_t bit patterns.
 *   - Calls are stream-ordered and asynchronous on the context's stream
 *     (lrq_set_stream); call lrq_sync or synchronize the stream to wait.
 *   - Every call returns 0 on success or a negative LRQ_E* code; the message
 *     is in lrq_last_error(ctx). No C++ exception crosses the ABI. Shape and
 *     layout violations return LRQ_EINVAL (the reference panics there:
 *     src/quant.rs:76-80), never a silent fallback.
 *   - A context belongs to one host thread at a time; distinct contexts may
 *     be used concurrently. Hot calls allocate only when the context's
 *     workspace must grow (pre-size it with lrq_reserve); while the stream
 *     is being captured into a graph they return LRQ_EINVAL instead of
 *     growing it. Once a call has been captured on a context, a later
 *     growth (lrq_reserve or a hot call with a larger shape) keeps the old
 *     workspace allocated until lrq_destroy, so graphs captured earlier
 *     stay valid; replays of one graph, and eager calls on the same
 *     context, are ordered by the stream like any other calls.
 *
 * Weight layouts (file layout [d_out = n, d_in = k], as QuantLinear keeps it,
 * src/mmdit.rs:413-444):
 *   LRQ_FMT_INT4: data = uint8 [n, k/2]; byte j of a row holds k=2j in its low
 *     nibble and k=2j+1 in its high nibble, each nibble storing q+8 with
 *     q in [-7, 7]; scales = f32 [n, k/group]; dequant = q * scale (f32).
 *   LRQ_FMT_FP8: data = e4m3fn bytes [n, k]; scales = f32 [n] (per_channel)
 *     or [1]; dequant = LUT[byte] * scale (f32).
 *   Those row layouts (LRQ_LAYOUT_ROWS) are the interchange format. The fused
 *   kernels read LRQ_LAYOUT_BLOCKED, produced once per weight by
 *   lrq_weight_block: 64 (n) x 64 (k) blocks contiguous in memory, block
 *   (nb, kb) at (nb * KB + kb) * block bytes with KB = ceil(k / 64); inside a
 *   block the rows keep the row-layout byte order (int4: 32 bytes per row,
 *   fp8 and int8: 64). int4 and int8 scales become [NB][Gp][64]
 *   (NB = ceil(n/64), Gp = 64*KB/group); fp8 scales are unchanged. Padding
 *   rows/columns hold q = 0 with scale 0 (int4, int8) or byte 0 (fp8). A
 *   transposed section of the same byte size follows, read by the
 *   input-gradient kernel (its reduction runs along n): the same blocking
 *   applied to W^T [k, n] (block (kb, nb) at (kb * NB + nb) * block bytes,
 *   rows along k), int4 nibbles holding q in two's complement (int8 bytes as
 *   in the row layout), and for int4 and int8 a second scale table
 *   ST [KGt][NB*64] (KGt = ceil(64*KB/group), ST[kg][n] = scale of row n,
 *   group kg) after the [NB][Gp][64] one. The blocked weight thus takes
 *   twice the packed bytes (38 MB for an int4 12288 x 3072 weight).
 *   LoRA factors in burn layout: A = [k, r] (d_in x rank), B = [r, n].
 */
#ifndef LORACTL_ROCM_H
#define LORACTL_ROCM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LRQ_ABI_VERSION 1

enum {
  LRQ_OK = 0,
  LRQ_EINVAL = -1,       /* bad shape, alignment, group size or argument */
  LRQ_EUNSUPPORTED = -2, /* valid request this build does not implement */
  LRQ_EHIP = -3,         /* a HIP runtime call failed */
  LRQ_ENOMEM = -4        /* device allocation for the workspace failed */
};

enum { LRQ_FMT_INT4 = 1, LRQ_FMT_FP8 = 2, LRQ_FMT_INT8 = 3 };
enum { LRQ_LAYOUT_ROWS = 0, LRQ_LAYOUT_BLOCKED = 1 };

typedef struct lrq_ctx lrq_ctx;

/* A frozen base weight: plain pointers and sizes, no ownership. */
typedef struct lrq_weight {
  int32_t format;       /* LRQ_FMT_INT4, LRQ_FMT_FP8 or LRQ_FMT_INT8 */
  int32_t group;        /* int4, int8: block size along k, a power of two >= 32 dividing k */
  int64_t n;            /* d_out */
  int64_t k;            /* d_in (a multiple of 32) */
  const void* data;     /* device: packed int4 [n, k/2], fp8 bytes [n, k] or int8 [n, k] */
  const float* scales;  /* device: int4, int8 [n, k/group]; fp8 [n] or [1] */
  int32_t per_channel;  /* fp8: 1 when scales has n entries, 0 for one scalar */
  int32_t layout;       /* LRQ_LAYOUT_ROWS or LRQ_LAYOUT_BLOCKED */
  const float* bias;    /* device f32 [n] or NULL (src/mmdit.rs:426-427) */
} lrq_weight;

/* Library version (LRQ_ABI_VERSION). */
int lrq_version(void);

/* Create a context on HIP device `device`; it owns a workspace and starts
 * on the device's null stream. */
int lrq_create(int device, lrq_ctx** out);
int lrq_destroy(lrq_ctx* ctx);

/* Run subsequent calls on `stream` (a hipStream_t; NULL is the null stream). */
int lrq_set_stream(lrq_ctx* ctx, void* stream);

/* Wait for the context's stream, then report a failure the few-token
 * kernels (m <= 16) flagged on the device: an epilogue whose bounded wait
 * for t (u) ran out, which also writes NaN to the outputs it owns. A
 * reported failure returns LRQ_EHIP once; the call then waits for the whole
 * device, clears the flag and resets the arrival counters (the context's
 * and the device's no-alloc scratch), so later calls start clean. */
int lrq_sync(lrq_ctx* ctx);
const char* lrq_last_error(const lrq_ctx* ctx);

/* Tokens per call of the LoRA calls (lrq_lora_fwd, lrq_lora_bwd) for m > 16:
 * the t and u kernels keep one arrival counter per 16 tokens. A larger m
 * returns LRQ_EUNSUPPORTED; split the batch. */
#define LRQ_MAX_LORA_TOKENS 259456

/* Pre-size the workspace for calls with up to m tokens, n outputs, k inputs
 * and rank r, so that later hot calls do not allocate. */
int lrq_reserve(lrq_ctx* ctx, int64_t m, int64_t n, int64_t k, int64_t r);

/* quantize_linear_weight (src/quant.rs:74-82) at Q4S with block `group`:
 * w f32 [n, k] -> packed [n, k/2] + scales [n, k/group], bit-exact with the
 * closed form scale = absmax/7, q = clamp(round_half_away(w/scale), -7, 7). */
int lrq_quantize_int4(lrq_ctx* ctx, const float* w, int64_t n, int64_t k, int64_t group,
                      uint8_t* packed, float* scales);

/* The same at Q8S (src/quant.rs:156-162 maps Quant::Int8 to it): w f32 [n, k]
 * -> int8 q [n, k] + scales [n, k/group], scale = absmax/127,
 * q = clamp(round_half_away(w/scale), -127, 127). */
int lrq_quantize_int8(lrq_ctx* ctx, const float* w, int64_t n, int64_t k, int64_t group,
                      int8_t* q, float* scales);

/* fp8 repack (reference/fp8_reference.py:83-91): scale = max(amax/448, 1e-12)
 * per tensor or per output row, byte = RNE e4m3fn of w/scale, saturating to
 * +-448, sign kept. scales has n entries (per_channel) or 1. */
int lrq_quantize_fp8(lrq_ctx* ctx, const float* w, int64_t n, int64_t k, int per_channel,
                     uint8_t* bytes, float* scales);

/* fp8 checkpoint tensor -> int4 on the device: e4m3fn bytes [n, k] and their
 * f32 scale (one value, or one per output row when per_channel) decode to
 * the f32 LUT[byte] * scale of src/fp8.rs:306-318, which is quantized as
 * lrq_quantize_int4 does (src/quant.rs:74-82); the reference's load pass
 * does both on the host, one tensor at a time, through an f32 copy
 * (src/diffusion_trainer.rs:1143-1169). Bit-identical to lrq_dequant of the
 * fp8 weight followed by lrq_quantize_int4. */
int lrq_requantize_fp8_int4(lrq_ctx* ctx, const uint8_t* bytes, const float* scale, int per_channel, int64_t n,
                            int64_t k, int64_t group, uint8_t* packed, float* scales);

/* Sizes of the blocked layout of a weight, both sections: data bytes and
 * scale count (0 for fp8, whose scales keep their shape). No device work. */
int lrq_weight_blocked_size(int format, int64_t n, int64_t k, int64_t group, int64_t* data_bytes,
                            int64_t* scale_count);

/* Re-lay a LRQ_LAYOUT_ROWS weight into LRQ_LAYOUT_BLOCKED (data_out of
 * data_bytes, scales_out of scale_count floats; fp8 scales are not copied).
 * A one-time step per frozen weight (no counterpart in the reference: burn
 * keeps its packed storage private, src/quant.rs:57-60). */
int lrq_weight_block(lrq_ctx* ctx, const lrq_weight* rows, uint8_t* data_out, float* scales_out);

/* Dequantize the whole weight to f32 [n, k] (src/quant.rs:232; fp8.rs:306-318).
 * Debug/parity surface: bit-exact with the CPU definition. */
int lrq_dequant(lrq_ctx* ctx, const lrq_weight* w, float* out);

/* The bf16 GEMM operand the fused kernels feed to the matrix cores:
 * bf16_rne(dequant) for int4 and int8; the exact e4m3fn value (no scale)
 * for fp8. */
int lrq_dequant_bf16(lrq_ctx* ctx, const lrq_weight* w, uint16_t* out);

/* QuantBackend::quant_matmul_t (src/quant.rs:172-178): y[m, n] = x[m, k] .
 * dequant(w)^T (+ bias), bf16 in/out, f32 accumulation. The fused calls
 * (this and the three below) take a LRQ_LAYOUT_BLOCKED weight. */
int lrq_quant_matmul_t(lrq_ctx* ctx, const lrq_weight* w, const uint16_t* x, int64_t m,
                       uint16_t* y);

/* QuantMatmulT::backward (src/quant.rs:221-235): dx[m, k] = dy[m, n] . dequant(w). */
int lrq_quant_matmul_t_bwd(lrq_ctx* ctx, const lrq_weight* w, const uint16_t* dy, int64_t m,
                           uint16_t* dx);

/* The fused site forward (src/mmdit.rs:526-536 with a registered delta):
 *   y = x . dequant(w)^T (+ bias) + scaling * (x . A) . B
 * x [m, k], A [k, r], B [r, n], y [m, n], all bf16. When t_out is not NULL it
 * receives t = scaling * x . A as bf16 [m, r], the activation lrq_lora_bwd
 * needs. 1 <= r <= 64. */
int lrq_lora_fwd(lrq_ctx* ctx, const lrq_weight* w, const uint16_t* x, int64_t m,
                 const uint16_t* a, const uint16_t* b, int64_t r, float scaling, uint16_t* y,
                 uint16_t* t_out);

/* Bytes of the fixed scratch array of lrq_lora_fwd_noalloc, per GPU. */
#define LRQ_NOALLOC_SCRATCH_BYTES (32u << 20)

/* lrq_lora_fwd without any allocation. No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same
 * arguments, kernels and results as lrq_lora_fwd; its workspace is a
 * file-scope device array of LRQ_NOALLOC_SCRATCH_BYTES held by every GPU
 * the library runs on until the process ends, so it calls no hipMalloc,
 * hipFree or event creation. Its first 64 KiB hold the few-token kernels'
 * arrival counters; a shape whose forward needs more scratch than the rest
 * returns LRQ_EINVAL. Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (two streams, two contexts, two threads)
 * race and must be ordered by the caller. */
int lrq_lora_fwd_noalloc(lrq_ctx* ctx, const lrq_weight* w, const uint16_t* x, int64_t m,
                         const uint16_t* a, const uint16_t* b, int64_t r, float scaling, uint16_t* y,
                         uint16_t* t_out);

/* The fused site backward (gradients to x, A, B; none to the frozen weight):
 *   u  = scaling * dy . B^T
 *   dx = dy . dequant(w) + u . A^T          bf16 [m, k]
 *   dA = x^T . u                            f32  [k, r]
 *   dB = t^T . dy   (t from lrq_lora_fwd)   f32  [r, n]
 * Any of dx, da, db may be NULL to skip that output. */
int lrq_lora_bwd(lrq_ctx* ctx, const lrq_weight* w, const uint16_t* x, const uint16_t* dy,
                 int64_t m, const uint16_t* a, const uint16_t* b, int64_t r, float scaling,
                 const uint16_t* t, uint16_t* dx, float* da, float* db);

/* Per-kernel timing: when enabled, every launch is bracketed by HIP events
 * on the launch stream; lrq_profile_read returns the summed milliseconds and
 * the launch count for kernel id `kid` (0 <= kid < lrq_profile_count()). */
int lrq_profile_enable(lrq_ctx* ctx, int on);
int lrq_profile_reset(lrq_ctx* ctx);
int lrq_profile_count(void);
const char* lrq_profile_name(int kid);
int lrq_profile_read(lrq_ctx* ctx, int kid, double* total_ms, int64_t* launches);

/* Repeat, n times, the context's last launch of kernel `kid` among the
 * fused calls' kernels (fwd_main, bwd_dx, lora_t, lora_u, lora_da, lora_db,
 * lora_dadb), with the same arguments and buffers, on the context's stream,
 * so that one kernel can be timed alone (a graph of back-to-back repeats).
 * The buffers of that launch must still be allocated; a workspace growth
 * forgets the kept launches, and each forward (backward) call forgets those
 * of the kernels its pass may launch, so only the pass's latest call's
 * launches repeat (a kernel that call did not launch is refused with
 * LRQ_EINVAL: at ranks 8 to 32 (multiples of 8) on the mid-size tiles, one bwd_dx launch
 * also forms u, dA and dB). A repeat writes the same outputs again while
 * the buffers it reads hold what they held at the launch: the workspace is
 * shared by the passes (the backward reuses the forward's slot of the B^T
 * rows for A), so a forward kernel repeated after a backward reads other
 * values (same work, other results). */
int lrq_profile_relaunch(lrq_ctx* ctx, int kid, int n);

/* Measurement probe, no counterpart in the reference: read `bytes` (a
 * multiple of 16, 16-byte aligned) of device memory once, as a plain
 * streaming read with 16-byte loads (its per-workgroup checksums go to the
 * workspace). Timed by the caller, it is the box's measured read rate for a
 * buffer of that size, the ceiling beside the HBM peak for the few-token
 * kernels. */
int lrq_probe_stream_read(lrq_ctx* ctx, const void* data, int64_t bytes);

/* Test hook, no counterpart in the reference: with on != 0, later
 * few-token launches (in this process) give their epilogues' bounded wait
 * for t a stamp that is never published and a cap of 16 polls, so every
 * such epilogue gives up, as a lost t would make it: the kernels still end,
 * the outputs are NaN and lrq_sync reports the flag. on = 0 restores the
 * normal wait. For tests of the failure path only. */
int lrq_debug_force_wait_timeout(int on);

/* Tuning and test hook, no counterpart in the reference: which kernel the
 * fused products of m > 16 tokens take in this process. 0 (the default) the
 * planned one; 1 the 256-token tiles (split in depth when too few); 2 and 3
 * the 64-row tiles of 64 or 128 tokens (depth ranges as planned); 4 and 5
 * the same tiles with at least two depth ranges wherever the depth has two
 * whole rounds of their pipeline. Every path computes the same products; a workspace sized by lrq_reserve under one
 * setting grows on the next hot call if another needs more. */
int lrq_debug_gemm_path(int path);

#ifdef __cplusplus
}
#endif

#endif /* LORACTL_ROCM_H */
