/*
 * loractl_mmdit.h — C ABI of libloractl_mmdit.so, the attention-input
 * and modulation kernels of the double-stream MMDiT step driver on MI355X
 * (gfx950).
 *
 * These sit beside the quantized LoRA linear (loractl_rocm.h). The first
 * pair runs between a block's QKV linears and its attention and replaces,
 * per block, the reference's head split, QK-norm and RoPE on q and k
 * (crates/loractl-core/src/mmdit.rs:599-619: ZRmsNorm forward
 * :307-330 with its frozen zero-initialised gain, so gain 1, and the
 * consecutive-pair rotation apply_rope :385-399), done on the joint
 * text-then-image token sequence, with the gradient of the same map.
 *
 * The rest are the block's elementwise glue: modulated norms, gated
 * residuals and the MLP's GELU, forward and gradient.
 *
 * Conventions (as loractl_rocm.h): device pointers owned by the caller,
 * 16-byte aligned, row-major; bf16 as uint16_t bits; stream-ordered and
 * asynchronous on `stream` (a hipStream_t, NULL for the default stream);
 * 0 on success or a negative LRQ-style code (-1 invalid argument, -3 HIP
 * launch error), message in lmd_last_error(). Nothing is allocated.
 *
 * Shapes: h = heads * head_dim, head_dim 64 or 128, L = l_txt + l_img.
 *   qkv_txt [l_txt, 3h], qkv_img [l_img, 3h]: the QKV linears' outputs,
 *     each row [q | k | v], each part head-major [heads, head_dim].
 *   cos, sin f32 [L, head_dim / 2]: pair j of a token's head turns by the
 *     angle whose cosine and sine these hold.
 *   q, k, v bf16 [L, heads, head_dim]: text tokens first.
 *   rstd f32 [2, L, heads]: 1 / sqrt(mean(x^2) + eps) of each q and k head.
 */
#ifndef LORACTL_MMDIT_H
#define LORACTL_MMDIT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failed call on this host thread ("" if none). */
const char* lmd_last_error(void);

/* q = rope(x_q * rstd_q), k = rope(x_k * rstd_k), v = x_v, per head, in f32,
 * rounded once to bf16 (mmdit.rs:599-619 for one token sequence). */
int lmd_attn_prep_fwd(const uint16_t* qkv_txt, int64_t l_txt, const uint16_t* qkv_img, int64_t l_img,
                      int heads, int head_dim, const float* cos, const float* sin, float eps,
                      uint16_t* q, uint16_t* k, uint16_t* v, float* rstd, void* stream);

/* Gradient of lmd_attn_prep_fwd: from dq, dk, dv [L, heads, head_dim], the
 * forward's inputs and its rstd, writes d qkv_txt [l_txt, 3h] and
 * d qkv_img [l_img, 3h]. With g = rope^-1(dq) per head and n = rstd * x:
 * dx = rstd * (g - n * sum(g * n) / head_dim). */
int lmd_attn_prep_bwd(const uint16_t* dq, const uint16_t* dk, const uint16_t* dv, const uint16_t* qkv_txt,
                      int64_t l_txt, const uint16_t* qkv_img, int64_t l_img, int heads, int head_dim,
                      const float* cos, const float* sin, const float* rstd, uint16_t* dqkv_txt,
                      uint16_t* dqkv_img, void* stream);

/* Modulated RMSNorm of a block's stream (mmdit.rs:857-870: the prenorm and
 * postnorm ZRmsNorm, gain 1, then (scale + 1) * norm + shift), per row of
 * x [rows, h] with scale, shift [h] bf16:
 *   out = (scale + 1) * x / sqrt(mean(x^2) + eps) + shift, in f32, one rounding;
 * rstd f32 [rows] = 1 / sqrt(mean(x^2) + eps) for the gradient. h <= 4096,
 * h % 8 == 0. */
int lmd_modnorm_fwd(const uint16_t* x, int64_t rows, int h, const uint16_t* scale, const uint16_t* shift,
                    float eps, uint16_t* out, float* rstd, void* stream);

/* Number of partial rows the column sums of the two gradients below use for
 * `rows` rows: their `part` workspace is f32 [groups][2][h] (modnorm) or
 * [groups][h] (gated residual). */
int64_t lmd_colsum_groups(int64_t rows);

/* Gradient of lmd_modnorm_fwd: dx [rows, h] and the vector gradients
 * dscale = sum over rows of dh * n, dshift = sum of dh (bf16 [h]), each
 * summed in a fixed order (bitwise reproducible). With n = rstd * x and
 * g = dh * (scale + 1): dx = rstd * (g - n * mean(g * n)). */
int lmd_modnorm_bwd(const uint16_t* dh, const uint16_t* x, int64_t rows, int h, const uint16_t* scale,
                    const float* rstd, uint16_t* dx, uint16_t* dscale, uint16_t* dshift, float* part, void* stream);

/* Gradient of the gated residual y = x + gate * o (mmdit.rs:860-869) in o and
 * gate: d_o = dy * gate [rows, h], dgate = sum over rows of dy * o (bf16
 * [h], fixed order). The gradient in x is dy itself. */
int lmd_gated_residual_bwd(const uint16_t* dy, const uint16_t* o, int64_t rows, int h, const uint16_t* gate,
                           uint16_t* d_o, uint16_t* dgate, float* part, void* stream);

/* The gated residual itself: y = x + gate * o (mmdit.rs:860-869), x, o, y
 * [rows, h], gate bf16 [h]; f32 fma, one rounding. */
int lmd_gated_residual_fwd(const uint16_t* x, const uint16_t* o, int64_t rows, int h, const uint16_t* gate,
                           uint16_t* y, void* stream);

/* The driver's MLP activation (FLUX-style blocks; the reference's own
 * single-stream block uses SwiGLU): g = gelu_tanh(u) =
 * u (1 + tanh(sqrt(2/pi) (u + 0.044715 u^3))) / 2 elementwise over n bf16
 * values (n % 8 == 0), computed in f32 as u * sigmoid(2 z). */
int lmd_gelu_tanh_fwd(const uint16_t* u, int64_t n, uint16_t* g, void* stream);

/* Its gradient: du = dg * d gelu_tanh(u) / du. */
int lmd_gelu_tanh_bwd(const uint16_t* dg, const uint16_t* u, int64_t n, uint16_t* du, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LORACTL_MMDIT_H */
