/*
 * lrq_oracle.c — CPU restatement of loractl's quantized frozen-base LoRA
 * linear. TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py are the only callers. The product path
 * (loractl_amd/, libloractl_rocm.so) never links or calls this file.
 *
 * Every function cites the reference behaviour it restates (paths are
 * relative to the reference checkout, laurigates/loractl):
 *
 *   quantize      crates/loractl-core/src/quant.rs:47-82 (scheme + entry),
 *                 tests/quant.rs:152-171 (closed form, rounding budget),
 *                 reference/quant_int4_reference.py:45-56 (scale = absmax/qmax)
 *   dequantize    quant.rs:232,250 (q*s into f32)
 *   chunk rows    quant.rs:102-117
 *   fp8 decode    crates/loractl-core/src/fp8.rs:39-56 (LUT), fp8.rs:279-329
 *                 (LUT[b]*scale, scalar or per-output-row)
 *   fp8 encode    reference/fp8_reference.py:83-91 (amax/448, RNE cast)
 *   linear fwd    quant.rs:172-178 (x * dequant(wq)^T), adapters.rs:75-85 and
 *                 lora.rs:199-203 (base_out + s * B(A(x)))
 *   linear bwd    quant.rs:221-235 (grad_x = grad * dequant(wq)) plus the
 *                 autodiff of the two bias-free LoRA Linears (lora.rs:199-203)
 *
 * Pinning (what checks each function, see tests/test_oracle.py):
 *   quantize/dequant: reference goldens quant_int{4,8}_golden.json (bit-exact
 *     dq), roundtrip bound of tests/quant.rs:141-229, brute-force nearest level.
 *   fp8 decode: fp8_lut_golden.json (256 entries), fp8_dequant_golden.json.
 *   fp8 encode: byte pairs from the reference fixtures (fp8_pairs.npz) and a
 *     brute-force nearest-value search over the decode table.
 *   linear fwd/bwd: quant golden y (1e-5), lora_toy.json (20 SGD steps), and
 *     finite-difference gradients on tiny shapes.
 *
 *   cpu_baseline dequant (lrq_o_cpu_dequant_int4 / _int8): bit-identical to
 *     dequant_int4 / dequant_q above (test_cpu_baseline_*_matches_oracle).
 *
 * Numbers: f32 storage, f64 accumulation for the parity oracle; the
 * cpu_baseline dequant (lrq_o_cpu_dequant_int4, lrq_o_cpu_dequant_int8)
 * follows the reference's own CPU algorithm: materialize the f32
 * dequantized weight, then f32 GEMMs (those run in numpy's cache-blocked
 * SGEMM; oracle/__init__.py).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------ */
/* bf16 helpers (round-to-nearest-even, NaN kept quiet)                 */
/* ------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

EXPORT uint16_t lrq_o_f32_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

EXPORT float lrq_o_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

EXPORT void lrq_o_round_bf16(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = lrq_o_f32_to_bf16(in[i]);
}

/* ------------------------------------------------------------------ */
/* Block-symmetric integer quantization (quant.rs:47-82)               */
/* ------------------------------------------------------------------ */

/*
 * w [N,K] f32 in file layout [d_out, d_in]; blocks of g contiguous values
 * along K (quant.rs:52 uses g=32; the block lies strictly inside a row).
 * scale = absmax / qmax in f32 (burn's 2*absmax/(2*qmax) is bit-identical);
 * q = clamp(round_half_away(w / scale), -qmax, qmax) (Rust f32::round).
 * An all-zero block gets scale 0 and q 0 (burn's behaviour there is not
 * visible from the reference; dequant gives 0 either way).
 * Returns 0, or -1 when K % g != 0 (the reference panics: quant.rs:76-80).
 */
EXPORT int lrq_o_quantize(const float* w, int64_t N, int64_t K, int64_t g,
                          int qmax, int8_t* q, float* scales) {
  if (g <= 0 || K % g != 0) return -1;
  const int64_t nb = K / g;
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t b = 0; b < nb; ++b) {
      const float* blk = w + n * K + b * g;
      float amax = 0.0f;
      for (int64_t i = 0; i < g; ++i) {
        float a = fabsf(blk[i]);
        if (a > amax) amax = a;
      }
      float s = amax / (float)qmax;
      scales[n * nb + b] = s;
      for (int64_t i = 0; i < g; ++i) {
        int v = 0;
        if (s != 0.0f) {
          float r = roundf(blk[i] / s);
          if (r > (float)qmax) r = (float)qmax;
          if (r < (float)-qmax) r = (float)-qmax;
          v = (int)r;
        }
        q[n * K + b * g + i] = (int8_t)v;
      }
    }
  }
  return 0;
}

/* dq = q * s in f32 (one rounding) — quant.rs:232,250 dequantize to F32. */
EXPORT void lrq_o_dequant_q(const int8_t* q, const float* scales, int64_t N,
                            int64_t K, int64_t g, float* out) {
  const int64_t nb = K / g;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k)
      out[n * K + k] = (float)q[n * K + k] * scales[n * nb + k / g];
}

/*
 * This build's packed int4 layout (the reference does not pin one, its
 * storage is backend-internal: quant.rs:57-60). Row n of W occupies K/2
 * bytes; byte j holds k=2j in its low nibble and k=2j+1 in its high nibble;
 * each nibble stores q+8 (offset binary, q in [-7,7] -> 1..15, 8 is zero).
 */
EXPORT void lrq_o_pack_int4(const int8_t* q, int64_t N, int64_t K, uint8_t* packed) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t j = 0; j < K / 2; ++j) {
      uint8_t lo = (uint8_t)(q[n * K + 2 * j] + 8) & 0xF;
      uint8_t hi = (uint8_t)(q[n * K + 2 * j + 1] + 8) & 0xF;
      packed[n * (K / 2) + j] = (uint8_t)(lo | (hi << 4));
    }
}

EXPORT void lrq_o_unpack_int4(const uint8_t* packed, int64_t N, int64_t K, int8_t* q) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t j = 0; j < K / 2; ++j) {
      uint8_t b = packed[n * (K / 2) + j];
      q[n * K + 2 * j] = (int8_t)((int)(b & 0xF) - 8);
      q[n * K + 2 * j + 1] = (int8_t)((int)(b >> 4) - 8);
    }
}

EXPORT void lrq_o_dequant_int4(const uint8_t* packed, const float* scales,
                               int64_t N, int64_t K, int64_t g, float* out) {
  const int64_t nb = K / g;
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      uint8_t b = packed[n * (K / 2) + k / 2];
      int q = (int)((k & 1) ? (b >> 4) : (b & 0xF)) - 8;
      out[n * K + k] = (float)q * scales[n * nb + k / g];
    }
}

/* quant.rs:102-117: balanced row chunks keeping each f32 transient under the
 * byte threshold. Writes up to max_out counts, returns the chunk count. */
EXPORT int64_t lrq_o_dequant_chunk_rows(int64_t d_out, int64_t d_in, uint64_t chunk_bytes,
                                        int64_t* rows, int64_t max_out) {
  uint64_t full = (uint64_t)d_out * (uint64_t)d_in * 4u;
  if (chunk_bytes == 0 || full <= chunk_bytes || d_out <= 1) {
    if (max_out > 0) rows[0] = d_out;
    return 1;
  }
  uint64_t row_bytes = (uint64_t)d_in * 4u;
  uint64_t max_rows = chunk_bytes / row_bytes;
  if (max_rows < 1) max_rows = 1;
  int64_t n_chunks = (int64_t)((d_out + max_rows - 1) / max_rows);
  int64_t base = d_out / n_chunks, rem = d_out % n_chunks;
  for (int64_t i = 0; i < n_chunks && i < max_out; ++i) rows[i] = (i < rem) ? base + 1 : base;
  return n_chunks;
}

/* ------------------------------------------------------------------ */
/* fp8 e4m3fn (fp8.rs:39-56, fp8.rs:279-329, fp8_reference.py:83-91)   */
/* ------------------------------------------------------------------ */

/* Decode one byte: subnormal sign*(m/8)*2^-6, normal sign*(1+m/8)*2^(e-7),
 * NaN only at 0x7f/0xff, no infinities (fp8.rs:45-56). */
EXPORT float lrq_o_fp8_decode(uint8_t b) {
  float sign = (b & 0x80) ? -1.0f : 1.0f;
  int e = (b >> 3) & 0xF, m = b & 7;
  if (e == 15 && m == 7) return NAN;
  if (e == 0) return sign * ((float)m / 8.0f) * ldexpf(1.0f, -6);
  return sign * (1.0f + (float)m / 8.0f) * ldexpf(1.0f, e - 7);
}

/* Encode one f32 as e4m3fn with round-to-nearest-even on the exact value,
 * the sign kept (so -0 and tiny negatives give 0x80), saturating to +-448.
 * NaN maps to 0x7f with its sign. */
EXPORT uint8_t lrq_o_fp8_encode(float x) {
  uint8_t sign = signbit(x) ? 0x80 : 0;
  if (isnan(x)) return (uint8_t)(sign | 0x7F);
  double a = fabs((double)x);
  if (a >= 448.0) return (uint8_t)(sign | 0x7E);
  if (a < ldexp(1.0, -6)) {
    /* subnormal grid: multiples of 2^-9; m == 8 rolls into the first normal */
    double m = nearbyint(a * 512.0);
    return (uint8_t)(sign | (uint8_t)m);
  }
  int e;
  frexp(a, &e);          /* a = f * 2^e, f in [0.5,1) */
  e -= 1;                /* a = (1+frac) * 2^e */
  double mant = a / ldexp(1.0, e) - 1.0; /* exact in double */
  double m = nearbyint(mant * 8.0);
  if (m >= 8.0) { m = 0.0; e += 1; }
  int code = ((e + 7) << 3) | (int)m;
  if (code > 0x7E) code = 0x7E;
  return (uint8_t)(sign | code);
}

/* scale = max(amax/448, 1e-12) per tensor (per_channel=0) or per output row,
 * byte = encode(w / scale) (fp8_reference.py:83-91). */
EXPORT void lrq_o_fp8_quantize(const float* w, int64_t N, int64_t K, int per_channel,
                               uint8_t* bytes, float* scales) {
  if (per_channel) {
    for (int64_t n = 0; n < N; ++n) {
      float amax = 0.0f;
      for (int64_t k = 0; k < K; ++k) { float a = fabsf(w[n * K + k]); if (a > amax) amax = a; }
      float s = amax / 448.0f;
      if (s < 1e-12f) s = 1e-12f;
      scales[n] = s;
      for (int64_t k = 0; k < K; ++k) bytes[n * K + k] = lrq_o_fp8_encode(w[n * K + k] / s);
    }
  } else {
    float amax = 0.0f;
    for (int64_t i = 0; i < N * K; ++i) { float a = fabsf(w[i]); if (a > amax) amax = a; }
    float s = amax / 448.0f;
    if (s < 1e-12f) s = 1e-12f;
    scales[0] = s;
    for (int64_t i = 0; i < N * K; ++i) bytes[i] = lrq_o_fp8_encode(w[i] / s);
  }
}

/* f32 = LUT[b] * scale, scale scalar (n_scale==1) or one per output row
 * (fp8.rs:306-318: row = len/len(scale), scale[i / row]). */
EXPORT void lrq_o_fp8_dequant(const uint8_t* bytes, int64_t N, int64_t K,
                              const float* scales, int64_t n_scale, float* out) {
  for (int64_t n = 0; n < N; ++n)
    for (int64_t k = 0; k < K; ++k) {
      float s = (n_scale == 1) ? scales[0] : scales[n];
      out[n * K + k] = lrq_o_fp8_decode(bytes[n * K + k]) * s;
    }
}

/* ------------------------------------------------------------------ */
/* Linear forward / backward, f64 accumulation (parity oracle)          */
/* ------------------------------------------------------------------ */

/*
 * Y[M,N] = X[M,K] * Wdq[N,K]^T + s * (X * A[K,r]) * B[r,N] (+ bias[N]).
 * quant.rs:175-176 (base), adapters.rs:82 (base_out + delta),
 * lora.rs:199-203 (delta = s * B(A(x)), A/B in burn layout [d_in,r]/[r,d_out]).
 * T[M,r] = s * X * A is written when T != NULL (the value the backward needs).
 * A or B may be NULL (base only).
 */
EXPORT void lrq_o_linear_fwd(const float* X, const float* Wdq, const float* A, const float* B,
                             const float* bias, double s, int64_t M, int64_t N, int64_t K,
                             int64_t r, float* Y, float* T) {
  double* t = (double*)calloc((size_t)(M * (r > 0 ? r : 1)), sizeof(double));
  if (A && B && r > 0) {
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m)
      for (int64_t j = 0; j < r; ++j) {
        double acc = 0.0;
        for (int64_t k = 0; k < K; ++k) acc += (double)X[m * K + k] * (double)A[k * r + j];
        t[m * r + j] = s * acc;
        if (T) T[m * r + j] = (float)(s * acc);
      }
  }
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k) acc += (double)X[m * K + k] * (double)Wdq[n * K + k];
      if (A && B && r > 0)
        for (int64_t j = 0; j < r; ++j) acc += t[m * r + j] * (double)B[j * N + n];
      if (bias) acc += (double)bias[n];
      Y[m * N + n] = (float)acc;
    }
  free(t);
}

/*
 * Backward of lrq_o_linear_fwd with respect to X, A and B (the frozen weight
 * gets no gradient: quant.rs:221-235, tests/quant.rs:302-310).
 *   U  = s * dY * B^T                     [M,r]
 *   dX = dY * Wdq + U * A^T               [M,K]
 *   dA = X^T * U                          [K,r]
 *   dB = (s * X * A)^T * dY = T^T * dY    [r,N]
 * Any of dX/dA/dB may be NULL.
 */
EXPORT void lrq_o_linear_bwd(const float* X, const float* Wdq, const float* A, const float* B,
                             double s, const float* dY, int64_t M, int64_t N, int64_t K,
                             int64_t r, float* dX, float* dA, float* dB) {
  double* u = (double*)calloc((size_t)(M * (r > 0 ? r : 1)), sizeof(double));
  double* t = (double*)calloc((size_t)(M * (r > 0 ? r : 1)), sizeof(double));
  if (A && B && r > 0) {
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m)
      for (int64_t j = 0; j < r; ++j) {
        double acc = 0.0, acc2 = 0.0;
        for (int64_t n = 0; n < N; ++n) acc += (double)dY[m * N + n] * (double)B[j * N + n];
        for (int64_t k = 0; k < K; ++k) acc2 += (double)X[m * K + k] * (double)A[k * r + j];
        u[m * r + j] = s * acc;
        t[m * r + j] = s * acc2;
      }
  }
  if (dX) {
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m)
      for (int64_t k = 0; k < K; ++k) {
        double acc = 0.0;
        for (int64_t n = 0; n < N; ++n) acc += (double)dY[m * N + n] * (double)Wdq[n * K + k];
        if (A && B)
          for (int64_t j = 0; j < r; ++j) acc += u[m * r + j] * (double)A[k * r + j];
        dX[m * K + k] = (float)acc;
      }
  }
  if (dA && A && B) {
#pragma omp parallel for schedule(static)
    for (int64_t k = 0; k < K; ++k)
      for (int64_t j = 0; j < r; ++j) {
        double acc = 0.0;
        for (int64_t m = 0; m < M; ++m) acc += (double)X[m * K + k] * u[m * r + j];
        dA[k * r + j] = (float)acc;
      }
  }
  if (dB && A && B) {
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; ++n)
      for (int64_t j = 0; j < r; ++j) {
        double acc = 0.0;
        for (int64_t m = 0; m < M; ++m) acc += t[m * r + j] * (double)dY[m * N + n];
        dB[j * N + n] = (float)acc;
      }
  }
  free(u);
  free(t);
}

/* ------------------------------------------------------------------ */
/* CPU baseline: the reference's own CPU algorithm in f32               */
/* (dequantize the whole weight to f32 on every forward and every        */
/* backward, quant.rs:232-233, quant.rs:250-251). The f32 GEMMs around it */
/* run in numpy's cache-blocked SGEMM (oracle/__init__.py, CpuStepInt4).  */
/* ------------------------------------------------------------------ */

/* Wdq[N,K] = q * scale in f32 from the packed row layout, OpenMP over rows.
 * Returns the number of threads used. */
EXPORT int lrq_o_cpu_dequant_int4(const uint8_t* packed, const float* scales, int64_t g, int64_t N, int64_t K,
                                  float* Wdq) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const int64_t nb = K / g;
    const uint8_t* row = packed + n * (K / 2);
    const float* sc = scales + n * nb;
    float* out = Wdq + n * K;
    for (int64_t k = 0; k < K; k += 2) {
      const uint8_t b = row[k / 2];
      const float s = sc[k / g];
      out[k] = (float)((int)(b & 0xF) - 8) * s;
      out[k + 1] = (float)((int)(b >> 4) - 8) * s;
    }
  }
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* The same for an int8 (Q8S) weight: Wdq[N,K] = q * scale in f32 from q [N,K]
 * and scales [N, K/g], OpenMP over rows. Returns the number of threads used. */
EXPORT int lrq_o_cpu_dequant_int8(const int8_t* q, const float* scales, int64_t g, int64_t N, int64_t K,
                                  float* Wdq) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    const int8_t* row = q + n * K;
    const float* sc = scales + n * (K / g);
    float* out = Wdq + n * K;
    for (int64_t k = 0; k < K; ++k) out[k] = (float)row[k] * sc[k / g];
  }
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
