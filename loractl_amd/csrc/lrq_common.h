// Shared device helpers for the gfx950 kernels: bf16 packing, int4/int8/fp8
// decode, and the matrix-core (MFMA) fragment layouts used by every GEMM.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "loractl_rocm.h"

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define LRQ_DEV __device__ __forceinline__

// ---------------------------------------------------------------- bf16
// Round-to-nearest-even f32 -> bf16 bits for two values packed (lo, hi):
// one v_cvt_pk_bf16_f32 on gfx950.
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
LRQ_DEV uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

LRQ_DEV float bf16_lo(uint32_t v) { return __builtin_bit_cast(float, v << 16); }
LRQ_DEV float bf16_hi(uint32_t v) { return __builtin_bit_cast(float, v & 0xffff0000u); }

LRQ_DEV uint16_t f32_to_bf16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

// ---------------------------------------------------------------- int4
// One dword holds 8 nibbles (k = 0..7 of a run: byte j = k 2j | 2j+1 << 4),
// each q+8. Dequantize all 8 to f32 as fma(u, s, -8s) == RN((u-8)*s) ==
// RN(q*s), i.e. bit-identical to the f32 product q*s, then round to bf16.
// `nib` must be 0x0f0f0f0f; callers pass it from a kernel argument so the
// compiler keeps whole-byte extracts (v_cvt_f32_ubyte0..3) instead of
// narrowing them to bit-field extracts.
LRQ_DEV void dequant8_int4_f32(uint32_t w, float s, float f[8], uint32_t nib = 0x0f0f0f0fu) {
  const float nb = -8.0f * s;
  const uint32_t lo = w & nib;         // k = 0,2,4,6 in bytes 0..3
  const uint32_t hi = (w >> 4) & nib;  // k = 1,3,5,7
  f[0] = __builtin_fmaf((float)(lo & 0xffu), s, nb);
  f[1] = __builtin_fmaf((float)(hi & 0xffu), s, nb);
  f[2] = __builtin_fmaf((float)((lo >> 8) & 0xffu), s, nb);
  f[3] = __builtin_fmaf((float)((hi >> 8) & 0xffu), s, nb);
  f[4] = __builtin_fmaf((float)((lo >> 16) & 0xffu), s, nb);
  f[5] = __builtin_fmaf((float)((hi >> 16) & 0xffu), s, nb);
  f[6] = __builtin_fmaf((float)(lo >> 24), s, nb);
  f[7] = __builtin_fmaf((float)(hi >> 24), s, nb);
}

LRQ_DEV u32x4 dequant8_int4_bf16(uint32_t w, float s, uint32_t nib = 0x0f0f0f0fu) {
  float f[8];
  dequant8_int4_f32(w, s, f, nib);
  u32x4 o;
  o[0] = pack_bf16x2(f[0], f[1]);
  o[1] = pack_bf16x2(f[2], f[3]);
  o[2] = pack_bf16x2(f[4], f[5]);
  o[3] = pack_bf16x2(f[6], f[7]);
  return o;
}

// ---------------------------------------------------------------- int8
// Two dwords hold 8 two's-complement bytes (k = 0..7 of a run, byte j of
// dword d is k = 4d + j). Flipping the sign bits gives u = q + 128, and
// fma(u, s, -128s) == RN((u - 128) * s) == RN(q * s) (-128s is exact): the
// f32 product bit for bit, with one byte convert and one fma per value.
LRQ_DEV void dequant8_int8_f32(u32x2 w, float s, float f[8]) {
  const float nb = -128.0f * s;
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const uint32_t u = w[d] ^ 0x80808080u;
    f[4 * d] = __builtin_fmaf((float)(u & 0xffu), s, nb);
    f[4 * d + 1] = __builtin_fmaf((float)((u >> 8) & 0xffu), s, nb);
    f[4 * d + 2] = __builtin_fmaf((float)((u >> 16) & 0xffu), s, nb);
    f[4 * d + 3] = __builtin_fmaf((float)(u >> 24), s, nb);
  }
}

LRQ_DEV u32x4 dequant8_int8_bf16(u32x2 w, float s) {
  float f[8];
  dequant8_int8_f32(w, s, f);
  u32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return o;
}

// Eight two's-complement nibbles (value e at bits 4e .. 4e+3 of w, the
// backward's transposed int4 layout) as q / 16 in f32, exactly:
// v_cvt_off_f32_i4 reads the low 4 bits of its operand as a signed value and
// returns it divided by 16. Each convert takes its nibble by an SDWA byte
// select of w (even e) or of w rotated right by 4 (odd e: a v_alignbit,
// which the compiler does not fold into bit-field extracts as it does a
// shift; the bits rotated in sit in byte 3's upper nibble, which the convert
// ignores): one rotate and eight converts for eight values, against a
// bit-field extract and a convert per value. The caller multiplies by 16 x
// the scale: (q / 16) (16 s) rounds to the same f32 as q s, since both
// scalings by 16 are exact. Used by the mid-size and few-token kernels (the
// mid input gradient at C1: 39 -> 36 us); the large kernel's input gradient,
// one wavefront per SIMD, measured 7% slower with it and keeps the extracts.
LRQ_DEV void int4x8_to_f32_div16(uint32_t w, float f[8]) {
  const uint32_t h = __builtin_amdgcn_alignbit(w, w, 4);
  f[0] = __builtin_amdgcn_cvt_off_f32_i4((int)(w & 0xffu));
  f[1] = __builtin_amdgcn_cvt_off_f32_i4((int)(h & 0xffu));
  f[2] = __builtin_amdgcn_cvt_off_f32_i4((int)((w >> 8) & 0xffu));
  f[3] = __builtin_amdgcn_cvt_off_f32_i4((int)((h >> 8) & 0xffu));
  f[4] = __builtin_amdgcn_cvt_off_f32_i4((int)((w >> 16) & 0xffu));
  f[5] = __builtin_amdgcn_cvt_off_f32_i4((int)((h >> 16) & 0xffu));
  f[6] = __builtin_amdgcn_cvt_off_f32_i4((int)(w >> 24));
  f[7] = __builtin_amdgcn_cvt_off_f32_i4((int)(h >> 24));
}

// Four two's-complement bytes -> their integer values as f32 (exact).
LRQ_DEV void int8x4_to_f32(uint32_t w, float f[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) f[j] = (float)((int)(w << (24 - 8 * j)) >> 24);
}

// ---------------------------------------------------------------- fp8 e4m3fn
// Exact e4m3fn -> f32 (the value of src/fp8.rs:45-56's table): subnormal
// m*2^-9, normal (1+m/8)*2^(e-7), NaN at |b| == 0x7f, no infinities.
LRQ_DEV float fp8_e4m3fn_to_f32(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 24;
  const uint32_t e = (b >> 3) & 0xfu;
  const uint32_t m = b & 7u;
  float v;
  if (e == 0) {
    v = (float)m * 0.001953125f;  // m * 2^-9, exact
    v = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) | sign);
  } else if (e == 15 && m == 7) {
    v = __builtin_bit_cast(float, sign | 0x7fc00000u);
  } else {
    v = __builtin_bit_cast(float, sign | ((e + 120u) << 23) | (m << 20));
  }
  return v;
}

// Four e4m3fn bytes -> four f32 with the gfx950 converter (OCP e4m3fn:
// exact values, NaN at 0x7f/0xff). f[j] is byte j.
typedef float f32x2 __attribute__((ext_vector_type(2)));
LRQ_DEV void fp8x4_to_f32(uint32_t w, float f[4]) {
  const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  f[0] = lo[0];
  f[1] = lo[1];
  f[2] = hi[0];
  f[3] = hi[1];
}

// Four e4m3fn bytes -> four bf16 (exact: 3 mantissa bits fit bf16's 7).
// Returns two dwords of bf16 pairs (byte 0 in the low half of dword 0).
LRQ_DEV u32x2 fp8x4_to_bf16(uint32_t w) {
  float f[4];
  fp8x4_to_f32(w, f);
  u32x2 o;
  o[0] = pack_bf16x2(f[0], f[1]);
  o[1] = pack_bf16x2(f[2], f[3]);
  return o;
}

// ---------------------------------------------------------------- MFMA
// v_mfma_f32_32x32x16_bf16: A-role lane l supplies row (l & 31) and the 8
// reduction values at offset 8 * (l >> 5) of the 16-wide k slice; B-role
// lane l supplies column (l & 31) with the same k mapping. Accumulator
// element v of lane l is C[row = 8*(v>>2) + 4*(l>>5) + (v&3)][col = l & 31].
LRQ_DEV f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x32_bf16: A-role lane l supplies row (l & 15), 8 values at
// k offset 8 * (l >> 4); B-role likewise for column (l & 15). Accumulator
// element v of lane l is C[row = 4*(l>>4) + v][col = l & 15].
LRQ_DEV f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// A zero accumulator of its own, already in accumulator registers. When many
// loop-carried accumulators start from one shared constant zero, the register
// allocator rotates them through other registers on every iteration (dozens
// of v_accvgpr moves per trip, and a loop back edge on which the compiler
// left one read short of its MFMA wait states); a separate opaque zero per
// accumulator keeps every MFMA in place.
LRQ_DEV f32x4 acc_zero4() {
  f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
  asm volatile("" : "+a"(z));
  return z;
}

LRQ_DEV bf16x8 as_bf16x8(const u32x4& v) { return __builtin_bit_cast(bf16x8, v); }

LRQ_DEV u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
LRQ_DEV void st16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }
LRQ_DEV void st8(void* p, const u32x2& v) { *reinterpret_cast<u32x2*>(p) = v; }

// ---------------------------------------------------------------- workgroup order
// Workgroup ids are dealt round-robin over the 8 XCDs (each with its own L2);
// map them to a logical order in which XCD x owns a contiguous range.
LRQ_DEV int xcd_remap(int bid, int nblk) {
  const int q = nblk / 8, r = nblk % 8;
  const int x = bid % 8, i = bid / 8;
  return x * q + min(x, r) + i;
}

// ---------------------------------------------------------------- lane broadcast
// f[e] *= lane 8h + e of v's 16-lane row (e = 0..7, h = 0 or 1): the
// per-depth scales of a transposed weight fragment. Written as eight VOP2
// multiplies that take the row broadcast as their DPP operand, because the
// compiler fuses only some of its v_mov_b32_dpp broadcasts into the multiply
// (it left half of them as separate moves in the backward GEMM's main loop:
// 64 extra VALU instructions per two steps; written out, that kernel's
// input gradient takes 2.5% less time). The compiler does not see the DPP
// reads inside the asm: s_nop 1 supplies the 2 wait states a DPP read needs
// after a VALU write of its source, and tests/test_isa_hazards.py checks on
// the emitted code that no EXEC write comes within the 5 wait states a DPP
// instruction needs after one (s_nop 4 here measured 1.5% slower). volatile
// keeps the blocks where the source puts them (without it the compiler's
// placement measured slower). h is a constant once the callers' loops are
// unrolled.
#define LRQ_MUL_BCAST(I, L) \
  "v_mul_f32_dpp %" #I ", %8, %" #I " row_newbcast:" #L " row_mask:0xf bank_mask:0xf bound_ctrl:1\n"
LRQ_DEV void mul_row_bcast8(float (&f)[8], float v, int h) {
  if (h == 0)
    asm volatile("s_nop 1\n" LRQ_MUL_BCAST(0, 0) LRQ_MUL_BCAST(1, 1) LRQ_MUL_BCAST(2, 2) LRQ_MUL_BCAST(3, 3)
            LRQ_MUL_BCAST(4, 4) LRQ_MUL_BCAST(5, 5) LRQ_MUL_BCAST(6, 6) LRQ_MUL_BCAST(7, 7)
        : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7])
        : "v"(v));
  else
    asm volatile("s_nop 1\n" LRQ_MUL_BCAST(0, 8) LRQ_MUL_BCAST(1, 9) LRQ_MUL_BCAST(2, 10) LRQ_MUL_BCAST(3, 11)
            LRQ_MUL_BCAST(4, 12) LRQ_MUL_BCAST(5, 13) LRQ_MUL_BCAST(6, 14) LRQ_MUL_BCAST(7, 15)
        : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7])
        : "v"(v));
}
#undef LRQ_MUL_BCAST

// ---------------------------------------------------------------- buffer loads
// Raw buffer loads with a wave-uniform resource: an offset at or past
// num_records reads zeros, so bounds handling needs no branches.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t LRQ_OOB = 0x80000000u;  // an offset past any resource

// Hide a value's provenance from the optimizer (no instruction is emitted).
// Applied to a selected buffer offset, it keeps the compiler from sinking the
// load into the arms of the select, which would turn a branch-free step into
// divergent branches.
LRQ_DEV uint32_t opaque_u32(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// `base` and `bytes` must be wave-uniform; they are read from the first
// active lane so the descriptor provably lives in scalar registers (without
// that, the compiler may wrap every load in a per-lane loop).
LRQ_DEV rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = (uint64_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  void* u = (void*)(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(u, (short)0, __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}
LRQ_DEV u32x4 bload16(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }
LRQ_DEV u32x2 bload8(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0); }
LRQ_DEV uint32_t bload4(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0); }
// zero-extended 16-bit load
LRQ_DEV uint32_t bload2(rsrc_t r, uint32_t off) { return (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0); }
LRQ_DEV float bloadf(rsrc_t r, uint32_t off) { return __builtin_bit_cast(float, bload4(r, off)); }
LRQ_DEV uint32_t clamp_bytes(int64_t b) { return b <= 0 ? 0u : (b >= 0xffffffffll ? 0xffffffffu : (uint32_t)b); }

LRQ_DEV u32x4 zero4() { return (u32x4){0u, 0u, 0u, 0u}; }

typedef __attribute__((address_space(3))) void lds_void;

// Blocked-layout sizes (lrq_quant.hip writes the layout): data bytes and
// group-scale count (int4, int8; none for fp8).
LRQ_DEV void blocked_sizes_dev(int fmt, int64_t n, int64_t k, int64_t* data_bytes, int64_t* nscales,
                               int gshift) {
  const int64_t NB = (n + 63) / 64, KB = (k + 63) / 64;
  *data_bytes = NB * KB * 64 * (fmt == LRQ_FMT_INT4 ? 32 : 64);
  *nscales = (fmt != LRQ_FMT_FP8) ? NB * ((KB * 64) >> gshift) * 64 : 0;
}

// 8 consecutive bf16 (16 bytes) from global with a validity predicate.
LRQ_DEV u32x4 ld16_pred(const void* p, bool ok) {
  u32x4 z = {0u, 0u, 0u, 0u};
  return ok ? ld16(p) : z;
}
