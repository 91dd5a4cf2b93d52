// Attention inputs of a double-stream MMDiT block: per-head RMSNorm of q and
// k, RoPE on both, and the head split, fused into one pass over the two
// streams' QKV rows (and its gradient in one pass the other way).
//
// Work item = (token, 8 consecutive channels of one part). A head of 128
// channels is 16 consecutive lanes (64: 8), so the head's sum of squares is
// a reduction over an aligned lane group of the wavefront, and RoPE pair j
// (channels 2j, 2j+1) is always inside one lane. Every load and store is 16
// bytes and a wavefront's 64 lanes cover 1 KiB of one row: the kernel is an
// HBM stream (forward: 6h bytes read, 6h written per token; backward about
// 10h read, 6h written), with no LDS.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <string>

#include "loractl_mmdit.h"

// the message of the last failed call on this thread, for every lmd_ entry point
__attribute__((visibility("hidden"))) thread_local std::string lmd_err_msg;

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

#define LMD_DEV __device__ __forceinline__

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
LMD_DEV f32x4 ldf4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
LMD_DEV void st16(void* p, const u32x4& v) { *reinterpret_cast<u32x4*>(p) = v; }

// sum over the aligned group of LPH lanes
template <int LPH>
LMD_DEV float group_sum(float v) {
#pragma unroll
  for (int m = 1; m < LPH; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

struct PrepArgs {
  const uint16_t* qkv[2];  // text rows, image rows: [l, 3h]
  int64_t l_txt;
  int64_t items;           // L * h / 8
  int chunks;              // h / 8 (work items per part per token)
  int heads;
  const float* cos;
  const float* sin;
  float eps;
  // forward
  uint16_t* out[3];        // q, k, v [L, h]
  float* rstd;             // [2, L, heads]
  // backward
  const uint16_t* grad[3];  // dq, dk, dv [L, h]
  uint16_t* dqkv[2];        // [l, 3h] per stream
};

template <int LPH>
__global__ __launch_bounds__(256) void k_attn_prep_fwd(PrepArgs a) {
  constexpr int HD = LPH * 8;
  const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (item >= a.items) return;  // items is a multiple of LPH: whole heads leave together
  const int64_t tok = item / a.chunks;
  const int c = (int)(item - tok * a.chunks);
  const int sub = c % LPH, head = c / LPH;
  const int64_t h = (int64_t)a.chunks * 8;
  const bool txt = tok < a.l_txt;
  const uint16_t* row = a.qkv[txt ? 0 : 1] + (txt ? tok : tok - a.l_txt) * 3 * h;
  const u32x4 xq = ld16(row + c * 8), xk = ld16(row + h + c * 8), xv = ld16(row + 2 * h + c * 8);
  const f32x4 cs = ldf4(a.cos + tok * (HD / 2) + sub * 4), sn = ldf4(a.sin + tok * (HD / 2) + sub * 4);
  const int64_t o = tok * h + c * 8;
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    float f[8];
    unpack8(part ? xk : xq, f);
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(f[e], f[e], ss);
    ss = group_sum<LPH>(ss);
    const float r = rsqrtf(ss * (1.0f / HD) + a.eps);
    u32x4 y;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const float x0 = f[2 * p] * r, x1 = f[2 * p + 1] * r;
      y[p] = pack2(x0 * cs[p] - x1 * sn[p], x0 * sn[p] + x1 * cs[p]);
    }
    st16(a.out[part] + o, y);
    if (sub == 0) a.rstd[((int64_t)part * (a.items / a.chunks) + tok) * a.heads + head] = r;
  }
  st16(a.out[2] + o, xv);
}

template <int LPH>
__global__ __launch_bounds__(256) void k_attn_prep_bwd(PrepArgs a) {
  constexpr int HD = LPH * 8;
  const int64_t item = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (item >= a.items) return;
  const int64_t tok = item / a.chunks;
  const int c = (int)(item - tok * a.chunks);
  const int sub = c % LPH, head = c / LPH;
  const int64_t h = (int64_t)a.chunks * 8;
  const bool txt = tok < a.l_txt;
  const int64_t rt = txt ? tok : tok - a.l_txt;
  const uint16_t* row = a.qkv[txt ? 0 : 1] + rt * 3 * h;
  uint16_t* drow = a.dqkv[txt ? 0 : 1] + rt * 3 * h;
  const int64_t o = tok * h + c * 8;
  const u32x4 gq = ld16(a.grad[0] + o), gk = ld16(a.grad[1] + o), gv = ld16(a.grad[2] + o);
  const u32x4 xq = ld16(row + c * 8), xk = ld16(row + h + c * 8);
  const f32x4 cs = ldf4(a.cos + tok * (HD / 2) + sub * 4), sn = ldf4(a.sin + tok * (HD / 2) + sub * 4);
  const int64_t L = a.items / a.chunks;
#pragma unroll
  for (int part = 0; part < 2; ++part) {
    const float r = a.rstd[((int64_t)part * L + tok) * a.heads + head];
    float f[8], g[8];
    unpack8(part ? xk : xq, f);
    unpack8(part ? gk : gq, g);
    float d[8], dot = 0.0f;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      // the rotation's transpose
      d[2 * p] = g[2 * p] * cs[p] + g[2 * p + 1] * sn[p];
      d[2 * p + 1] = g[2 * p + 1] * cs[p] - g[2 * p] * sn[p];
      f[2 * p] *= r;
      f[2 * p + 1] *= r;
      dot = __builtin_fmaf(d[2 * p], f[2 * p], dot);
      dot = __builtin_fmaf(d[2 * p + 1], f[2 * p + 1], dot);
    }
    dot = group_sum<LPH>(dot) * (1.0f / HD);
    u32x4 y;
#pragma unroll
    for (int p = 0; p < 4; ++p)
      y[p] = pack2(r * (d[2 * p] - f[2 * p] * dot), r * (d[2 * p + 1] - f[2 * p + 1] * dot));
    st16(drow + part * h + c * 8, y);
  }
  st16(drow + 2 * h + c * 8, gv);
}

int fail(int code, const char* what) {
  lmd_err_msg = what;
  return code;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check(const uint16_t* t0, int64_t l_txt, const uint16_t* t1, int64_t l_img, int heads, int head_dim,
          const float* cos, const float* sin, PrepArgs& a) {
  if (l_txt < 0 || l_img < 0 || l_txt + l_img <= 0) return fail(-1, "token counts must be >= 0 with a positive sum");
  if (head_dim != 64 && head_dim != 128) return fail(-1, "head_dim must be 64 or 128");
  if (heads <= 0) return fail(-1, "heads must be positive");
  if ((l_txt > 0 && !t0) || (l_img > 0 && !t1) || !cos || !sin) return fail(-1, "null input pointer");
  if (!aligned16(t0) || !aligned16(t1) || !aligned16(cos) || !aligned16(sin))
    return fail(-1, "inputs must be 16-byte aligned");
  const int64_t h = (int64_t)heads * head_dim;
  a.qkv[0] = t0;
  a.qkv[1] = t1;
  a.l_txt = l_txt;
  a.chunks = (int)(h / 8);
  a.heads = heads;
  a.items = (l_txt + l_img) * (h / 8);
  a.cos = cos;
  a.sin = sin;
  if (a.items > ((int64_t)1 << 40)) return fail(-1, "too many tokens");
  return 0;
}

template <typename K>
int launch(K kern, const PrepArgs& a, void* stream) {
  const int64_t blocks = (a.items + 255) / 256;
  if (blocks > 0x7fffffff) return fail(-1, "grid too large");
  hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(-3, hipGetErrorString(e));
  return 0;
}

}  // namespace

extern "C" const char* lmd_last_error(void) { return lmd_err_msg.c_str(); }

extern "C" int lmd_attn_prep_fwd(const uint16_t* qkv_txt, int64_t l_txt, const uint16_t* qkv_img, int64_t l_img,
                                 int heads, int head_dim, const float* cos, const float* sin, float eps,
                                 uint16_t* q, uint16_t* k, uint16_t* v, float* rstd, void* stream) {
  PrepArgs a{};
  if (int rc = check(qkv_txt, l_txt, qkv_img, l_img, heads, head_dim, cos, sin, a)) return rc;
  if (!q || !k || !v || !rstd) return fail(-1, "null output pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v)) return fail(-1, "outputs must be 16-byte aligned");
  if (!(eps > 0.0f)) return fail(-1, "eps must be positive");
  a.eps = eps;
  a.out[0] = q;
  a.out[1] = k;
  a.out[2] = v;
  a.rstd = rstd;
  lmd_err_msg.clear();
  return head_dim == 128 ? launch(k_attn_prep_fwd<16>, a, stream) : launch(k_attn_prep_fwd<8>, a, stream);
}

extern "C" int lmd_attn_prep_bwd(const uint16_t* dq, const uint16_t* dk, const uint16_t* dv, const uint16_t* qkv_txt,
                                 int64_t l_txt, const uint16_t* qkv_img, int64_t l_img, int heads, int head_dim,
                                 const float* cos, const float* sin, const float* rstd, uint16_t* dqkv_txt,
                                 uint16_t* dqkv_img, void* stream) {
  PrepArgs a{};
  if (int rc = check(qkv_txt, l_txt, qkv_img, l_img, heads, head_dim, cos, sin, a)) return rc;
  if (!dq || !dk || !dv || !rstd || (l_txt > 0 && !dqkv_txt) || (l_img > 0 && !dqkv_img))
    return fail(-1, "null pointer");
  if (!aligned16(dq) || !aligned16(dk) || !aligned16(dv) || !aligned16(dqkv_txt) || !aligned16(dqkv_img))
    return fail(-1, "gradients must be 16-byte aligned");
  a.grad[0] = dq;
  a.grad[1] = dk;
  a.grad[2] = dv;
  a.rstd = const_cast<float*>(rstd);
  a.dqkv[0] = dqkv_txt;
  a.dqkv[1] = dqkv_img;
  lmd_err_msg.clear();
  return head_dim == 128 ? launch(k_attn_prep_bwd<16>, a, stream) : launch(k_attn_prep_bwd<8>, a, stream);
}
