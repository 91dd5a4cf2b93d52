// The token reduction of the LoRA weight gradients as one workgroup's work,
// shared by the standalone launch (lrq_lora.hip) and the mid-size input
// gradient that runs it in its own launch (lrq_gemm_mid.hip):
//
//   out[c, j] = sum over tokens m of p[m, c] * q[m, j]
//   dA = x^T . u  (p = x, q = u),  dB = t^T . dy  (p = dy, q = t)
//
// (the weight gradients of src/lora.rs:199-203's two linears.)
//
// The reduction runs over tokens, which are strided in p. A workgroup (four
// wavefronts) owns 128 columns and one token slice; wavefront w takes tokens
// [128 it + 32 w, +32) of every 128-token chunk. Each lane loads an
// 8 (tokens) x 8 (columns) block with eight 16-byte loads and transposes it
// in registers (byte permutes), so every load is a contiguous 256-byte run
// per 16 lanes; the token-major factor q is transposed once into LDS. The
// wavefronts' accumulators are combined in a fixed order through an LDS
// buffer, in column rounds that fit it; a slice writes f32 partials, and
// the last slice of a column group to arrive sums the slices in order (one
// slice writes the result directly).
#pragma once

#include "lrq_common.h"
#include "lrq_kernels.h"

namespace {

constexpr int TW = TN_WAVES;  // wavefronts per tn workgroup
constexpr int TNT = 64 * TW;

// Transpose-pack: the 16-bit element `e` (0..7) of eight 8-element rows into
// one 8-element vector (rows in order).
LRQ_DEV u32x4 column8(const u32x4 (&v)[8], int e) {
  const int d = e >> 1;
  const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
  u32x4 o;
  o[0] = __builtin_amdgcn_perm(v[1][d], v[0][d], sel);
  o[1] = __builtin_amdgcn_perm(v[3][d], v[2][d], sel);
  o[2] = __builtin_amdgcn_perm(v[5][d], v[4][d], sel);
  o[3] = __builtin_amdgcn_perm(v[7][d], v[6][d], sel);
  return o;
}

// device-scope (sc1) accesses of the partials the last slice reads
LRQ_DEV void store_dev(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
LRQ_DEV void store16_dev(rsrc_t r, uint32_t off, const u32x4& v) { __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 16); }
LRQ_DEV u32x4 bload16_dev(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16); }
LRQ_DEV uint32_t add_dev(uint32_t* c) { return __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
LRQ_DEV void zero_dev(uint32_t* c) { __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// Block `bid` of job `a` (column tile bid % a.tiles, token slice
// bid / a.tiles). sQ holds the factor slice, RP (a.m_per + 8) bf16 (the
// plan keeps it within QBYTES); red is the combine buffer of RBYTES (it may
// be sQ itself: the slice is dead by then). QDEV: the factor was written
// in the same launch, so it is read at device scope (past the per-XCD L2s;
// a.ldq a multiple of 8). `poison`: the factor is not trustworthy (a wait
// for it ran out), so the slice's sums are NaN.
template <int NJT, int QBYTES, int RBYTES, bool QDEV>
LRQ_DEV void tn_block(const TnArgs& a, int bid, uint16_t* sQ, float* red, bool poison) {
  constexpr int RP = 16 * NJT;
  // combine rounds: RCOLS columns at a time (128 when the buffer holds a
  // rank tile of all of them), RT rank tiles at a time
  constexpr int RCOLS = (TW * 128 * 16 * 4 <= RBYTES) ? 128 : 64;
  static_assert(TW * RCOLS * 16 * 4 <= RBYTES, "the combine buffer holds one rank tile of a column round");
  constexpr int NH = 128 / RCOLS;
  constexpr int CPW = RCOLS / TW;  // columns a wavefront sums per round
  static_assert(QBYTES >= RP * (128 + 8) * 2, "the factor slice holds at least 128 tokens");
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t c0 = (int64_t)(bid % a.tiles) * 128;
  const int split = bid / a.tiles;
  const int64_t m_lo = split * a.m_per;
  const int64_t m_hi = min(a.M, m_lo + a.m_per);
  const int64_t C = a.C;
  const int l16 = lane & 15, g = lane >> 4;
  const int64_t toks = m_hi - m_lo;

  const int SQ = (int)a.m_per + 8;
  const rsrc_t rpv = make_rsrc(a.p + m_lo * C, clamp_bytes(toks * C * 2));
  const int64_t col = c0 + l16 * 8;
  const uint32_t coff = (col < C) ? (uint32_t)(col * 2) : LRQ_OOB;

  f32x4 acc[8][NJT];
#pragma unroll
  for (int q = 0; q < 8; ++q)
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt) acc[q][jt] = acc_zero4();

  const int64_t nchunks = (toks + 127) / 128;
  u32x4 pv[2][8];
  auto load = [&](int set, int64_t it) {
    const int64_t mrow = it * 128 + wv * 32 + g * 8;  // slice-relative token of row 0
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t off = opaque_u32(coff + (uint32_t)((mrow + i) * C * 2));
      pv[set][i] = bload16(rpv, off);
    }
  };
  auto compute = [&](int set, int64_t it) {
    const int64_t mrow = it * 128 + wv * 32 + g * 8;
    bf16x8 fq[NJT];
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt) fq[jt] = as_bf16x8(ld16(sQ + (jt * 16 + l16) * SQ + mrow));
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const bf16x8 fa = as_bf16x8(column8(pv[set], q));
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt) acc[q][jt] = mfma16(fa, fq[jt], acc[q][jt]);
    }
  };

  load(0, 0);  // overlaps the factor staging
  // factor slice q [m_lo, m_hi) x R -> LDS as [j][m - m_lo] (stride SQ):
  // 8 (tokens) x 8 (j) blocks, loaded as rows and transposed in registers
  if ((a.ldq & 7) == 0) {
    const rsrc_t rq = make_rsrc(a.q + m_lo * a.ldq, clamp_bytes(toks * a.ldq * 2));
    const int jb = RP / 8;
    for (int blk = tid; blk < jb * (int)(a.m_per / 8); blk += TNT) {
      const int j0 = (blk % jb) * 8, mm = (blk / jb) * 8;
      u32x4 v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t off = opaque_u32(j0 < a.ldq ? (uint32_t)(((mm + i) * a.ldq + j0) * 2) : LRQ_OOB);
        v[i] = QDEV ? bload16_dev(rq, off) : bload16(rq, off);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        u32x4 cv = column8(v, e);
        if (j0 + e >= a.R) cv = (u32x4){0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(sQ + (j0 + e) * SQ + mm) = cv;
      }
    }
  } else {
    for (int64_t id = tid; id < (int64_t)RP * a.m_per; id += TNT) {
      const int j = (int)(id % RP);
      const int64_t mm = id / RP;
      uint16_t v = 0;
      if (j < a.R && mm < toks) v = a.q[(m_lo + mm) * a.ldq + j];
      sQ[j * SQ + mm] = v;
    }
  }
  __syncthreads();

  int64_t it = 0;
  for (; it + 1 < nchunks; it += 2) {
    load(1, it + 1);
    compute(0, it);
    load(0, it + 2);
    compute(1, it + 1);
  }
  if (it < nchunks) compute(0, it);
  if (poison) {
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt) acc[q][jt] = (f32x4){__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")};
  }
  __syncthreads();  // every read of the factor slice is done (red may be it)

  // combine the wavefronts (fixed order); accumulator row 4g+v of MFMA q is
  // column c0 + 8*(4g+v) + q. Per round, RT rank tiles (all when they fit)
  // of RCOLS columns go through LDS; each thread then sums four consecutive
  // rank entries of a column and stores them together. Wavefront w sums
  // columns h RCOLS + [CPW w, CPW w + CPW) of round h.
  const rsrc_t rpart = make_rsrc(a.partial + (int64_t)split * C * RP, clamp_bytes(C * RP * 4));
  constexpr int RT = (TW * RCOLS * RP * 4 <= RBYTES) ? NJT : 1;  // rank tiles per round
  constexpr int RW = 16 * RT;                                     // rank entries per round
  constexpr int PL = RCOLS * RW / 1024;                           // items of four per lane
#pragma unroll
  for (int jr = 0; jr < NJT; jr += RT) {
#pragma unroll
    for (int h = 0; h < NH; ++h) {
#pragma unroll
      for (int jt = 0; jt < RT; ++jt)
#pragma unroll
        for (int q = 0; q < 8; ++q)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int cl = 8 * (4 * g + v) + q - h * RCOLS;
            if (NH == 1 || (cl >= 0 && cl < RCOLS)) red[(wv * RCOLS + cl) * RW + jt * 16 + l16] = acc[q][jr + jt][v];
          }
      __syncthreads();
#pragma unroll
      for (int k = 0; k < PL; ++k) {
        const int id = wv * 64 * PL + k * 64 + lane;
        const int cl = id / (RW / 4), jl = (id % (RW / 4)) * 4;
        f32x4 sum = *reinterpret_cast<const f32x4*>(red + cl * RW + jl);
#pragma unroll
        for (int w = 1; w < TW; ++w) sum += *reinterpret_cast<const f32x4*>(red + (w * RCOLS + cl) * RW + jl);
        const int j = jr * 16 + jl;
        const int64_t c = c0 + h * RCOLS + cl;
        if (c < C) {
          if (a.splits == 1) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (j + e < a.R) a.out[c * a.sc + (int64_t)(j + e) * a.sj] = sum[e];
          } else {
            store16_dev(rpart, (uint32_t)((c * RP + j) * 4), __builtin_bit_cast(u32x4, sum));
          }
        }
      }
      __syncthreads();
    }
  }
  if (a.splits == 1) return;
  // count this wavefront's 32 columns done in this slice once its stores are
  // acknowledged (no barrier); the last wavefront to arrive sums the slices
  // in order, NE entries of four per lane, every load of a batch of SB
  // slices issued before the first sum
  __builtin_amdgcn_s_waitcnt(0);
  uint32_t* const ctr = a.cnt + (bid % a.tiles) * TW + wv;
  uint32_t old = 0;
  if (lane == 0) old = add_dev(ctr);
  if (__builtin_amdgcn_readfirstlane(old) + 1 != (uint32_t)a.splits) return;
  if (lane == 0) zero_dev(ctr);
  constexpr int NE = 32 * RP / 4 / 64, SB = 16 / NE;
  const rsrc_t rp_ = make_rsrc(a.partial, clamp_bytes((int64_t)a.splits * C * RP * 4));
  // the wavefront's owned column of item e
  auto ocol = [&](int e) -> int64_t {
    const int oc = e / (RP / 4);
    return c0 + (oc / CPW) * RCOLS + wv * CPW + oc % CPW;
  };
  f32x4 v[NE];
#pragma unroll
  for (int k = 0; k < NE; ++k) v[k] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = 0; s0 < a.splits; s0 += SB) {  // slices in order
    u32x4 pv2[NE][SB];
#pragma unroll
    for (int k = 0; k < NE; ++k) {
      const int e = k * 64 + lane;
      const int64_t c = ocol(e);
      const int j = (e % (RP / 4)) * 4;
#pragma unroll
      for (int u = 0; u < SB; ++u)
        pv2[k][u] = bload16_dev(rp_, opaque_u32(s0 + u < a.splits && c < C
                                                    ? (uint32_t)((((int64_t)(s0 + u) * C + c) * RP + j) * 4)
                                                    : LRQ_OOB));
    }
#pragma unroll
    for (int k = 0; k < NE; ++k)
#pragma unroll
      for (int u = 0; u < SB; ++u) v[k] += __builtin_bit_cast(f32x4, pv2[k][u]);
  }
#pragma unroll
  for (int k = 0; k < NE; ++k) {
    const int e = k * 64 + lane;
    const int64_t c = ocol(e);
    const int j = (e % (RP / 4)) * 4;
    if (c >= C) continue;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (j + q < a.R) a.out[c * a.sc + (int64_t)(j + q) * a.sj] = v[k][q];
  }
}

}  // namespace
