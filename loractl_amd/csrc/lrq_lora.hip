// The low-rank (LoRA) side products of the fused linear, as matrix-core
// kernels that stream the big operand once and reduce deterministically:
//
//   t  = s . x  . A      [m, r]  (src/lora.rs:199-203, A-linear then scale)
//   u  = s . dy . B^T    [m, r]  (autodiff of the B-linear, input side)
//   dA = x^T . u         [k, r]  (weight grad of the A-linear)
//   dB = t^T . dy        [r, n]  (weight grad of the B-linear)
//
// All four read one large bf16 operand (x or dy, HBM-bound) against one
// small rank-wide factor. Two kernel shapes cover them:
//
//   nt (t, u): the reduction runs along the contiguous dimension of p (k for
//     x, n for dy). A workgroup owns 128 tokens and one column slice; the
//     factor slice (B rows as stored, or A transposed in registers) is
//     staged once in LDS and shared by the 8 wavefronts, each of which
//     streams its own 16 token rows (64-byte runs per row and load). Slices
//     write f32 partials and count themselves done per token tile; the last
//     slice of a tile sums them in slice order and writes the bf16 result
//     (in the same launch, as the few-token kernel finishes a block row:
//     device-scope stores acknowledged before the count, device-scope
//     loads). Every workgroup also copies its share of the fused GEMM's
//     weight-side factor rows (B^T or A, padded to rp).
//   tn (dA, dB): the reduction runs over tokens, which are strided in p.
//     Each lane loads an 8 (tokens) x 8 (columns) block with eight 16-byte
//     loads and transposes it in registers (byte permutes), so every load is
//     a contiguous 256-byte run per 16 lanes; the token-major factor (u or t)
//     is transposed once into LDS. Workgroups own 128 columns and a token
//     slice and write f32 partials; the last slice of a column tile sums the
//     slices in order and writes the result, in the same launch (both
//     reductions in one launch).
//
// Nothing depends on timing: every sum has a fixed order, and no workgroup
// waits for another.
#include <algorithm>

#include "lrq_common.h"
#include "lrq_kernels.h"
#include "lrq_tn.h"

namespace {

constexpr int LW = 8;          // nt: wavefronts per workgroup, at most (LoraPlan.lw: 4 or 8)

// ------------------------------------------------------------------ nt
struct NtArgs {
  const uint16_t* p;   // [M, C] bf16
  const uint16_t* q;   // QROW: [R, ldq], row j over c (B [r, n]); else [C, ldq], row c over j (A [k, r])
  int64_t M, C, ldq;
  int R;               // valid factor rank entries (the rest read as zero)
  int64_t c_per;       // columns per slice (multiple of 32)
  float* partial;      // [splits][M][rp] f32
  NtFinish f;
};

constexpr int NQ_BYTES = 100 * 1024;  // factor slice in LDS

// LDS row stride of the factor slice: whole 512-column runs plus 8 bf16 of
// padding (16 consecutive rows at one column then cover all banks)
LRQ_DEV int nt_stride(int64_t c_per) { return (int)((c_per + 511) / 512 * 512) + 8; }
// columns of the factor slice that fit in LDS at once (whole runs)
constexpr int nt_cap(int rp) { return ((NQ_BYTES / 2) / rp - 8) / 512 * 512; }

// Stage the factor slice [c_lo, c_hi) into LDS as sQ[j][c - c_lo] (stride
// SQ), zero outside j < R and c < c_hi. B rows are copied global -> LDS by
// buffer loads with an LDS destination, all issued at once (one load moves
// 512 columns of one row; a row's loads end on its stride's run boundary,
// and chunks past the slice or the rank read zeros). A arrives as 8 (c) x 8
// (j) blocks transposed in registers.
template <bool QROW, int RP>
LRQ_DEV void stage_factor(const NtArgs& a, int64_t c_lo, int64_t c_hi, int width, uint16_t* sQ, int SQ,
                          int nthreads) {
  const int tid = threadIdx.x;
  const int64_t cols = c_hi - c_lo;
  if (QROW && (a.ldq & 7) == 0) {
    const int lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6), nw = nthreads / 64;
    const rsrc_t rq = make_rsrc(a.q, clamp_bytes((int64_t)a.R * a.ldq * 2));
    const int runs = (width + 511) / 512;
    for (int t = wv; t < RP * runs; t += nw) {
      const int j = t / runs, c0 = (t % runs) * 512;
      const int cc = c0 + lane * 8;
      const uint32_t off = (j < a.R && cc < cols) ? (uint32_t)(((int64_t)j * a.ldq + c_lo + cc) * 2) : LRQ_OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (lds_void*)(sQ + j * SQ + c0), 16, opaque_u32(off), 0, 0, 0);
    }
  } else if (!QROW && (a.ldq & 7) == 0) {
    const int jb = RP / 8;
    for (int blk = tid; blk < jb * (width / 8); blk += nthreads) {
      const int j0 = (blk % jb) * 8, cc = (blk / jb) * 8;
      u32x4 v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v[i] = (u32x4){0u, 0u, 0u, 0u};
        if (j0 < a.ldq && cc + i < cols) v[i] = ld16(a.q + (c_lo + cc + i) * a.ldq + j0);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        u32x4 cv = column8(v, e);
        if (j0 + e >= a.R) cv = (u32x4){0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(sQ + (j0 + e) * SQ + cc) = cv;
      }
    }
  } else {
    for (int64_t id = tid; id < (int64_t)RP * width; id += nthreads) {
      const int j = (int)(id / width);
      const int64_t cc = id % width;
      uint16_t v = 0;
      if (j < a.R && cc < cols) v = QROW ? a.q[(int64_t)j * a.ldq + c_lo + cc] : a.q[(c_lo + cc) * a.ldq + j];
      sQ[j * SQ + cc] = v;
    }
  }
}

// The weight-side factor rows fr [N, rp] of the fused GEMM's LoRA epilogue
// (columns >= r zero): B^T from B [r, N], or (b_rows) A [N, r] row for row,
// divided by bdiv[n] (bdiv_rows) or bdiv[0] when set (an fp8 weight scale).
// Workgroup wg of nwg copies an equal contiguous share (so that no workgroup
// carries much of it); nothing in the launch reads them.
template <int RP>
LRQ_DEV void copy_factor_rows(const NtFinish& f, int64_t wg, int64_t nwg, int nthreads) {
  const int tid = threadIdx.x;
  if (!f.b_rows && (f.N & 7) == 0) {
    // B^T as 8 (n) x 8 (j) blocks: eight 16-byte row loads of B, transposed
    // in registers, eight 16-byte stores
    constexpr int JB = RP / 8;
    const int64_t total = f.N / 8 * JB, share = (total + nwg - 1) / nwg;
    const int64_t hi = min(total, (wg + 1) * share);
    for (int64_t bi = wg * share + tid; bi < hi; bi += nthreads) {
      const int j0 = (int)(bi % JB) * 8;
      const int64_t n0 = bi / JB * 8;
      u32x4 v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = j0 + i < f.r ? ld16(f.B + (int64_t)(j0 + i) * f.N + n0) : zero4();
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        u32x4 cv = column8(v, e);
        if (f.bdiv) {
          const float d = f.bdiv[f.bdiv_rows ? n0 + e : 0];
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const uint32_t lo = j0 + 2 * h < f.r ? f32_to_bf16_bits(bf16_lo(cv[h]) / d) : 0u;
            const uint32_t hi = j0 + 2 * h + 1 < f.r ? f32_to_bf16_bits(bf16_hi(cv[h]) / d) : 0u;
            cv[h] = lo | (hi << 16);
          }
        }
        st16(f.fr + (n0 + e) * RP + j0, cv);
      }
    }
  } else {
    const int64_t total = f.N * RP, share = (total + nwg - 1) / nwg;
    const int64_t hi = min(total, (wg + 1) * share);
    for (int64_t i2 = wg * share + tid; i2 < hi; i2 += nthreads) {
      const int64_t n = i2 / RP;
      const int j = (int)(i2 % RP);
      uint16_t v = j < f.r ? f.B[f.b_rows ? n * f.r + j : (int64_t)j * f.N + n] : (uint16_t)0;
      if (f.bdiv && j < f.r) {
        const float d = f.bdiv[f.bdiv_rows ? n : 0];
        v = f32_to_bf16_bits(__builtin_bit_cast(float, (uint32_t)v << 16) / d);
      }
      f.fr[i2] = v;
    }
  }
}

// partial[split][m][j] = sum over the slice's columns of p[m, c] * q(j, c).
// A workgroup owns 16 LWT tokens (16 per wavefront) and one column slice;
// the factor slice is staged once in LDS and shared by the LWT wavefronts,
// which each stream their own 16 token rows through a ring of D loads.
template <int NJT, bool QROW, int LWT>
__global__ void __launch_bounds__(64 * LWT) k_lora_nt(NtArgs a) {
  constexpr int LNT = 64 * LWT;
  constexpr int RP = 16 * NJT;
  __shared__ __attribute__((aligned(16))) uint16_t sQ[NQ_BYTES / 2];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int split = blockIdx.y;
  const int64_t c_lo = split * a.c_per;
  const int64_t c_hi = min(a.C, c_lo + a.c_per);
  const int64_t C = a.C;
  const int l16 = lane & 15, g = lane >> 4;
  // the slice is staged in sub-slices of at most nt_cap(RP) columns
  const int sub = (int)min(a.c_per, (int64_t)nt_cap(RP));
  const int SQ = nt_stride(sub);

  const int64_t m0 = (int64_t)blockIdx.x * (16 * LWT) + wv * 16;  // this wavefront's tokens
  const int64_t rows = max((int64_t)0, min((int64_t)16, a.M - m0));
  const rsrc_t rpv = make_rsrc(a.p + min(m0, a.M) * C, clamp_bytes(rows * C * 2));
  const uint32_t roff = (uint32_t)(l16 * C * 2);

  f32x4 acc[NJT];
#pragma unroll
  for (int jt = 0; jt < NJT; ++jt) acc[jt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};

  // chunks of 32 columns; lane group g reads 8 of them; chunks past the
  // sub-slice load zeros (out-of-range offsets) and add nothing
  constexpr int D = 8;
  u32x4 pv[D];
  auto load = [&](int k, int64_t s_lo, int64_t s_hi, int64_t it) {
    const int64_t c = s_lo + it * 32 + g * 8;
    pv[k] = bload16(rpv, opaque_u32(c < s_hi ? roff + (uint32_t)(c * 2) : LRQ_OOB));
  };
  auto compute = [&](int k, int64_t it) {
    const int cc = (int)(it * 32) + g * 8;  // sub-slice-relative; < sub + 32
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt) {
      const int off = min(cc, sub - 8);  // chunks past the sub-slice: zero p, any finite q
      acc[jt] = mfma16(as_bf16x8(pv[k]), as_bf16x8(ld16(sQ + (jt * 16 + l16) * SQ + off)), acc[jt]);
    }
  };
  for (int64_t s_lo = c_lo; s_lo < c_hi; s_lo += sub) {
    const int64_t s_hi = min(c_hi, s_lo + sub);
    const int64_t nchunks = (s_hi - s_lo + 31) / 32;
    // every wavefront's reads of the previous sub-slice are done
    if (s_lo != c_lo) __syncthreads();
    // the first loads overlap the factor staging
#pragma unroll
    for (int k = 0; k < D; ++k) load(k, s_lo, s_hi, k);
    stage_factor<QROW, RP>(a, s_lo, s_hi, sub, sQ, SQ, LNT);
    __syncthreads();
    for (int64_t it = 0; it < nchunks; it += D) {
#pragma unroll
      for (int k = 0; k < D; ++k) {
        compute(k, it + k);
        load(k, s_lo, s_hi, it + k + D);
      }
    }
  }

  // this wavefront's partial, in the accumulator's own layout (lane l's
  // f32x4 of rank tile jt: token 4g+v of the wavefront's 16, rank column
  // 16jt + l16), one 16-byte store per tile, in slot (split, wavefront)
  const NtFinish& f = a.f;
  const int splits = (int)gridDim.y;
  const int64_t nwv = (int64_t)gridDim.x * LWT, slot = (int64_t)blockIdx.x * LWT + wv;
  const rsrc_t rpart = make_rsrc(a.partial, clamp_bytes((int64_t)splits * nwv * RP * 64));
  auto poff = [&](int64_t sp, int jt) { return (uint32_t)((((sp * nwv + slot) * NJT + jt) * 64 + lane) * 16); };
#pragma unroll
  for (int jt = 0; jt < NJT; ++jt) store16_dev(rpart, poff(split, jt), __builtin_bit_cast(u32x4, acc[jt]));

  // count these 16 tokens done in this slice once the stores are
  // acknowledged (wavefront by wavefront: no barrier); the last wavefront
  // to arrive sums the slices in order, every load of a batch of SB slices
  // issued before the first sum
  __builtin_amdgcn_s_waitcnt(0);
  uint32_t old = 0;
  if (lane == 0) old = add_dev(f.cnt + slot);
  const bool last = __builtin_amdgcn_readfirstlane(old) + 1 == (uint32_t)splits;
  if (last) {
    if (lane == 0) zero_dev(f.cnt + slot);
    constexpr int SB = 16 / NJT;
    f32x4 sum[NJT];
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt) sum[jt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < splits; s0 += SB) {
      u32x4 pv[NJT][SB];
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt)
#pragma unroll
        for (int u = 0; u < SB; ++u) pv[jt][u] = bload16_dev(rpart, opaque_u32(s0 + u < splits ? poff(s0 + u, jt) : LRQ_OOB));
#pragma unroll
      for (int jt = 0; jt < NJT; ++jt)
#pragma unroll
        for (int u = 0; u < SB; ++u) sum[jt] += __builtin_bit_cast(f32x4, pv[jt][u]);
    }
#pragma unroll
    for (int jt = 0; jt < NJT; ++jt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t m = m0 + 4 * g + v;
        const int j = 16 * jt + l16;
        if (m >= a.M) continue;
        const uint16_t h = f32_to_bf16_bits(j < f.r ? sum[jt][v] * f.s : 0.0f);
        if (f.out) f.out[m * RP + j] = h;
        if (f.out_user && j < f.r) f.out_user[m * f.r + j] = h;
      }
  }

  if (f.fr)
    copy_factor_rows<RP>(f, (int64_t)blockIdx.y * gridDim.x + blockIdx.x, (int64_t)gridDim.x * gridDim.y, LNT);
}

// ------------------------------------------------------------------ tn
// One or two jobs per launch (the first j0.blocks workgroups run job 0).
constexpr int TQ_BYTES = 72 * 1024;  // factor slice in LDS (later reused for the combine); two per CU

template <int NJT>
__global__ void __launch_bounds__(TNT) k_lora_tn(TnArgs j0, TnArgs j1) {
  __shared__ __attribute__((aligned(16))) uint16_t sQ[TQ_BYTES / 2];
  const bool second = (int)blockIdx.x >= j0.blocks;
  tn_block<NJT, TQ_BYTES, TQ_BYTES, false>(second ? j1 : j0, (int)blockIdx.x - (second ? j0.blocks : 0), sQ,
                                           reinterpret_cast<float*>(sQ), false);
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace

// nt: 128-token tiles x column slices (multiples of 32) so that the grid is
// up to ~256 workgroups (one per CU, 8 wavefronts each), in at most 8 slices
// (more for very few tokens, below):
// each slice costs the finishing wavefronts a load, and short slices stream
// too little to hide their staging (3072 -> 3072 at M = 1024: t 17.8 -> 11.4
// us and u 16.7 -> 11.1 us going from 32 slices to 8; 16 gave 12.6 and 12.3);
// a slice wider than the LDS factor slice holds (nt_cap) is staged and
// streamed in sub-slices.
LoraPlan lora_plan_nt(int64_t M, int64_t C, int rp) {
  LoraPlan p{};
  // 64-token workgroups when 128-token ones cannot give 256 workgroups with
  // at most 8 slices (fewer than 4096 tokens): more CUs stream (3072 -> 3072
  // at M = 1024: t 11.4 -> 10.5 us, u 11.1 -> 9.7 us); at 4096 tokens the
  // 128-token workgroups share each staged factor slice among more
  // wavefronts (u 24.8 -> 23.8 us)
  p.lw = cdiv(M > 0 ? M : 1, 128) * 8 < 256 ? 4 : 8;
  const int64_t tiles = cdiv(M > 0 ? M : 1, 16 * p.lw);
  // slices: at most 8, but 32 for one or two token tiles and 16 for up to
  // four, where 8 slices leave most CUs idle (u = s dy B^T, us, 8 / 16 /
  // 32 / 64 slices: M = 1, 18432 columns 28.2 / 18.2 / 13.5 / 15.3; M = 64,
  // 9216 columns 26.2 / 17.0 / 13.0 / 15.0; M = 256, 9728 columns t + u
  // 25.5 / 24.0 / 28.5 / 38.7)
  const int64_t cap = tiles <= 2 ? 32 : (tiles <= 4 ? 16 : 8);
  const int64_t want = std::min<int64_t>(cap, cdiv(256, tiles));
  int64_t per = 32 * cdiv(cdiv(C, want), 32);
  if (per < 32) per = 32;
  p.per = per;
  p.splits = (int)cdiv(C, per);
  p.tiles = tiles;
  return p;
}

// tn: token slices (multiples of 128) so that the column tiles of every job
// in the launch (this job's C and other_c, 0 when it runs alone) times the
// slices fill at most the 512 workgroup slots (two resident per CU): a
// partial second round would cost a whole slice's time. Within the LDS
// factor slice.
LoraPlan lora_plan_tn(int64_t M, int64_t C, int rp, int64_t other_c) {
  LoraPlan p{};
  const int64_t tiles = cdiv(C, 128);
  const int64_t want = std::max<int64_t>(1, 512 / (tiles + cdiv(other_c, 128)));
  int64_t per = 128 * cdiv(cdiv(M > 0 ? M : 1, want), 128);
  const int64_t cap = ((TQ_BYTES / 2) / rp - 8) / 128 * 128;
  if (per > cap) per = cap;
  if (per < 128) per = 128;
  p.per = per;
  p.splits = (int)cdiv(M > 0 ? M : 1, per);
  p.tiles = tiles;
  return p;
}

LoraPlan mid_tn_plan(int64_t M, int64_t C, int rp) {
  LoraPlan p{};
  const int64_t cap = rp > 0 ? ((MID_TN_LDS / 2) / rp - 8) / 128 * 128 : 0;
  if (cap < 128) return p;  // no slice fits (ranks past 16 do not run there)
  const int64_t m = M > 0 ? M : 1;
  const int64_t S = cdiv(m, cap);
  p.per = 128 * cdiv(cdiv(m, S), 128);
  p.splits = (int)cdiv(m, p.per);
  p.tiles = cdiv(C, 128);
  return p;
}

hipError_t launch_lora_nt(hipStream_t st, const uint16_t* p, const uint16_t* q, bool qrow, int64_t ldq,
                          int R, int64_t M, int64_t C, int rp, const LoraPlan& plan, float* partial,
                          const NtFinish& fin) {
  if (M == 0) return hipSuccess;
  if (!fin.cnt || plan.tiles * plan.lw > SK_MAX_NB || (plan.lw != 4 && plan.lw != 8)) return hipErrorInvalidValue;
  NtArgs a{p, q, M, C, ldq, R, plan.per, partial, fin};
  const dim3 grid((unsigned)plan.tiles, (unsigned)plan.splits);
#define LRQ_NT(NJT, QR)                                                                   \
  if (plan.lw == 8)                                                                       \
    hipLaunchKernelGGL((k_lora_nt<NJT, QR, 8>), grid, dim3(512), 0, st, a);               \
  else                                                                                    \
    hipLaunchKernelGGL((k_lora_nt<NJT, QR, 4>), grid, dim3(256), 0, st, a)
  switch ((qrow ? 4 : 0) + rp / 16 - 1) {
    case 0: LRQ_NT(1, false); break;
    case 1: LRQ_NT(2, false); break;
    case 2: LRQ_NT(3, false); break;
    case 3: LRQ_NT(4, false); break;
    case 4: LRQ_NT(1, true); break;
    case 5: LRQ_NT(2, true); break;
    case 6: LRQ_NT(3, true); break;
    case 7: LRQ_NT(4, true); break;
    default: return hipErrorInvalidValue;
  }
#undef LRQ_NT
  return hipGetLastError();
}

TnArgs tn_args(const TnSpec& j, uint32_t* cnt) {
  const int64_t blocks = j.C > 0 ? j.plan.tiles * j.plan.splits : 0;
  return TnArgs{j.p,   j.q,  j.M,  j.C,           j.ldq, j.R, j.plan.per, j.partial, (int)j.plan.tiles, (int)blocks,
                j.out, j.sc, j.sj, j.plan.splits, cnt};
}

hipError_t launch_lora_tn(hipStream_t st, const TnSpec* jobs, int njobs, int rp, uint32_t* cnt) {
  TnArgs t[2] = {};
  int64_t total = 0, ntiles = 0;
  for (int i = 0; i < njobs && i < 2; ++i) {
    const TnSpec& j = jobs[i];
    const int64_t blocks = j.C > 0 ? j.plan.tiles * j.plan.splits : 0;
    // each job's column tiles count on their own counters
    t[i] = tn_args(j, cnt + ntiles * TW);
    total += blocks;
    ntiles += j.plan.tiles;
  }
  if (!cnt || ntiles * TW > SK_MAX_NB) return hipErrorInvalidValue;
  if (total == 0) return hipSuccess;
  const dim3 grid((unsigned)total);
  switch (rp / 16) {
    case 1: hipLaunchKernelGGL(k_lora_tn<1>, grid, dim3(TNT), 0, st, t[0], t[1]); break;
    case 2: hipLaunchKernelGGL(k_lora_tn<2>, grid, dim3(TNT), 0, st, t[0], t[1]); break;
    case 3: hipLaunchKernelGGL(k_lora_tn<3>, grid, dim3(TNT), 0, st, t[0], t[1]); break;
    case 4: hipLaunchKernelGGL(k_lora_tn<4>, grid, dim3(TNT), 0, st, t[0], t[1]); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
