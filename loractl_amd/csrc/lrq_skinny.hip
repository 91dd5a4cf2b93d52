// Forward of the quantized LoRA linear for a few tokens (m <= 16):
//
//   y[m, n] = x[m, k] . bf16(dq(w))[n, k]^T (+bias) + t[m, :] . B[:, n],
//   t = bf16(s . x . A)
//
// (src/quant.rs:175-176 and src/lora.rs:199-203, as the large-m kernel.)
//
// With so few tokens the forward is a stream of the packed weight from HBM;
// the matrix-core and dequantization work per byte is small, and what
// matters is keeping enough loads in flight and finishing the math on each
// block as its bytes arrive. Two launches:
//
// k_sk_part: workgroups (block row nb, reduction split s) own 64 weight rows
//   x KS 64-wide reduction blocks; each of the four wavefronts takes a run of
//   those blocks for all 64 rows. A wavefront issues every load of its run
//   at once, in block order (the x fragments, then per 16-row tile 8 packed
//   bytes int4 or 16 bytes fp8 per lane; the 16 lanes of a k quarter read 16
//   consecutive rows, so one load covers 512 or 1024 contiguous bytes), and
//   dequantizes and multiplies block by block as the loads land, with
//   v_mfma_f32_16x16x32_bf16 (tokens as the A-role rows, weight rows as the
//   B-role columns; lane quarter q takes k = 16q + 8j .. +8 in sub-step j;
//   each x fragment serves the four row tiles). No wavefront waits for
//   another until the four runs are summed in LDS; the f32 partial of each
//   split goes to a workspace. A few more workgroups (scheduled first)
//   compute the f32 partials of x . A over slices of k.
// k_sk_epi: per output column, sums the split partials in a fixed order,
//   applies the fp8 per-channel scale, adds t . B (t rounded to bf16 as in
//   the large-m path) and the bias, and writes y (and t).
//
// int4 with groups of 64 or more multiplies the integer q exactly and
// applies the group scale in f32 per 64-wide block (see MQ below), which is
// the oracle's f32 dequantization; groups of 32 and fp8 use the large-m
// kernel's operand (bf16(q s), exact e4m3). No atomics: results are bitwise
// reproducible.

#include "lrq_common.h"
#include "lrq_kernels.h"

namespace {

constexpr int SK_NT = 256;     // threads per workgroup (4 wavefronts)
constexpr int SK_MAXKS = 16;   // reduction blocks per split, at most
constexpr int SK_TSTEPS = 2;   // 32-wide k steps of a t (u) slice per wavefront (slices <= 256)
constexpr int SK_WB = SK_MAXKS / 4;  // blocks per wavefront run, at most

struct SkArgs {
  GemmArgs g;
  const uint16_t* A;  // [k, r] (LoRA down factor), or null
  SkinnyPlan p;
  float* part;        // [S][m][n]
  float* tpart;       // [TS][16][rp]
};

// MQ (int4 forward, groups of 64 or more, so one group per 64-wide block):
// the matrix-core operand is the stored nibble u = q + 8 as the exact bf16
// value 128 + u (bits 0x4300 | u, two bit operations per pair), each block
// is multiplied into fresh accumulators, and the block's partial is scaled
// in f32: s * (sum x (128 + u) - 136 sum x) = s * sum x q. The block sums of
// x come from one more matrix-core step against ones.
template <int FMT, bool BWD, bool MQ>
__global__ void __launch_bounds__(SK_NT) k_sk_part(SkArgs sa) {
  constexpr bool I4 = FMT == LRQ_FMT_INT4;
  // cross-wavefront reduction buffer: [4 wavefronts][64 columns][16 tokens]
  __shared__ __attribute__((aligned(16))) float xs[4 * 64 * 16];
  const GemmArgs& a = sa.g;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, kq = lane >> 4;
  const int64_t M = a.m, K = a.l, E = a.e;  // K: the depth (d_in forward, d_out backward)
  const int64_t KB = (K + 63) / 64;
  const int TS = sa.p.TS;

  if ((int)blockIdx.x < TS) {
    // ---------------- t partial: tpart[ts][m][j] = sum over the slice of x[m, k] A[k, j]
    // (backward: of dy[m, n] B[j, n], for u)
    const int ts = blockIdx.x, rp = a.rp, r = a.r;
    const int64_t kt0 = (int64_t)ts * sa.p.KT, kt1 = kt0 + sa.p.KT < K ? kt0 + sa.p.KT : K;
    const int nsteps = (int)((kt1 - kt0 + 31) / 32);  // <= 4 * SK_TSTEPS
    const rsrc_t rx = make_rsrc(a.act, clamp_bytes(M * K * 2));
    const rsrc_t ra = make_rsrc(sa.A, clamp_bytes(K * r * 2));
    f32x4 acc[4];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) acc[jt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    // one k step per phase: each issues all its loads (out-of-range ones
    // read zero) before its matrix-core steps, in few enough registers that
    // the streaming workgroups keep their occupancy
    u32x4 xf[SK_TSTEPS];
    uint32_t bw[SK_TSTEPS][4][4];
#pragma unroll
    for (int i = 0; i < SK_TSTEPS; ++i) {
      {
        const int st = wv + (SK_NT / 64) * i;
        const int64_t k = kt0 + (int64_t)st * 32 + kq * 8;
        const bool kok = st < nsteps && k < kt1;  // K % 8 == 0 and slices are multiples of 32
        xf[i] = bload16(rx, opaque_u32(kok ? (uint32_t)(((int64_t)c16 * K + k) * 2) : LRQ_OOB));
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
          const int j = jt * 16 + c16;
          const bool ok = kok && j < r;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if (BWD) {
              // B[j][k + 2q], B[j][k + 2q + 1] (one dword: the depth is a multiple of 8)
              bw[i][jt][q] = bload4(ra, opaque_u32(ok ? (uint32_t)(((int64_t)j * K + k + 2 * q) * 2) : LRQ_OOB));
            } else {
              // A[k + 2q][j], A[k + 2q + 1][j]
              const uint32_t off = (uint32_t)(((k + 2 * q) * r + j) * 2);
              const uint32_t lo = bload2(ra, opaque_u32(ok ? off : LRQ_OOB));
              const uint32_t hi = bload2(ra, opaque_u32(ok ? off + (uint32_t)(2 * r) : LRQ_OOB));
              bw[i][jt][q] = lo | (hi << 16);
            }
          }
        }
      }
      // every column tile runs (tiles past rp multiply zeros): a matrix-core
      // result read in a block other than the one that wrote it has come
      // back stale here, so the steps stay branch-free
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
        acc[jt] = mfma16(as_bf16x8(xf[i]), as_bf16x8((u32x4){bw[i][jt][0], bw[i][jt][1], bw[i][jt][2], bw[i][jt][3]}),
                         acc[jt]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // reduce the four wavefronts; C element v of lane l: token 4*(l/16) + v, column l%16
    float* tred = xs;  // [4][16][64]
#pragma unroll
    for (int jt = 0; jt < 4; ++jt)
#pragma unroll
      for (int v = 0; v < 4; ++v) tred[(wv * 16 + 4 * kq + v) * 64 + jt * 16 + c16] = acc[jt][v];
    __syncthreads();
    for (int i = tid; i < 16 * rp; i += SK_NT) {
      const int m = i / rp, j = i % rp;
      float v = 0.0f;
#pragma unroll
      for (int w2 = 0; w2 < SK_NT / 64; ++w2) v += tred[(w2 * 16 + m) * 64 + j];
      sa.tpart[((int64_t)ts * 16 + m) * rp + j] = v;
    }
    return;
  }

  // ---------------- base partial of split s over block row nb: the four
  // wavefronts take consecutive runs of the split's blocks, each for all 64
  // rows (so no two wavefronts read the same x), and meet in LDS at the end
  const int S = sa.p.S, KS = sa.p.KS;
  const int bid = (int)blockIdx.x - TS;
  const int64_t nb = bid / S;
  const int s = bid % S;
  const int kbs = s * KS;
  const int nks = (int)(KB - kbs < KS ? KB - kbs : KS);  // blocks of this split (>= 1)
  const int kb0 = kbs + (nks * wv) / 4, nkb = kbs + (nks * (wv + 1)) / 4 - kb0;  // this wavefront's run

  constexpr uint32_t blkb = I4 ? 2048u : 4096u;
  constexpr uint32_t rowb = I4 ? 32u : 64u;
  const rsrc_t rw = make_rsrc(a.wdata + nb * KB * blkb, clamp_bytes(KB * (int64_t)blkb));
  const int64_t Gp = I4 ? ((KB * 64) >> a.gshift) : 0;
  // forward: int4 group scales of the block row ([NB][Gp][64]); backward: the
  // per-depth scales (int4 the transposed table ST [KGt][64 KB], fp8 the
  // channel scales [depth] or one scalar)
  const int64_t NP = KB * 64;
  const int64_t KGt = (BWD && I4) ? (((E + 63) / 64 * 64 + (1 << a.gshift) - 1) >> a.gshift) : 0;
  const rsrc_t rs = BWD ? (I4 ? make_rsrc(a.wscale, clamp_bytes(KGt * NP * 4))
                              : make_rsrc(a.wscale, a.per_channel ? clamp_bytes(K * 4) : 0u))
                        : (I4 ? make_rsrc(a.wscale + nb * Gp * 64, clamp_bytes(Gp * 64 * 4)) : make_rsrc(a.wscale, 4u));
  const float s0add = (BWD && !I4 && !a.per_channel) ? a.wscale[0] : 0.0f;
  const rsrc_t rx = make_rsrc(a.act, clamp_bytes(M * K * 2));
  const uint32_t woff = (uint32_t)c16 * rowb + (uint32_t)kq * (I4 ? 8u : 16u);
  const uint32_t xoff = (uint32_t)(((int64_t)c16 * K + kq * 16) * 2);

  // all loads in block order: x fragments, then the four row tiles' packed
  // words (and int4 scales); block b is consumed once its loads are in
  u32x4 xf[SK_WB][2];
  u32x2 w4[I4 ? SK_WB : 1][4];
  u32x2 w8[I4 ? 1 : SK_WB][4][2];
  float sc[(I4 || BWD) ? SK_WB : 1][4];  // forward int4: per row tile; backward: lane c16's depth (fp8: [b][0])
#pragma unroll
  for (int b = 0; b < SK_WB; ++b) {
    const bool ok = b < nkb;
    const uint32_t kb = (uint32_t)(kb0 + b);
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int64_t k = (int64_t)kb * 64 + kq * 16 + jj * 8;
      const bool xok = ok && k < K;  // K % 8 == 0
      xf[b][jj] = bload16(rx, opaque_u32(xok ? xoff + (uint32_t)(((int64_t)kb * 64 + jj * 8) * 2) : LRQ_OOB));
    }
    // backward: lane (kq, c16) holds the scale of depth 64 kb + 16 kq + c16,
    // which the 16 lanes of its DPP row (one kq) broadcast among themselves
    const uint32_t dpos = kb * 64u + (uint32_t)(kq * 16 + c16);
    if (BWD && !I4) sc[b][0] = bloadf(rs, opaque_u32(ok ? dpos * 4u : LRQ_OOB)) + s0add;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const uint32_t wo = kb * blkb + (uint32_t)(rt * 16) * rowb + woff;
      if constexpr (I4) {
        w4[b][rt] = bload8(rw, opaque_u32(ok ? wo : LRQ_OOB));
        if (BWD) {
          // group of output rows 64 nb + 16 rt .. +16 (groups are >= 32 and aligned)
          const uint32_t kg = (uint32_t)((nb * 64 + rt * 16) >> a.gshift);
          sc[b][rt] = bloadf(rs, opaque_u32(ok ? (uint32_t)((kg * NP + dpos) * 4) : LRQ_OOB));
        } else {
          const uint32_t j = (kb * 64u + (uint32_t)kq * 16u) >> a.gshift;
          sc[b][rt] = bloadf(rs, opaque_u32(ok ? (j * 64u + (uint32_t)(rt * 16 + c16)) * 4u : LRQ_OOB));
        }
      } else {
        const u32x4 v = bload16(rw, opaque_u32(ok ? wo : LRQ_OOB));
        w8[b][rt][0] = (u32x2){v[0], v[1]};
        w8[b][rt][1] = (u32x2){v[2], v[3]};
      }
    }
  }

  // keep every load ahead of the math (the scheduler would otherwise trade
  // loads in flight for registers)
  __builtin_amdgcn_sched_barrier(0);
  f32x4 acc[4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt) acc[rt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int b = 0; b < SK_WB; ++b) {
    // blocks past this wavefront's run hold zeros: the steps stay
    // unconditional (a matrix-core result read in another block than the
    // one that wrote it has come back stale)
    if constexpr (MQ) {
      const u32x4 ones = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
      f32x4 xsum = {0.0f, 0.0f, 0.0f, 0.0f};
      u32x4 xp[2];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const u32x4 v = xf[b][jj];
        xsum = mfma16(as_bf16x8(v), as_bf16x8(ones), xsum);
        // k order 0 4 1 5 2 6 3 7, as the weight pairs below
        xp[jj] = (u32x4){__builtin_amdgcn_perm(v[2], v[0], 0x05040100u), __builtin_amdgcn_perm(v[2], v[0], 0x07060302u),
                         __builtin_amdgcn_perm(v[3], v[1], 0x05040100u), __builtin_amdgcn_perm(v[3], v[1], 0x07060302u)};
      }
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) {
        f32x4 ab = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const uint32_t d = w4[b][rt][jj];
          // (u_e, u_e+4) as bf16 (128 + u) pairs
          const u32x4 wb = {(d & 0x000f000fu) | 0x43004300u, ((d >> 4) & 0x000f000fu) | 0x43004300u,
                            ((d >> 8) & 0x000f000fu) | 0x43004300u, ((d >> 12) & 0x000f000fu) | 0x43004300u};
          ab = mfma16(as_bf16x8(xp[jj]), as_bf16x8(wb), ab);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[rt][v] = __builtin_fmaf(sc[b][rt], __builtin_fmaf(-136.0f, xsum[v], ab[v]), acc[rt][v]);
      }
      continue;
    }
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        u32x4 wb;
        if constexpr (BWD) {
          // transposed section: value e is q (a sign-extended nibble, or the
          // e4m3 value) times the scale of its depth 16 kq + 8 jj + e, then bf16
          float f[8];
          if (I4) {
            const uint32_t d = w4[b][rt][jj];
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = (float)((int)(d << (28 - 4 * e)) >> 28);
          } else {
            fp8x4_to_f32(w8[b][rt][jj][0], f);
            fp8x4_to_f32(w8[b][rt][jj][1], f + 4);
          }
          const float S = sc[b][I4 ? rt : 0];
#pragma unroll
          for (int e = 0; e < 8; ++e) f[e] = row_bcast_n(S, 8 * jj + e) * f[e];
#pragma unroll
          for (int q = 0; q < 4; ++q) wb[q] = pack_bf16x2(f[2 * q], f[2 * q + 1]);
        } else if constexpr (I4) {
          wb = dequant8_int4_bf16(w4[b][rt][jj], sc[b][rt], a.nib);
        } else {
          const u32x2 p0 = fp8x4_to_bf16(w8[b][rt][jj][0]), p1 = fp8x4_to_bf16(w8[b][rt][jj][1]);
          wb = (u32x4){p0[0], p0[1], p1[0], p1[1]};
        }
        acc[rt] = mfma16(as_bf16x8(xf[b][jj]), as_bf16x8(wb), acc[rt]);
      }
    }
  }
  // reduce the four runs: C element v of lane l is token 4*(l/16) + v,
  // weight row 16 rt + l%16
  float* red = xs;  // [4 runs][4 rt][16 tokens][16 rows]
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[((wv * 4 + rt) * 16 + 4 * kq + v) * 16 + c16] = acc[rt][v];
  __syncthreads();
  // thread: token m = tid / 16 (tid < 256 covers 16 tokens), rows (tid % 16) + 16 rt
  const int m = tid >> 4, c = tid & 15;
  if (m < M) {
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) {
      const int64_t n = nb * 64 + rt * 16 + c;
      float v = 0.0f;
#pragma unroll
      for (int w2 = 0; w2 < 4; ++w2) v += red[((w2 * 4 + rt) * 16 + m) * 16 + c];
      if (n < E) sa.part[((int64_t)s * M + m) * E + n] = v;
    }
  }
}

// y[m, n] = bf16(sc[n] * sum_s part[s][m][n] + sum_j t[m, j] B[j, n] + bias[n]).
// Every workgroup first reduces t = bf16(scale * sum_ts tpart[ts]) into LDS.
// Backward: dx[m, k] = bf16(sum_s part[s][m][k] + sum_j u[m, j] A[k, j]) with
// u = bf16(scaling * sum_ts tpart[ts]) (t_out gets u [m, rp]) and A = a.lw
// [k, r] (no scale: the transposed weight's scales are applied per value,
// no bias).
// A thread owns two adjacent columns and four tokens. Every load is a
// buffer load whose out-of-range offsets read zero, so none sits behind a
// branch and all of a thread's loads issue together.
template <int FMT, bool BWD>
__global__ void __launch_bounds__(SK_NT) k_sk_epi(SkArgs sa, float scaling, uint16_t* t_out) {
  const GemmArgs& a = sa.g;
  const int tid = threadIdx.x;
  const int64_t M = a.m, E = a.e;
  const int rp = a.rp, r = a.r, S = sa.p.S, TS = sa.p.TS;
  __shared__ __attribute__((aligned(16))) float tt[16][64];
  const int64_t n = (int64_t)blockIdx.x * 128 + 2 * (tid & 63);  // E % 8 == 0: n < E implies n + 1 < E
  const int mg = tid >> 6;                                        // tokens 4 mg .. 4 mg + 3
  const bool live = n < E && 4 * mg < M;
  // this thread's loads go out first, so that they share one memory round
  // trip with the reduction of t below (dead threads' offsets read zero)
  const rsrc_t rb = make_rsrc(a.lw, clamp_bytes((int64_t)r * E * 2));
  const rsrc_t rpt = make_rsrc(sa.part, clamp_bytes((int64_t)S * M * E * 4));
  const rsrc_t rbias = make_rsrc(a.bias, a.bias ? clamp_bytes(E * 4) : 0u);
  // bp[j]: the weight-side factor at columns n (low half) and n + 1 (high)
  uint32_t bp[64];
  if (BWD) {
    // A[n][j] and A[n + 1][j] from A [k, r]: rows of 16-byte runs when r is
    // a multiple of 8 and A is 16-byte aligned, else value by value
    if ((r & 7) == 0 && (reinterpret_cast<uintptr_t>(a.lw) & 15) == 0) {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const bool ok = live && q * 8 < r;
        const u32x4 v0 = bload16(rb, opaque_u32(ok ? (uint32_t)((n * r + q * 8) * 2) : LRQ_OOB));
        const u32x4 v1 = bload16(rb, opaque_u32(ok ? (uint32_t)(((n + 1) * r + q * 8) * 2) : LRQ_OOB));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          bp[q * 8 + 2 * e] = __builtin_amdgcn_perm(v1[e], v0[e], 0x05040100u);
          bp[q * 8 + 2 * e + 1] = __builtin_amdgcn_perm(v1[e], v0[e], 0x07060302u);
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < 64; ++j) {
        const bool ok = live && j < r;
        const uint32_t lo = bload2(rb, opaque_u32(ok ? (uint32_t)((n * r + j) * 2) : LRQ_OOB));
        const uint32_t hi = bload2(rb, opaque_u32(ok ? (uint32_t)(((n + 1) * r + j) * 2) : LRQ_OOB));
        bp[j] = lo | (hi << 16);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 64; ++j)
      bp[j] = bload4(rb, opaque_u32(live && j < r ? (uint32_t)(((int64_t)j * E + n) * 2) : LRQ_OOB));
  }
  u32x2 pv[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * mg + i;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      pv[i][s] = bload8(rpt, opaque_u32((live && s < S && m < M) ? (uint32_t)((((int64_t)s * M + m) * E + n) * 4)
                                                                   : LRQ_OOB));
  }
  float sc0 = 1.0f, sc1 = 1.0f;
  if (!BWD && FMT == LRQ_FMT_FP8) {
    const rsrc_t rsc = make_rsrc(a.wscale, clamp_bytes((a.per_channel ? E : 1) * 4));
    const uint32_t c0 = a.per_channel ? (uint32_t)(n * 4) : 0u;
    sc0 = bloadf(rsc, opaque_u32(live ? c0 : LRQ_OOB));
    sc1 = bloadf(rsc, opaque_u32(live ? c0 + (a.per_channel ? 4u : 0u) : LRQ_OOB));
  }
  const u32x2 bias = bload8(rbias, opaque_u32(live ? (uint32_t)(n * 4) : LRQ_OOB));

  const rsrc_t rtp = make_rsrc(sa.tpart, clamp_bytes((int64_t)TS * 16 * rp * 4));
  // two outputs per thread and pass (entries i and i + SK_NT of [16][rp]),
  // slices in order, 16 loads of each issued together per batch
  for (int i0 = tid; i0 < 16 * rp; i0 += 2 * SK_NT) {
    float v[2] = {0.0f, 0.0f};
    for (int q0 = 0; q0 < TS; q0 += 16) {
      float part[2][16];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          const int i = i0 + h * SK_NT;
          part[h][q] = bloadf(rtp, opaque_u32((q0 + q < TS && i < 16 * rp) ? (uint32_t)(((q0 + q) * 16 * rp + i) * 4)
                                                                           : LRQ_OOB));
        }
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int q = 0; q < 16; ++q) v[h] += part[h][q];
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = i0 + h * SK_NT;
      if (i >= 16 * rp) break;
      const int m = i / rp, j = i % rp;
      const uint32_t hb = pack_bf16x2(scaling * v[h], 0.0f) & 0xffffu;  // t (u) as the caller sees it
      tt[m][j] = __uint_as_float(hb << 16);
      // t [m, r]; u [m, rp] (columns >= r zero), dA's factor
      if (blockIdx.x == 0 && t_out && m < M && (BWD || j < r)) t_out[(int64_t)m * (BWD ? rp : r) + j] = (uint16_t)hb;
    }
  }
  __syncthreads();
  if (!live) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = 4 * mg + i;
    if (m >= M) break;
    float base0 = 0.0f, base1 = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      base0 += __uint_as_float(pv[i][s][0]);
      base1 += __uint_as_float(pv[i][s][1]);
    }
    // splits past the first eight, in order, eight loads issued together
    for (int s0 = 8; s0 < S; s0 += 8) {
      u32x2 pw[8];
#pragma unroll
      for (int s = 0; s < 8; ++s)
        pw[s] = bload8(rpt, opaque_u32(s0 + s < S ? (uint32_t)((((int64_t)(s0 + s) * M + m) * E + n) * 4) : LRQ_OOB));
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        base0 += __uint_as_float(pw[s][0]);
        base1 += __uint_as_float(pw[s][1]);
      }
    }
    float l0 = 0.0f, l1 = 0.0f;
#pragma unroll
    for (int jc = 0; jc < 4; ++jc) {
      if (jc * 16 < rp) {  // rank chunks of 16 (rp is a multiple of 16)
        float4 tv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) tv[q] = *reinterpret_cast<const float4*>(&tt[m][jc * 16 + 4 * q]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float t4[4] = {tv[q].x, tv[q].y, tv[q].z, tv[q].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t bv = bp[jc * 16 + 4 * q + e];
            l0 = __builtin_fmaf(t4[e], __uint_as_float(bv << 16), l0);
            l1 = __builtin_fmaf(t4[e], __uint_as_float(bv & 0xffff0000u), l1);
          }
        }
      }
    }
    const uint32_t o = pack_bf16x2(base0 * sc0 + l0 + __uint_as_float(bias[0]),
                                   base1 * sc1 + l1 + __uint_as_float(bias[1]));
    *reinterpret_cast<uint32_t*>(a.out + (int64_t)m * E + n) = o;
  }
}

}  // namespace

SkinnyPlan skinny_plan(int64_t n, int64_t k, int rp, int num_cus) {
  SkinnyPlan p{};
  const int64_t KB = (k + 63) / 64, NB = (n + 63) / 64;
  // enough workgroups for about 9/4 per CU (fewer, longer splits measured
  // faster than three per CU: fewer partials), at most 16 blocks per split,
  // and split partials (S * m * n f32) no larger than a quarter of the weight
  int64_t S = (9 * (int64_t)num_cus + 4 * NB - 1) / (4 * NB);
  const int64_t s_min = (KB + SK_MAXKS - 1) / SK_MAXKS;
  int64_t s_max = k / 512;
  if (s_max < s_min) s_max = s_min;
  if (S > s_max) S = s_max;
  if (S < s_min) S = s_min;
  if (S > KB) S = KB;
  if (S < 1) S = 1;
  p.KS = (int)((KB + S - 1) / S);
  p.S = (int)((KB + p.KS - 1) / p.KS);  // every split holds at least one block
  // t: slices of at most 256 k (multiples of 32)
  if (rp > 0) {
    const int64_t kmax = 32 * 4 * SK_TSTEPS;
    int64_t TS = (k + kmax - 1) / kmax;
    if (TS < 1) TS = 1;
    p.KT = ((k + TS - 1) / TS + 31) / 32 * 32;
    p.TS = (int)((k + p.KT - 1) / p.KT);
  }
  return p;
}

size_t skinny_ws_bytes(const SkinnyPlan& p, int64_t m, int64_t n, int rp) {
  const size_t part = (size_t)p.S * m * n * 4, tp = (size_t)p.TS * 16 * rp * 4;
  return (part + 255) / 256 * 256 + tp + 256;
}

hipError_t launch_skinny_part(hipStream_t st, int fmt, bool bwd, const GemmArgs& a, const uint16_t* A,
                              const SkinnyPlan& p, float* part, float* tpart) {
  if (a.m <= 0 || a.m > 16 || p.S < 1 || p.KS < 1 || p.KS > SK_MAXKS) return hipErrorInvalidValue;
  SkArgs sa{a, A, p, part, tpart};
  if (a.rp == 0 || !A) sa.p.TS = 0;
  const int64_t NB = (a.e + 63) / 64;
  const unsigned grid = (unsigned)(NB * p.S + sa.p.TS);
  if (fmt == LRQ_FMT_INT4) {
    if (bwd)
      hipLaunchKernelGGL((k_sk_part<LRQ_FMT_INT4, true, false>), dim3(grid), dim3(SK_NT), 0, st, sa);
    else if (a.gshift >= 6)
      hipLaunchKernelGGL((k_sk_part<LRQ_FMT_INT4, false, true>), dim3(grid), dim3(SK_NT), 0, st, sa);
    else
      hipLaunchKernelGGL((k_sk_part<LRQ_FMT_INT4, false, false>), dim3(grid), dim3(SK_NT), 0, st, sa);
  } else {
    if (bwd)
      hipLaunchKernelGGL((k_sk_part<LRQ_FMT_FP8, true, false>), dim3(grid), dim3(SK_NT), 0, st, sa);
    else
      hipLaunchKernelGGL((k_sk_part<LRQ_FMT_FP8, false, false>), dim3(grid), dim3(SK_NT), 0, st, sa);
  }
  return hipGetLastError();
}

hipError_t launch_skinny_epi(hipStream_t st, int fmt, bool bwd, const GemmArgs& a, const SkinnyPlan& p,
                             const float* part, const float* tpart, float scaling, uint16_t* t_out) {
  if (a.m <= 0 || a.m > 16) return hipErrorInvalidValue;
  SkArgs sa{a, nullptr, p, const_cast<float*>(part), const_cast<float*>(tpart)};
  if (a.rp == 0 || !tpart) sa.p.TS = 0;
  const unsigned grid = (unsigned)((a.e + 127) / 128);
  if (fmt == LRQ_FMT_INT4) {
    if (bwd)
      hipLaunchKernelGGL((k_sk_epi<LRQ_FMT_INT4, true>), dim3(grid), dim3(SK_NT), 0, st, sa, scaling, t_out);
    else
      hipLaunchKernelGGL((k_sk_epi<LRQ_FMT_INT4, false>), dim3(grid), dim3(SK_NT), 0, st, sa, scaling, t_out);
  } else {
    if (bwd)
      hipLaunchKernelGGL((k_sk_epi<LRQ_FMT_FP8, true>), dim3(grid), dim3(SK_NT), 0, st, sa, scaling, t_out);
    else
      hipLaunchKernelGGL((k_sk_epi<LRQ_FMT_FP8, false>), dim3(grid), dim3(SK_NT), 0, st, sa, scaling, t_out);
  }
  return hipGetLastError();
}
