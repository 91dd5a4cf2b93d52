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
// block as its bytes arrive. One launch, k_sk:
//
// - Split workgroups (block row nb, reduction split s) own 64 weight rows x
//   KS 64-wide reduction blocks; each of the four wavefronts takes a run of
//   those blocks for all 64 rows. A wavefront issues every load of its run
//   at once, in block order (the x fragments, then 16 bytes per lane: fp8
//   one 16-row tile, 1024 contiguous bytes per load; int4 two tiles, two runs
//   of 512 bytes, split between the lanes by v_permlane32_swap), and
//   dequantizes and multiplies block by block as the loads land, with
//   v_mfma_f32_16x16x32_bf16 (tokens as the A-role rows, weight rows as the
//   B-role columns; lane quarter q takes 16 depths of each block, 16q (fp8)
//   or 32 (q % 2) + 16 (q / 2) (int4) .. +16, eight per sub-step; each x
//   fragment serves the four row tiles). The four runs meet in LDS
//   and the split's f32 partial goes to a workspace.
// - A few more workgroups (scheduled first) compute the f32 partials of
//   x . A over slices of k and count themselves done; the last of them sums
//   the slices in order, rounds t to bf16 (as the large-m path does) and
//   publishes it (and t itself), every entry stamped with the launch's
//   epoch in the same 8-byte store.
// - Each split workgroup then arrives at its block row's counter, and the
//   last of the S splits runs the block row's epilogue: the split partials
//   summed in a fixed order, the fp8 per-channel scale, t . B and the bias,
//   y written. The epilogue reads t with its other loads and takes it once
//   every stamp is current, reading it again otherwise (the t workgroups
//   can finish after some splits). That wait always ends: the t workgroups
//   have the lowest ids, so they are dispatched before any split
//   workgroup, and they wait on nothing; a cap on the polls (far above any
//   real wait) ends it even so and flags the failure in the counter area.
// - Cross-workgroup data is written and read at device scope (sc1: written
//   through past the non-coherent per-XCD L2s before the store is
//   acknowledged, and read past them), and each workgroup waits for its
//   stores before it counts itself, so the epilogue sees every partial
//   without a cache write-back or invalidate (a device-scope fence per
//   workgroup costs tens of microseconds here). The counters start at zero and end at zero:
//   the last split of a block row resets its counter, and the last of the
//   epilogues resets the t and epilogue counters and advances the epoch.
//
// int4 with groups of 64 or more multiplies the integer q exactly and
// applies the group scale in f32 per 64-wide block (see MQ below), which is
// the oracle's f32 dequantization; groups of 32, int8 and fp8 use the
// large-m kernel's operand (bf16(q s), exact e4m3). int8 loads like fp8 (16
// bytes of one row tile per lane) and scales like int4. No atomic touches a result and
// every sum has a fixed order: results are bitwise reproducible.

#include "lrq_common.h"
#include "lrq_kernels.h"

namespace {

constexpr int SK_NT = 256;     // threads per workgroup (4 wavefronts)
constexpr int SK_MAXKS = 16;   // reduction blocks per split, at most
constexpr int SK_TMAX = 32;    // t (u) slices, at most, while a slice needs no more than 4 steps per wavefront
constexpr int SK_WB = SK_MAXKS / 4;  // blocks per wavefront run, at most
// floats of k_sk's LDS buffer: the cross-wavefront reduction [4][64][16],
// or a t slice's A^T (rank 32 by 512 depths, rank 64 by 256), or a u
// slice's dy and t for the folded dB
constexpr int SK_LDSF = 8704;

struct SkArgs {
  GemmArgs g;
  const uint16_t* A;  // [k, r] (LoRA down factor), or null
  SkinnyPlan p;
  float* part;        // [S][m][n]
  float* tpart;       // [TS][16][rp] f32, then t itself [16][rp] as (bf16 value as f32, epoch stamp)
  uint32_t* cnt;      // [ceil(n / 64)] arrival counters, zero on entry and exit
  float scaling;
  uint16_t* t_out;    // t [m, r] (backward: u [m, rp]), or null
  uint32_t max_polls; // cap of an epilogue's polls for t (SK_MAX_POLLS)
  uint32_t skew;      // added to the awaited stamp: 0 (a test hook sets it to force the timeout)
  SkGrads gr;         // backward: the LoRA factors' gradients folded into the launch (null: skipped)
};

// device-scope accesses of the cross-workgroup data: stores written through
// and loads read past the per-XCD L2s (sc1), atomics at device scope
// (system scope, sc0 sc1, measured the same)
constexpr int XSCOPE = __HIP_MEMORY_SCOPE_AGENT;
constexpr int XAUX = 16;  // sc1 on a buffer load
LRQ_DEV void store_dev(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, XSCOPE); }
LRQ_DEV u32x4 bload16_dev(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, XAUX); }
LRQ_DEV float bloadf_dev(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, XAUX));
}
LRQ_DEV u32x2 bload8_dev(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, XAUX); }
// the stamp of epoch ep (never 0, the value of unwritten memory)
LRQ_DEV uint32_t stamp(uint32_t ep) { return ep + 1 == 0 ? 1u : ep + 1; }

constexpr uint32_t SK_MAX_POLLS = 1u << 22;  // about 0.2 s of s_sleep 2
// what an epilogue takes for t after its wait ran out: NaN as an f32 and as
// both bf16 halves, so the outputs it writes are NaN, not stale
constexpr uint32_t SK_NAN2 = 0x7fc07fc0u;

LRQ_DEV uint32_t add_dev(uint32_t* c) { return __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, XSCOPE); }
LRQ_DEV void zero_dev(uint32_t* c) { __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, XSCOPE); }


LRQ_DEV void bstore4(rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, 0);
}

// One matrix-core step over the tokens, C[i][j] = sum_m P[i][m] Q[j][m], with
// both operands staged token-minor in LDS as bf16 ([row][16 tokens]): lane
// (c16, kq) takes tokens 8 kq .. + 8 of row c16 (kq < 2; tokens 16 .. 31 are
// zero). C element v of lane (c16, kq): row i = 4 kq + v of the P tile,
// column j = c16 of the Q tile.
LRQ_DEV f32x4 sk_token_step(const uint16_t* p_rows, const uint16_t* q_rows) {
  const int lane = threadIdx.x & 63, c16 = lane & 15, kq = lane >> 4;
  const u32x4 z = {0u, 0u, 0u, 0u};
  const u32x4 pa = kq < 2 ? *reinterpret_cast<const u32x4*>(p_rows + c16 * 16 + 8 * kq) : z;
  const u32x4 qb = kq < 2 ? *reinterpret_cast<const u32x4*>(q_rows + c16 * 16 + 8 * kq) : z;
  return mfma16(as_bf16x8(pa), as_bf16x8(qb), (f32x4){0.0f, 0.0f, 0.0f, 0.0f});
}

// The epilogue of block row nb (output columns 64 nb .. +64), run by the last
// workgroup to arrive there (all 256 threads, uniform control flow):
//   y[m, n] = bf16(sc[n] * sum_s part[s][m][n] + sum_j t[m, j] B[j, n] + bias[n])
// with t as published. Backward: dx[m, k] = bf16(sum_s part[s][m][k] +
// sum_j u[m, j] A[k, j]) with u from the partials of dy . B^T and A = a.lw
// [k, r]; no scale, no bias. `lds` holds 3072 floats.
template <int FMT, bool BWD>
LRQ_DEV void sk_epilogue(const SkArgs& sa, int64_t nb, float* lds) {
  const GemmArgs& a = sa.g;
  const int tid = threadIdx.x;
  const int64_t M = a.m, E = a.e, n0 = nb * 64;
  const int rp = a.rp, r = a.r, S = sa.p.S, TS = sa.p.TS;
  float* tt = lds;                                                  // [16][64] t (bf16 values)
  uint16_t* bs = reinterpret_cast<uint16_t*>(lds + 16 * 64);       // [64 ranks][64 columns] bf16
  // thread: token m = tid / 16, columns n .. n + 3 (E % 8 == 0: n < E implies n + 3 < E)
  const int m = tid >> 4, cq = tid & 15;
  const int64_t n = n0 + 4 * cq;
  const bool live = m < M && n < E;
  // what does not depend on t goes out first: the first four split
  // partials and the weight-side factor of the block row (B[j][n0 + c]
  // forward, A[n0 + c][j] backward), so that these loads overlap the t reads
  const rsrc_t rpt = make_rsrc(sa.part, clamp_bytes((int64_t)S * M * E * 4));
  u32x4 pv[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    pv[s] = bload16_dev(rpt, opaque_u32(live && s < S ? (uint32_t)((((int64_t)s * M + m) * E + n) * 4) : LRQ_OOB));
  const rsrc_t rb = make_rsrc(a.lw, TS > 0 ? clamp_bytes((int64_t)r * E * 2) : 0u);
  uint32_t bv[16];  // rp * 64 entries over 256 threads
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int i = tid + q * SK_NT, j = i / 64, c = i % 64;
    const bool ok = j < r && n0 + c < E;
    const uint32_t off = BWD ? (uint32_t)(((n0 + c) * r + j) * 2) : (uint32_t)(((int64_t)j * E + n0 + c) * 2);
    bv[q] = bload2(rb, opaque_u32(ok ? off : LRQ_OOB));
  }
  // t (u) [16][rp] as published: this thread's entries i = tid + 256 q,
  // stamped with the launch's epoch
  const rsrc_t rtf = make_rsrc(sa.tpart + (int64_t)TS * 16 * rp, TS > 0 ? clamp_bytes((int64_t)16 * rp * 8) : 0u);
  u32x2 tv[4];
  auto load_t = [&]() {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = tid + q * SK_NT;
      tv[q] = bload8_dev(rtf, opaque_u32(i < 16 * rp ? (uint32_t)(i * 8) : LRQ_OOB));
    }
  };
  load_t();
  // backward with dA: the x tile [16 tokens][64 columns n0 ..] of this block
  // row (dA rows n0 .. n0 + 63), loaded with the rest (x is [m, E])
  const bool fold_da = BWD && sa.gr.da != nullptr && TS > 0;
  u32x2 xv = {0u, 0u};
  if (fold_da) {
    const rsrc_t rx = make_rsrc(sa.gr.x, clamp_bytes(M * E * 2));
    xv = bload8(rx, opaque_u32(live ? (uint32_t)((m * E + n) * 2) : LRQ_OOB));
  }
  if (TS > 0) {
    const uint32_t want = stamp(__hip_atomic_load(sa.cnt + SK_EPOCH, __ATOMIC_RELAXED, XSCOPE)) + sa.skew;
    // not all published yet: read all of this thread's entries again
    for (uint32_t polls = 0;; ++polls) {
      bool ok = true;
#pragma unroll
      for (int q = 0; q < 4; ++q) ok = ok && (tid + q * SK_NT >= 16 * rp || tv[q][1] == want);
      if (ok) break;
      if (polls == sa.max_polls) {
        __hip_atomic_store(sa.cnt + SK_FAIL, 1u, __ATOMIC_RELAXED, XSCOPE);
#pragma unroll
        for (int q = 0; q < 4; ++q) tv[q][0] = SK_NAN2;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
      load_t();
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = tid + q * SK_NT;
      if (i < 16 * rp) tt[(i / rp) * 64 + i % rp] = __uint_as_float(tv[q][0]);
    }
#pragma unroll
    for (int q = 0; q < 16; ++q)
      if (tid + q * SK_NT < rp * 64) bs[tid + q * SK_NT] = (uint16_t)bv[q];
    if (fold_da) {
      // x and u token-minor for the dA step: xT [64 columns][16 tokens],
      // uT [64 ranks][16 tokens] (bf16, after tt and bs)
      uint16_t* xT = reinterpret_cast<uint16_t*>(lds + 3 * 1024);
      uint16_t* uT = xT + 64 * 16;
#pragma unroll
      for (int e = 0; e < 4; ++e) xT[(4 * cq + e) * 16 + m] = (uint16_t)(xv[e >> 1] >> (16 * (e & 1)));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i = tid + q * SK_NT;
        if (i < 16 * rp) uT[(i % rp) * 16 + i / rp] = (uint16_t)(tv[q][0] >> 16);
      }
    }
  }
  __syncthreads();
  if (live) {
    float base[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int e = 0; e < 4; ++e) base[e] += __uint_as_float(pv[s][e]);
    for (int s0 = 4; s0 < S; s0 += 4) {  // splits past the first four, in order, four loads issued together
#pragma unroll
      for (int s = 0; s < 4; ++s)
        pv[s] = bload16_dev(rpt, opaque_u32(s0 + s < S ? (uint32_t)((((int64_t)(s0 + s) * M + m) * E + n) * 4) : LRQ_OOB));
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int e = 0; e < 4; ++e) base[e] += __uint_as_float(pv[s][e]);
    }
    float l[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < (TS > 0 ? rp : 0); ++j) {  // t and the factor rows exist only with t slices
      const float tv = tt[m * 64 + j];
      const u32x2 bv = *reinterpret_cast<const u32x2*>(bs + j * 64 + 4 * cq);
      l[0] = __builtin_fmaf(tv, __uint_as_float(bv[0] << 16), l[0]);
      l[1] = __builtin_fmaf(tv, __uint_as_float(bv[0] & 0xffff0000u), l[1]);
      l[2] = __builtin_fmaf(tv, __uint_as_float(bv[1] << 16), l[2]);
      l[3] = __builtin_fmaf(tv, __uint_as_float(bv[1] & 0xffff0000u), l[3]);
    }
    float sc[4] = {1.0f, 1.0f, 1.0f, 1.0f}, bias[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (!BWD && FMT == LRQ_FMT_FP8) {
#pragma unroll
      for (int e = 0; e < 4; ++e) sc[e] = a.wscale[a.per_channel ? n + e : 0];
    }
    if (!BWD && a.bias) {
#pragma unroll
      for (int e = 0; e < 4; ++e) bias[e] = a.bias[n + e];
    }
    u32x2 o;
    o[0] = pack_bf16x2(base[0] * sc[0] + l[0] + bias[0], base[1] * sc[1] + l[1] + bias[1]);
    o[1] = pack_bf16x2(base[2] * sc[2] + l[2] + bias[2], base[3] * sc[3] + l[3] + bias[3]);
    *reinterpret_cast<u32x2*>(a.out + (int64_t)m * E + n) = o;
  }
  if (fold_da) {
    // dA[n0 + i][j] = sum_m x[m][n0 + i] u[m][j] (f32): wave w takes rows
    // 16 w .. + 16 of the block row, one matrix-core step per rank tile
    // (ranks past rp read entries never written and are not stored)
    const uint16_t* xT = reinterpret_cast<const uint16_t*>(lds + 3 * 1024);
    const uint16_t* uT = xT + 64 * 16;
    const int w = tid >> 6, kq = (tid & 63) >> 4, c16 = tid & 15;
    const rsrc_t rda = make_rsrc(sa.gr.da, clamp_bytes(E * r * 4));
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      const f32x4 c = sk_token_step(xT + w * 256, uT + jt * 256);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t row = n0 + 16 * w + 4 * kq + v;
        const int j = 16 * jt + c16;
        const bool ok = row < E && j < r && j < rp;
        bstore4(rda, opaque_u32(ok ? (uint32_t)((row * r + j) * 4) : LRQ_OOB), c[v]);
      }
    }
  }
}

// Backward with dB: dB[j][c] = sum_m t[m][j] dy[m][c] (f32 [r, n]) over the
// depth slice [kt0, kt1) of dy that a u slice has just read, straight from
// its fragments: xf[i] holds dy[c16][kt0 + 32 st + 8 kq ..] (st = wave + 4 i).
// Each column has one owner and nothing waits for it. The slice's dy goes
// to LDS token-minor (dyT [KT columns][16 tokens]) and t likewise (tT [64
// ranks][16 tokens]); each wave then takes every fourth 16-column tile, all
// four rank tiles. `lds` holds 128 * TSTEPS * 16 + 1024 bf16; `tq` is this
// thread's four entries of t (bf16 in the low half), i = tid + 256 q as
// (token i / 64, rank i % 64).
template <int TSTEPS>
LRQ_DEV void sk_fold_db(const SkArgs& sa, int64_t kt0, int64_t kt1, const u32x4 (&xf)[TSTEPS],
                        const uint32_t (&tq)[4], uint16_t* lds) {
  static_assert(TSTEPS >= 1 && TSTEPS <= 4, "a u slice of four 32-wide steps per wavefront at most");
  const GemmArgs& a = sa.g;
  const int tid = threadIdx.x, lane = tid & 63, c16 = lane & 15, kq = lane >> 4;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t N = a.l;  // the depth of the backward is the weight's n
  const int r = a.r;
  constexpr int KT = 128 * TSTEPS;
  uint16_t* dyT = lds;            // [KT][16]
  uint16_t* tT = lds + KT * 16;   // [64][16]
  __syncthreads();  // the slice's reads of the LDS buffer are over
#pragma unroll
  for (int i = 0; i < TSTEPS; ++i) {
    const int cl = (wv + 4 * i) * 32 + 8 * kq;
#pragma unroll
    for (int e = 0; e < 8; ++e) dyT[(cl + e) * 16 + c16] = (uint16_t)(xf[i][e >> 1] >> (16 * (e & 1)));
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int i = tid + q * SK_NT;
    tT[(i & 63) * 16 + (i >> 6)] = (uint16_t)tq[q];
  }
  __syncthreads();
  const rsrc_t rdb = make_rsrc(sa.gr.db, clamp_bytes((int64_t)r * N * 4));
#pragma unroll
  for (int h = 0; h < 2 * TSTEPS; ++h) {
    const int ct = wv + 4 * h;  // column tile (16 columns) of the slice
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) {
      const f32x4 c = sk_token_step(tT + jt * 256, dyT + ct * 256);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int j = 16 * jt + 4 * kq + v;
        const int64_t col = kt0 + 16 * ct + c16;
        const bool ok = j < r && col < kt1;
        bstore4(rdb, opaque_u32(ok ? (uint32_t)(((int64_t)j * N + col) * 4) : LRQ_OOB), c[v]);
      }
    }
  }
}


// t partial of slice blockIdx.x (< TS): tpart[ts][m][j] = sum over the slice
// of x[m, k] A[k, j] (backward: of dy[m, n] B[j, n], for u); the last slice
// to finish sums the slices in order and publishes t stamped with the
// launch's epoch. `xs` is the kernel's LDS buffer (4096 floats), `last` a
// shared flag.
template <bool BWD, int TSTEPS, int NT, int LDSF>
LRQ_DEV void sk_t_slices(const SkArgs& sa, float* xs, int& last) {
  const GemmArgs& a = sa.g;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, kq = lane >> 4;
  const int64_t M = a.m, K = a.l;
  const int TS = sa.p.TS;
  // ---------------- t partial: tpart[ts][m][j] = sum over the slice of x[m, k] A[k, j]
  // (backward: of dy[m, n] B[j, n], for u)
  const int ts = blockIdx.x, rp = a.rp, r = a.r;
  const int64_t kt0 = (int64_t)ts * sa.p.KT, kt1 = kt0 + sa.p.KT < K ? kt0 + sa.p.KT : K;
  const int nsteps = (int)((kt1 - kt0 + 31) / 32);
  const rsrc_t rx = make_rsrc(a.act, clamp_bytes(M * K * 2));
  const rsrc_t ra = make_rsrc(sa.A, clamp_bytes(K * r * 2));
  f32x4 acc[4];
#pragma unroll
  for (int jt = 0; jt < 4; ++jt) acc[jt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
  // every load of the slice (at most 4 * TSTEPS steps) is issued at once
  // (out-of-range ones read zero), then the matrix-core steps run as they land
  // The factor operand, lane (c16, kq) of rank tile jt: rank 16 jt + c16 at
  // depths k .. k + 7. Backward: B [r, n] rows as stored, one 16-byte load.
  // Forward: A [k, r] is rank-contiguous, so (when the rank is a multiple of
  // 8 and the slice's A^T fits the LDS buffer) the slice's rows come in as
  // 16-byte runs, go to LDS transposed (aT [rp][KT + 8] bf16, the padding
  // spreads a read's 16 rows over the banks) and are read back as 16-byte
  // runs; otherwise as 2-byte pairs.
  constexpr int KT = 128 * TSTEPS, AST = KT + 8;
  const bool staged = !BWD && (r & 7) == 0 && rp * AST * 2 <= LDSF * 4;
  u32x4 xf[TSTEPS];
  u32x4 bw[TSTEPS][4];
  // (depth, 8-rank run) pairs per thread, at most: the largest rank (a
  // multiple of 16, at most 64) whose A^T fits the buffer
  constexpr int RPMAX = ((LDSF * 4) / (2 * AST)) / 16 * 16 < 64 ? ((LDSF * 4) / (2 * AST)) / 16 * 16 : 64;
  constexpr int AQ = (KT * (RPMAX / 8) + NT - 1) / NT;
  u32x4 av[AQ > 0 ? AQ : 1];
#pragma unroll
  for (int i = 0; i < TSTEPS; ++i) {
    const int st = wv + (NT / 64) * i;
    const int64_t k = kt0 + (int64_t)st * 32 + kq * 8;
    const bool kok = st < nsteps && k < kt1;  // K % 8 == 0 and slices are multiples of 32
    xf[i] = bload16(rx, opaque_u32(kok ? (uint32_t)(((int64_t)c16 * K + k) * 2) : LRQ_OOB));
  }
  if (staged) {
    // pair i = tid + NT q: depth i / (rp / 8) of the slice, ranks 8 (i % (rp / 8)) ..
    const int jb = rp >> 3;
#pragma unroll
    for (int q = 0; q < AQ; ++q) {
      const int i = tid + NT * q, kk = i / jb, j0 = (i % jb) * 8;
      const bool ok = kk < KT && kt0 + kk < kt1 && j0 < r;
      av[q] = bload16(ra, opaque_u32(ok ? (uint32_t)(((kt0 + kk) * r + j0) * 2) : LRQ_OOB));
    }
  } else {
#pragma unroll
    for (int i = 0; i < TSTEPS; ++i) {
      const int st = wv + (NT / 64) * i;
      const int64_t k = kt0 + (int64_t)st * 32 + kq * 8;
      const bool kok = st < nsteps && k < kt1;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const int j = jt * 16 + c16;
        const bool ok = kok && j < r;
        if (BWD) {
          // B[j][k .. k + 7]: 16 bytes (the depth is a multiple of 8)
          bw[i][jt] = bload16(ra, opaque_u32(ok ? (uint32_t)(((int64_t)j * K + k) * 2) : LRQ_OOB));
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            // A[k + 2q][j], A[k + 2q + 1][j]
            const uint32_t off = (uint32_t)(((k + 2 * q) * r + j) * 2);
            const uint32_t lo = bload2(ra, opaque_u32(ok ? off : LRQ_OOB));
            const uint32_t hi = bload2(ra, opaque_u32(ok ? off + (uint32_t)(2 * r) : LRQ_OOB));
            bw[i][jt][q] = lo | (hi << 16);
          }
        }
      }
    }
  }
  // backward with dB: this thread's entries of t (bf16 [m, r]) for the fold,
  // out with the slice's loads
  uint32_t tq[4] = {0u, 0u, 0u, 0u};
  if (BWD && sa.gr.db) {
    const rsrc_t rt = make_rsrc(sa.gr.t, clamp_bytes(M * r * 2));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = tid + q * SK_NT, mm = i >> 6, j = i & 63;
      tq[q] = bload2(rt, opaque_u32(mm < M && j < r ? (uint32_t)((mm * r + j) * 2) : LRQ_OOB));
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  if (staged) {
    // A^T of the slice into LDS (every entry of ranks < rp and depths < KT
    // written, zeros outside A), then each lane's runs out of it
    uint16_t* aT = reinterpret_cast<uint16_t*>(xs);
    const int jb = rp >> 3;
#pragma unroll
    for (int q = 0; q < AQ; ++q) {
      const int i = tid + NT * q, kk = i / jb, j0 = (i % jb) * 8;
      if (kk < KT) {
#pragma unroll
        for (int e = 0; e < 8; ++e) aT[(j0 + e) * AST + kk] = (uint16_t)(av[q][e >> 1] >> (16 * (e & 1)));
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TSTEPS; ++i) {
      const int st = wv + (NT / 64) * i;
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) {
        const int j = jt * 16 + c16;
        // (steps past the slice, which 512-thread workgroups have, read zeros:
        // their x is zero, and zero times a stale NaN would not be)
        bw[i][jt] = j < rp && st * 32 < KT ? *reinterpret_cast<const u32x4*>(aT + j * AST + st * 32 + kq * 8) : zero4();
      }
    }
  }
  // every column tile runs (tiles past rp multiply zeros): a matrix-core
  // result read in a block other than the one that wrote it has come back
  // stale here, so the steps stay branch-free
#pragma unroll
  for (int i = 0; i < TSTEPS; ++i)
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) acc[jt] = mfma16(as_bf16x8(xf[i]), as_bf16x8(bw[i][jt]), acc[jt]);
  // reduce the four wavefronts; C element v of lane l: token 4*(l/16) + v, column l%16
  if (staged) __syncthreads();  // every read of aT is over
  float* tred = xs;  // [NT / 64][16][64]
#pragma unroll
  for (int jt = 0; jt < 4; ++jt)
#pragma unroll
    for (int v = 0; v < 4; ++v) tred[(wv * 16 + 4 * kq + v) * 64 + jt * 16 + c16] = acc[jt][v];
  __syncthreads();
  for (int i = tid; i < 16 * rp; i += NT) {
    const int m = i / rp, j = i % rp;
    float v = 0.0f;
#pragma unroll
    for (int w2 = 0; w2 < NT / 64; ++w2) v += tred[(w2 * 16 + m) * 64 + j];
    store_dev(sa.tpart + ((int64_t)ts * 16 + m) * rp + j, v);
  }
  // counted done once every store of the workgroup is acknowledged at
  // device scope; the last slice's workgroup sums the slices in order (two
  // entries per thread, every slice's loads issued at once), rounds t to
  // bf16 and publishes it, stamped with the launch's epoch
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) last = add_dev(sa.cnt + SK_TCNT) + 1 == (uint32_t)TS;
  __syncthreads();
  // backward with dB: this slice's columns of dB, once the slice is counted
  // (the last slice publishes u first)
  if (!last) {
    if constexpr (BWD && NT == SK_NT) {
      if (sa.gr.db) sk_fold_db<TSTEPS>(sa, kt0, kt1, xf, tq, reinterpret_cast<uint16_t*>(xs));
    }
    return;
  }
  const rsrc_t rtp = make_rsrc(sa.tpart, clamp_bytes((int64_t)TS * 16 * rp * 4));
  uint64_t* tfin = reinterpret_cast<uint64_t*>(sa.tpart + (int64_t)TS * 16 * rp);
  // the epoch cannot advance before this workgroup publishes t: every
  // epilogue of the launch waits for it
  const uint32_t mark = stamp(__hip_atomic_load(sa.cnt + SK_EPOCH, __ATOMIC_RELAXED, XSCOPE));
  // two entries per thread and pass (rp % 16 == 0: both in one token row)
  for (int e0 = 2 * tid; e0 < 16 * rp; e0 += 2 * NT) {
    float v[2] = {0.0f, 0.0f};
    for (int q0 = 0; q0 < TS; q0 += SK_TMAX) {  // slices in order
      u32x2 part[SK_TMAX];
#pragma unroll
      for (int q = 0; q < SK_TMAX; ++q)
        part[q] = bload8_dev(rtp, opaque_u32(q0 + q < TS ? (uint32_t)(((q0 + q) * 16 * rp + e0) * 4) : LRQ_OOB));
#pragma unroll
      for (int q = 0; q < SK_TMAX; ++q) {
        v[0] += __uint_as_float(part[q][0]);
        v[1] += __uint_as_float(part[q][1]);
      }
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int i = e0 + e, m = i / rp, j = i % rp;
      const uint32_t hb = pack_bf16x2(sa.scaling * v[e], 0.0f) & 0xffffu;  // t (u) as the caller sees it
      // value and stamp in one 8-byte store: a reader sees both or neither
      __hip_atomic_store(tfin + i, ((uint64_t)mark << 32) | (hb << 16), __ATOMIC_RELAXED, XSCOPE);
      if (sa.t_out && m < M && (BWD || j < r)) sa.t_out[(int64_t)m * (BWD ? rp : r) + j] = (uint16_t)hb;
    }
  }
  if constexpr (BWD && NT == SK_NT) {
    if (sa.gr.db) sk_fold_db<TSTEPS>(sa, kt0, kt1, xf, tq, reinterpret_cast<uint16_t*>(xs));
  }
}

// The loads of one wavefront's run of reduction blocks [kb0, kb0 + nkb)
// (at most WB; the rest read zeros) for row tiles rt0 .. rt0 + RTN - 1 (16
// weight rows each) of block row nb, all issued at once in block order: the
// x fragments, then the row tiles' packed words (and int4 scales); block b
// is consumed once its loads are in.
//
// int4 words are loaded 16 bytes per lane, two row tiles per instruction:
// lane l reads row 16 (2p + l / 32) + l % 16, depth half (l / 16) % 2 (32
// values), and two v_permlane32_swap hand each tile's 8 bytes to all 64
// lanes (sk_int4_pair). Lane (c16, kq) then holds depths
// sk_depth(kq) .. + 16 = 32 (kq % 2) + 16 (kq / 2) of its row; its x
// fragment and (backward) its depth scale follow the same order. Half as
// many load instructions as 8-byte loads per tile (a load-only copy of the
// forward's stream: 9.7 -> 7.2 us; the whole NS forward, with the in-place
// partial products of sk_math: 12.6 -> 12.2 us).
template <int FMT, bool BWD, int WB, int RTN>
struct SkRun {
  static constexpr bool I4 = FMT == LRQ_FMT_INT4;
  static constexpr bool GS = FMT != LRQ_FMT_FP8;  // group scales
  static_assert(!I4 || RTN % 2 == 0, "int4 row tiles are loaded in pairs");
  u32x4 xf[WB][2];
  u32x4 w4[I4 ? WB : 1][I4 ? RTN / 2 : 1];  // tile pairs as loaded
  u32x2 w8[I4 ? 1 : WB][RTN][2];
  // forward int4 / int8: per row tile; backward: lane c16's depth (fp8: [b][0])
  float sc[(GS || BWD) ? WB : 1][RTN];
};

// first depth (within a 64-wide block) of lane group kq's 16 values
template <int FMT>
LRQ_DEV int sk_depth(int kq) {
  return FMT == LRQ_FMT_INT4 ? 32 * (kq & 1) + 16 * (kq >> 1) : 16 * kq;
}

// the two row tiles' fragments (dwords jj = 0, 1) from a pair as loaded:
// lanes 0-31 hold tile 0's words, lanes 32-63 tile 1's; swapping the upper
// half of words 0, 1 with the lower half of words 2, 3 leaves tile 0 in
// words 0, 1 and tile 1 in words 2, 3 of every lane
LRQ_DEV void sk_int4_pair(const u32x4& v, u32x2& t0, u32x2& t1) {
  const auto s0 = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
  const auto s1 = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
  t0 = (u32x2){s0[0], s1[0]};
  t1 = (u32x2){s0[1], s1[1]};
}

template <int FMT, bool BWD, int WB, int RTN, bool ONEG = false>
LRQ_DEV void sk_load(const GemmArgs& a, SkRun<FMT, BWD, WB, RTN>& R, int64_t nb, int rt0, int kb0, int nkb) {
  constexpr bool I4 = FMT == LRQ_FMT_INT4;
  constexpr bool GS = FMT != LRQ_FMT_FP8;
  const int lane = threadIdx.x & 63, c16 = lane & 15, kq = lane >> 4;
  const int64_t M = a.m, K = a.l, E = a.e;
  const int64_t KB = (K + 63) / 64;
  constexpr uint32_t blkb = I4 ? 2048u : 4096u;
  constexpr uint32_t rowb = I4 ? 32u : 64u;
  const rsrc_t rw = make_rsrc(a.wdata + nb * KB * blkb, clamp_bytes(KB * (int64_t)blkb));
  const int64_t Gp = GS ? ((KB * 64) >> a.gshift) : 0;
  // forward: int4 / int8 group scales of the block row ([NB][Gp][64]);
  // backward: the per-depth scales (int4 / int8 the transposed table
  // ST [KGt][64 KB], fp8 the channel scales [depth] or one scalar)
  const int64_t NP = KB * 64;
  const int64_t KGt = (BWD && GS) ? (((E + 63) / 64 * 64 + (1 << a.gshift) - 1) >> a.gshift) : 0;
  const rsrc_t rs = BWD ? (GS ? make_rsrc(a.wscale, clamp_bytes(KGt * NP * 4))
                              : make_rsrc(a.wscale, a.per_channel ? clamp_bytes(K * 4) : 0u))
                        : (GS ? make_rsrc(a.wscale + nb * Gp * 64, clamp_bytes(Gp * 64 * 4)) : make_rsrc(a.wscale, 4u));
  const float s0add = (BWD && !GS && !a.per_channel) ? a.wscale[0] : 0.0f;
  const rsrc_t rx = make_rsrc(a.act, clamp_bytes(M * K * 2));
  const int kd = sk_depth<FMT>(kq);
  // fp8, int8: 16 bytes of row c16 per tile; int4: 16 bytes of row c16 of tile
  // lane / 32 of the pair, depth half (lane / 16) % 2
  const uint32_t woff = I4 ? (uint32_t)((lane >> 5) * 16 + c16) * rowb + (uint32_t)((lane >> 4) & 1) * 16u
                           : (uint32_t)c16 * rowb + (uint32_t)kq * 16u;
  const uint32_t xoff = (uint32_t)(((int64_t)c16 * K + kd) * 2);
#pragma unroll
  for (int b = 0; b < WB; ++b) {
    const bool ok = b < nkb;
    const uint32_t kb = (uint32_t)(kb0 + b);
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int64_t k = (int64_t)kb * 64 + kd + jj * 8;
      const bool xok = ok && k < K;  // K % 8 == 0
      R.xf[b][jj] = bload16(rx, opaque_u32(xok ? xoff + (uint32_t)(((int64_t)kb * 64 + jj * 8) * 2) : LRQ_OOB));
    }
    // backward: lane (kq, c16) holds the scale of depth 64 kb + kd + c16,
    // which the 16 lanes of its DPP row (one kq) broadcast among themselves
    const uint32_t dpos = kb * 64u + (uint32_t)(kd + c16);
    if (BWD && !GS) R.sc[b][0] = bloadf(rs, opaque_u32(ok ? dpos * 4u : LRQ_OOB)) + s0add;
#pragma unroll
    for (int rt = 0; rt < RTN; ++rt) {
      const int rg = rt0 + rt;  // row tile within the 64-row block row
      const uint32_t wo = kb * blkb + (uint32_t)(rg * 16) * rowb + woff;
      if constexpr (I4) {
        if (rt % 2 == 0) R.w4[b][rt / 2] = bload16(rw, opaque_u32(ok ? wo : LRQ_OOB));
      } else {
        const u32x4 v = bload16(rw, opaque_u32(ok ? wo : LRQ_OOB));
        R.w8[b][rt][0] = (u32x2){v[0], v[1]};
        R.w8[b][rt][1] = (u32x2){v[2], v[3]};
      }
      if constexpr (GS) {
        if (BWD) {
          // group of output rows 64 nb + 16 rg .. +16 (groups are >= 32 and
          // aligned); with groups of 64 or more (ONEG) one for all the row
          // tiles, loaded once
          const uint32_t kg = (uint32_t)((nb * 64 + rg * 16) >> a.gshift);
          if (!ONEG || rt == 0) R.sc[b][rt] = bloadf(rs, opaque_u32(ok ? (uint32_t)((kg * NP + dpos) * 4) : LRQ_OOB));
        } else {
          const uint32_t j = (kb * 64u + (uint32_t)kd) >> a.gshift;
          R.sc[b][rt] = bloadf(rs, opaque_u32(ok ? (j * 64u + (uint32_t)(rg * 16 + c16)) * 4u : LRQ_OOB));
        }
      }
    }
  }
}

// The matrix-core steps of a run, block by block into acc[RTN] (C element v
// of lane l: token 4*(l/16) + v, weight row 16 rt + l%16 of the run's tiles).
template <int FMT, bool BWD, bool MQ, int WB, int RTN>
LRQ_DEV void sk_math(const GemmArgs& a, const SkRun<FMT, BWD, WB, RTN>& R, f32x4 (&acc)[RTN]) {
  constexpr bool I4 = FMT == LRQ_FMT_INT4;
  constexpr bool I8 = FMT == LRQ_FMT_INT8;
#pragma unroll
  for (int rt = 0; rt < RTN; ++rt) acc[rt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int b = 0; b < WB; ++b) {
    // blocks past this wavefront's run hold zeros: the steps stay
    // unconditional (a matrix-core result read in another block than the
    // one that wrote it has come back stale)
    u32x2 w4[I4 ? RTN : 1];
    if constexpr (I4) {
#pragma unroll
      for (int p = 0; p < RTN / 2; ++p) sk_int4_pair(R.w4[b][p], w4[2 * p], w4[2 * p + 1]);
    }
    if constexpr (MQ && !BWD) {
      const u32x4 ones = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
      f32x4 xsum = {0.0f, 0.0f, 0.0f, 0.0f};
      u32x4 xp[2];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const u32x4 v = R.xf[b][jj];
        xsum = mfma16(as_bf16x8(v), as_bf16x8(ones), xsum);
        // k order 0 4 1 5 2 6 3 7, as the weight pairs below
        xp[jj] = (u32x4){__builtin_amdgcn_perm(v[2], v[0], 0x05040100u), __builtin_amdgcn_perm(v[2], v[0], 0x07060302u),
                         __builtin_amdgcn_perm(v[3], v[1], 0x05040100u), __builtin_amdgcn_perm(v[3], v[1], 0x07060302u)};
      }
#pragma unroll
      for (int rt = 0; rt < RTN; ++rt) {
        // an opaque zero in VGPRs: the two chained steps then accumulate in
        // place (with a literal zero the second step's destination was
        // allocated partly over the first's within its 8 wait states; the
        // AGPR-pinned zero also fixes that but moved the scales to AGPRs
        // and cost 0.3 us per NS forward)
        f32x4 ab = {0.0f, 0.0f, 0.0f, 0.0f};
        asm volatile("" : "+v"(ab));
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          const uint32_t d = w4[rt][jj];
          // (u_e, u_e+4) as bf16 (128 + u) pairs
          const u32x4 wb = {(d & 0x000f000fu) | 0x43004300u, ((d >> 4) & 0x000f000fu) | 0x43004300u,
                            ((d >> 8) & 0x000f000fu) | 0x43004300u, ((d >> 12) & 0x000f000fu) | 0x43004300u};
          ab = mfma16(as_bf16x8(xp[jj]), as_bf16x8(wb), ab);
        }
#pragma unroll
        for (int v = 0; v < 4; ++v)
          acc[rt][v] = __builtin_fmaf(R.sc[b][rt], __builtin_fmaf(-136.0f, xsum[v], ab[v]), acc[rt][v]);
      }
      continue;
    }
#pragma unroll
    for (int rt = 0; rt < RTN; ++rt) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        u32x4 wb;
        if constexpr (BWD) {
          // transposed section: value e is q (a sign-extended nibble or
          // byte, or the e4m3 value) times the scale of its depth
          // kd + 8 jj + e, then bf16
          float f[8];
          if (I4) {
            int4x8_to_f32_div16(w4[rt][jj], f);  // q / 16, times 16 x the scale below
          } else if (I8) {
            int8x4_to_f32(R.w8[b][rt][jj][0], f);
            int8x4_to_f32(R.w8[b][rt][jj][1], f + 4);
          } else {
            fp8x4_to_f32(R.w8[b][rt][jj][0], f);
            fp8x4_to_f32(R.w8[b][rt][jj][1], f + 4);
          }
          const float S = (I4 ? 16.0f : 1.0f) * R.sc[b][(I4 || I8) && !MQ ? rt : 0];
          mul_row_bcast8(f, S, jj);
#pragma unroll
          for (int q = 0; q < 4; ++q) wb[q] = pack_bf16x2(f[2 * q], f[2 * q + 1]);
        } else if constexpr (I4) {
          wb = dequant8_int4_bf16(w4[rt][jj], R.sc[b][rt], a.nib);
        } else if constexpr (I8) {
          wb = dequant8_int8_bf16(R.w8[b][rt][jj], R.sc[b][rt]);
        } else {
          const u32x2 p0 = fp8x4_to_bf16(R.w8[b][rt][jj][0]), p1 = fp8x4_to_bf16(R.w8[b][rt][jj][1]);
          wb = (u32x4){p0[0], p0[1], p1[0], p1[1]};
        }
        acc[rt] = mfma16(as_bf16x8(R.xf[b][jj]), as_bf16x8(wb), acc[rt]);
      }
    }
  }
}

// MQ (int4 forward, groups of 64 or more, so one group per 64-wide block):
// the matrix-core operand is the stored nibble u = q + 8 as the exact bf16
// value 128 + u (bits 0x4300 | u, two bit operations per pair), each block
// is multiplied into fresh accumulators, and the block's partial is scaled
// in f32: s * (sum x (128 + u) - 136 sum x) = s * sum x q. The block sums of
// x come from one more matrix-core step against ones.
// MQ in the backward (int4 or int8, groups of 64 or more): one scale group
// over a block row's 64 output rows, so its per-depth scales are loaded
// once for the four row tiles.
// TSTEPS: 32-wide k steps per wavefront of a t (u) slice (1, 2 or 4)
template <int FMT, bool BWD, bool MQ, int TSTEPS>
__global__ void __launch_bounds__(SK_NT) k_sk(SkArgs sa) {
  constexpr bool I4 = FMT == LRQ_FMT_INT4;
  // cross-wavefront reduction buffer: [4 wavefronts][64 columns][16 tokens]
  // (backward with dB: the u slices then stage dy and t there, 128 TSTEPS * 16
  // + 1024 bf16)
  __shared__ __attribute__((aligned(16))) float xs[SK_LDSF];
  __shared__ int last;  // this workgroup was the last of its block row (t: of the t slices)
  const GemmArgs& a = sa.g;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, kq = lane >> 4;
  const int64_t M = a.m, K = a.l, E = a.e;  // K: the depth (d_in forward, d_out backward)
  const int64_t KB = (K + 63) / 64;
  const int TS = sa.p.TS;

  if ((int)blockIdx.x < TS) {
    sk_t_slices<BWD, TSTEPS, SK_NT, SK_LDSF>(sa, xs, last);
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

  SkRun<FMT, BWD, SK_WB, 4> R;
  sk_load<FMT, BWD, SK_WB, 4, BWD && MQ>(a, R, nb, 0, kb0, nkb);

  // keep every load ahead of the math (the scheduler would otherwise trade
  // loads in flight for registers)
  __builtin_amdgcn_sched_barrier(0);
  f32x4 acc[4];
  sk_math<FMT, BWD, MQ, SK_WB, 4>(a, R, acc);
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
      if (n < E) store_dev(sa.part + ((int64_t)s * M + m) * E + n, v);
    }
  }
  // arrive once every store of the workgroup is acknowledged at device scope;
  // the last of the block row's S splits runs its epilogue, once t is in
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    last = add_dev(sa.cnt + nb) + 1 == (uint32_t)S;
    if (last) zero_dev(sa.cnt + nb);
  }
  __syncthreads();
  if (!last) return;
  sk_epilogue<FMT, BWD>(sa, nb, xs);
  // the last epilogue of the launch resets the t and epilogue counters and
  // advances the epoch (every read of t, and of the epoch, is over by then)
  if (tid == 0 && add_dev(sa.cnt + SK_DCNT) + 1 == (uint32_t)((E + 63) / 64)) {
    zero_dev(sa.cnt + SK_TCNT);
    zero_dev(sa.cnt + SK_DCNT);
    add_dev(sa.cnt + SK_EPOCH);
  }
}

// ---------------------------------------------------------------- full depth
// Forward with d_in <= 4 * SKF_WB * 64: a workgroup owns 16 RT weight rows (RT
// of the four 16-row tiles of a 64-row block row) over the whole reduction. Its four wavefronts take
// consecutive runs of the blocks (every load of a run issued at once, as in
// k_sk), meet in LDS and the workgroup finishes its rows itself:
//   y[m, n] = bf16(sc[n] * base[m, n] + sum_j t[m, j] B[j, n] + bias[n])
// so no split partial, counter or finishing epilogue sits between the weight
// stream and y. t comes from the same t workgroups and stamped publication
// as in k_sk (dispatched first, waiting on nothing).
constexpr int SKF_WB = 12;  // blocks per run of four wavefronts (d_in <= 3072); NT / 64 runs share them
constexpr int SKF_RT = 4;   // 16-row tiles per workgroup
constexpr int SKF_NT = 512; // threads per workgroup

// The epilogue of the 16 RT rows n0 ..: `red` holds the runs' sums
// [NT / 64][RT tiles][16 tokens][16 rows], then (with t) the LoRA term in the
// same layout. Thread (tid < 256): token m = tid / 16, column pairs cq + 16 h.
template <int FMT, int RT, int NT>
LRQ_DEV void skf_epilogue(const SkArgs& sa, int64_t n0, const float* red) {
  constexpr int NP = 8 * RT;                 // column pairs
  constexpr int NW = NT / 64;                // runs
  constexpr int PH = NP > 16 ? NP / 16 : 1;  // pairs per thread
  const GemmArgs& a = sa.g;
  const int tid = threadIdx.x;
  const int64_t M = a.m, E = a.e;
  const bool lora = sa.p.TS > 0;
  if (tid >= 256) return;
  const int m = tid >> 4, cq = tid & 15;
#pragma unroll
  for (int h = 0; h < PH; ++h) {
    const int pc = cq + 16 * h;  // column pair: row tile pc / 8
    const int64_t n = n0 + 2 * pc;
    if (!(m < M && pc < NP && n < E)) continue;  // E % 8 == 0: n < E implies n + 1 < E
    float base[2], l[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int cl = 2 * pc + e, rt = cl >> 4, c = cl & 15;
      float v = 0.0f;
#pragma unroll
      for (int w2 = 0; w2 < NW; ++w2) v += red[((w2 * RT + rt) * 16 + m) * 16 + c];
      base[e] = v;
      l[e] = lora ? red[((NW * RT + rt) * 16 + m) * 16 + c] : 0.0f;
    }
    float sc[2] = {1.0f, 1.0f}, bias[2] = {0.0f, 0.0f};
    if (FMT == LRQ_FMT_FP8) {
#pragma unroll
      for (int e = 0; e < 2; ++e) sc[e] = a.wscale[a.per_channel ? n + e : 0];
    }
    if (a.bias) {
#pragma unroll
      for (int e = 0; e < 2; ++e) bias[e] = a.bias[n + e];
    }
    *reinterpret_cast<uint32_t*>(a.out + (int64_t)m * E + n) =
        pack_bf16x2(base[0] * sc[0] + l[0] + bias[0], base[1] * sc[1] + l[1] + bias[1]);
  }
}

template <int FMT, bool MQ, int TSTEPS, int RT, int NT>
__global__ void __launch_bounds__(NT) k_skf(SkArgs sa) {
  constexpr int NP = 8 * RT;   // column pairs of the workgroup's rows
  constexpr int NW = NT / 64;  // runs
  // LDS: the runs' sums and the LoRA term [NW + 1][RT][16][16], then the
  // factor slice B[j][rows] as column pairs [64][NP]; the t slices use the
  // first NW * 1024 floats
  constexpr int RED = (NW + 1) * RT * 16 * 16, XS = RED + 64 * NP;
  __shared__ __attribute__((aligned(16))) float xs[XS > NW * 1024 ? XS : NW * 1024];
  __shared__ int last;
  const GemmArgs& a = sa.g;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, kq = lane >> 4;
  const int64_t K = a.l, E = a.e;
  const int64_t KB = (K + 63) / 64;
  const int TS = sa.p.TS, rp = a.rp;
  if ((int)blockIdx.x < TS) {
    sk_t_slices<false, TSTEPS, NT, (XS > NW * 1024 ? XS : NW * 1024)>(sa, xs, last);
    return;
  }
  const int64_t hb = (int64_t)blockIdx.x - TS;  // this workgroup's rows: tiles RT (hb % (4 / RT)) .. of block row nb
  const int64_t nb = hb / (4 / RT);
  const int rt0 = (int)(hb % (4 / RT)) * RT;
  const int64_t n0 = hb * 16 * RT;
  const int kb0 = (int)((KB * wv) / NW), nkb = (int)((KB * (wv + 1)) / NW) - kb0;

  // the factor slice B[j][n0 ..] as column pairs (4-byte loads), out ahead of
  // the weight stream: entry i = tid + NT q is (j = i / NP, pair i % NP)
  constexpr int NBQ = (64 * NP + NT - 1) / NT;
  uint32_t bq[NBQ];
  {
    const rsrc_t rb = make_rsrc(a.lw, TS > 0 ? clamp_bytes((int64_t)a.r * E * 2) : 0u);
#pragma unroll
    for (int q = 0; q < NBQ; ++q) {
      const int i = tid + q * NT, j = i / NP, pc = i % NP;
      const int64_t nn = n0 + 2 * pc;
      const bool ok = j < a.r && nn < E;
      bq[q] = bload4(rb, opaque_u32(ok ? (uint32_t)(((int64_t)j * E + nn) * 2) : LRQ_OOB));
    }
  }
  constexpr int WB = (SKF_WB * 4 + NW - 1) / NW;  // blocks per run, at most
  SkRun<FMT, false, WB, RT> R;
  sk_load<FMT, false, WB, RT>(a, R, nb, rt0, kb0, nkb);
  // keep every load ahead of the rest
  __builtin_amdgcn_sched_barrier(0);
  uint32_t* bsl = reinterpret_cast<uint32_t*>(xs + RED);
#pragma unroll
  for (int q = 0; q < NBQ; ++q)
    if (tid + q * NT < 64 * NP) bsl[tid + q * NT] = bq[q];
  __syncthreads();  // (the factor slice only waits for its own loads, issued first)
  f32x4 acc[RT];
  sk_math<FMT, false, MQ, WB, RT>(a, R, acc);
  float* red = xs;
  if (TS > 0 && wv == 0) {
    // the first run to finish adds t . B for the workgroup's rows, a
    // rank-wide matrix-core step per row tile, while the others still
    // stream: t in the A role (lane (c16, kq): t[c16][32 ks + 8 kq ..]) as
    // published, every entry stamped with the launch's epoch
    const uint32_t want = stamp(__hip_atomic_load(sa.cnt + SK_EPOCH, __ATOMIC_RELAXED, XSCOPE)) + sa.skew;
    const rsrc_t rtf = make_rsrc(sa.tpart + (int64_t)TS * 16 * rp, clamp_bytes((int64_t)16 * rp * 8));
    u32x2 tv[2][8];
    auto load_t = [&]() {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int j = 32 * ks + 8 * kq + e;
          tv[ks][e] = bload8_dev(rtf, opaque_u32(j < rp ? (uint32_t)((c16 * rp + j) * 8) : LRQ_OOB));
        }
    };
    load_t();
    for (uint32_t polls = 0;; ++polls) {
      bool ok = true;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) ok = ok && (32 * ks + 8 * kq + e >= rp || tv[ks][e][1] == want);
      if (__all(ok)) break;
      if (polls == sa.max_polls) {
        __hip_atomic_store(sa.cnt + SK_FAIL, 1u, __ATOMIC_RELAXED, XSCOPE);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int e = 0; e < 8; ++e) tv[ks][e][0] = SK_NAN2;
        break;
      }
      __builtin_amdgcn_s_sleep(2);
      load_t();
    }
    // B in the B role (lane (c16, kq): B[32 ks + 8 kq ..][row 16 rt + c16])
    // from the staged slice; rank steps past rp multiply zeros
    f32x4 lacc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) lacc[rt] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
    const uint16_t* bsh = reinterpret_cast<const uint16_t*>(bsl);  // [64 j][2 NP] bf16
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      u32x4 ta;
#pragma unroll
      for (int q = 0; q < 4; ++q) ta[q] = (tv[ks][2 * q][0] >> 16) | (tv[ks][2 * q + 1][0] & 0xffff0000u);
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        u32x4 bb;
        const int col = 16 * rt + c16;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int j = 32 * ks + 8 * kq + 2 * q;
          bb[q] = (uint32_t)bsh[j * 2 * NP + col] | ((uint32_t)bsh[(j + 1) * 2 * NP + col] << 16);
        }
        lacc[rt] = mfma16(as_bf16x8(ta), as_bf16x8(bb), lacc[rt]);
      }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[((NW * RT + rt) * 16 + 4 * kq + v) * 16 + c16] = lacc[rt][v];
  }
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[((wv * RT + rt) * 16 + 4 * kq + v) * 16 + c16] = acc[rt][v];
  __syncthreads();
  skf_epilogue<FMT, RT, NT>(sa, n0, red);
  // the last workgroup of the launch resets the t and epilogue counters and
  // advances the epoch (every read of t, and of the epoch, is over by then)
  if (tid == 0 && add_dev(sa.cnt + SK_DCNT) + 1 == (uint32_t)((E + 16 * RT - 1) / (16 * RT))) {
    zero_dev(sa.cnt + SK_TCNT);
    zero_dev(sa.cnt + SK_DCNT);
    add_dev(sa.cnt + SK_EPOCH);
  }
}

}  // namespace

bool g_force_wait_timeout = false;
void set_force_wait_timeout(bool on) { g_force_wait_timeout = on; }
bool force_wait_timeout() { return g_force_wait_timeout; }

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
  // t: slices of 128, 256 or 512 k (one, two or four 32-wide steps per
  // wavefront), the smallest that keeps the slices at 32 or fewer
  if (rp > 0) {
    int64_t steps = 1;
    while (steps < 4 && (k + 128 * steps - 1) / (128 * steps) > SK_TMAX) steps *= 2;
    p.KT = 128 * steps;
    p.TS = (int)((k + p.KT - 1) / p.KT);
    if (p.TS < 1) p.TS = 1;
  }
  // whole-depth workgroups (k_skf, forward only) when the depth fits a
  // workgroup's runs and its workgroups are many (>= 128) yet fit the CUs in
  // one round with the t slices. Measured per shape at m = 16 (graph
  // replay over rotated weights, us, k_skf against splits): 3072 -> 12288
  // 12.7 / 13.4, 3072 -> 9216 11.9 / 12.6, 2560 -> 9728 11.9 / 12.4; but
  // 2560 -> 4096 10.8 / 10.8, 2560 -> 1024 9.9 / 9.0, 3072 -> 18432 (288
  // workgroups) 20.6 / 16.3.
  const int64_t nwf = (n + 16 * SKF_RT - 1) / (16 * SKF_RT);  // k_skf workgroups
  p.full = KB <= 4 * SKF_WB && nwf >= 128 && nwf + p.TS <= num_cus;
  return p;
}

size_t skinny_ws_bytes(const SkinnyPlan& p, int64_t m, int64_t n, int rp) {
  const size_t part = (size_t)p.S * m * n * 4, tp = (size_t)(p.TS + 2) * 16 * rp * 4;
  return (part + 255) / 256 * 256 + tp + 256;
}

hipError_t launch_skinny(hipStream_t st, int fmt, bool bwd, const GemmArgs& a, const uint16_t* A,
                         const SkinnyPlan& p, float* part, float* tpart, uint32_t* cnt, float scaling,
                         uint16_t* t_out, const SkGrads& gr) {
  const int64_t NB = (a.e + 63) / 64;
  if (a.m <= 0 || a.m > 16 || p.S < 1 || p.KS < 1 || p.KS > SK_MAXKS || !cnt || NB > SK_MAX_NB)
    return hipErrorInvalidValue;
  if (!bwd && (gr.da || gr.db)) return hipErrorInvalidValue;
  if ((gr.da && !gr.x) || (gr.db && !gr.t) || ((gr.da || gr.db) && (a.rp == 0 || !A))) return hipErrorInvalidValue;
  SkArgs sa{a, A, p, part, tpart, cnt, scaling, t_out, SK_MAX_POLLS, 0u, gr};
  if (g_force_wait_timeout) {
    sa.max_polls = 16;
    sa.skew = 0x40000000u;  // a stamp no launch publishes
  }
  if (a.rp == 0 || !A) sa.p.TS = 0;
  // 32-wide steps per wavefront of a t slice (skinny_plan; 0 without t)
  const int steps = (int)(p.KT / 128);
  if (!bwd && p.full) {
    // whole-depth workgroups, no splits (skinny_plan)
    const unsigned gridf = (unsigned)((a.e + 16 * SKF_RT - 1) / (16 * SKF_RT) + sa.p.TS);
#define SKF_LAUNCH(F, Q)                                                                                 \
  switch (steps) {                                                                                       \
    case 4: case 3: hipLaunchKernelGGL((k_skf<F, Q, 4, SKF_RT, SKF_NT>), dim3(gridf), dim3(SKF_NT), 0, st, sa); break; \
    case 2: hipLaunchKernelGGL((k_skf<F, Q, 2, SKF_RT, SKF_NT>), dim3(gridf), dim3(SKF_NT), 0, st, sa); break;         \
    default: hipLaunchKernelGGL((k_skf<F, Q, 1, SKF_RT, SKF_NT>), dim3(gridf), dim3(SKF_NT), 0, st, sa); break;        \
  }
    if (fmt == LRQ_FMT_INT4) {
      if (a.gshift >= 6) {
        SKF_LAUNCH(LRQ_FMT_INT4, true)
      } else {
        SKF_LAUNCH(LRQ_FMT_INT4, false)
      }
    } else if (fmt == LRQ_FMT_INT8) {
      SKF_LAUNCH(LRQ_FMT_INT8, false)
    } else {
      SKF_LAUNCH(LRQ_FMT_FP8, false)
    }
#undef SKF_LAUNCH
    return hipGetLastError();
  }
  const unsigned grid = (unsigned)(NB * p.S + sa.p.TS);
#define SK_LAUNCH(F, B, Q)                                                                             \
  switch (steps) {                                                                                     \
    case 4: case 3: hipLaunchKernelGGL((k_sk<F, B, Q, 4>), dim3(grid), dim3(SK_NT), 0, st, sa); break; \
    case 2: hipLaunchKernelGGL((k_sk<F, B, Q, 2>), dim3(grid), dim3(SK_NT), 0, st, sa); break;       \
    default: hipLaunchKernelGGL((k_sk<F, B, Q, 1>), dim3(grid), dim3(SK_NT), 0, st, sa); break;      \
  }
  if (fmt == LRQ_FMT_INT4) {
    if (bwd) {
      if (a.gshift >= 6) {
        SK_LAUNCH(LRQ_FMT_INT4, true, true)
      } else {
        SK_LAUNCH(LRQ_FMT_INT4, true, false)
      }
    } else if (a.gshift >= 6) {
      SK_LAUNCH(LRQ_FMT_INT4, false, true)
    } else {
      SK_LAUNCH(LRQ_FMT_INT4, false, false)
    }
  } else if (fmt == LRQ_FMT_INT8) {
    if (bwd) {
      if (a.gshift >= 6) {
        SK_LAUNCH(LRQ_FMT_INT8, true, true)
      } else {
        SK_LAUNCH(LRQ_FMT_INT8, true, false)
      }
    } else {
      SK_LAUNCH(LRQ_FMT_INT8, false, false)
    }
  } else {
    if (bwd) {
      SK_LAUNCH(LRQ_FMT_FP8, true, false)
    } else {
      SK_LAUNCH(LRQ_FMT_FP8, false, false)
    }
  }
#undef SK_LAUNCH
  return hipGetLastError();
}
