// The two GEMMs of the quantized LoRA linear for mid token counts (the
// token count that leaves the 256 x 256 tiles of lrq_gemm.hip too few to
// fill the CUs), without splitting the depth:
//
//   forward   y[m, n]  = x[m, k]  . bf16(dq(w))[n, k]^T (+bias) + t[m, :] . B[:, n]
//   backward  dx[m, k] = dy[m, n] . bf16(dq(w))[n, k]            + u[m, :] . A[k, :]^T
//
// (src/quant.rs:175-176 and :229-233; the LoRA terms of src/lora.rs:199-203
// with t, u and the weight-side factor rows prepared by the LoRA side
// kernels, as for the large tiles.)
//
// "Rows" are the output columns (n forward, k backward), "depth" the
// reduction index. A tile is 64 rows x T tokens (T = 16 TT: 64 or 128) over
// the whole depth, one workgroup of four wavefronts, two workgroups per CU:
//   - wavefront w owns rows 16w .. 16w+15 of the tile for all T tokens, so
//     each weight element is dequantized once per tile and each dequantized
//     fragment feeds TT matrix-core steps (v_mfma_f32_16x16x32_bf16, weight
//     rows in the A role, tokens in the B role);
//   - weight: per 64-wide depth step a lane loads the packed bytes of its
//     row (l & 15) for depths 16 (l >> 4) .. +16 from the blocked layout
//     (int4 8 bytes, fp8 and int8 16): the 16 rows x 64 depth of a
//     wavefront are one contiguous 512- or 1024-byte run. Sub-step kk of a
//     step takes depths 16 (l >> 4) + 8 kk .. +8 in the MFMA's k slots
//     8 (l >> 4) .. +8, and the activation fragments follow the same order.
//     Forward: fma(u, s, -8s) = q s exactly (int4), the int8 analogue, or
//     the exact e4m3 value (its channel scale multiplies the accumulators in
//     the epilogue), then bf16. Backward (the transposed section): each of a
//     lane's values has its own depth's scale; lane l of each 16-lane row
//     loads the scale of depth 16 (l >> 4) + (l & 15) and a DPP row
//     broadcast hands it to the lanes that need it: bf16(q s) again;
//   - activations: the T x 64 slice of a step is copied global -> LDS by
//     buffer loads with an LDS destination (16-byte chunk c of row r stored
//     at chunk c ^ ((r >> 1) & 7)), four stages in flight, each in its own
//     LDS array so that the compiler's waits track them apart; one barrier
//     per step;
//   - epilogue: the LoRA term as rank-wide matrix-core steps (the tile's
//     token-side rows t or u and weight-side rows B^T or A from the
//     workspace), the forward fp8 channel scales and the bias, bf16 stores;
//   - FOLD (ranks 8 to 32, multiples of 8): the token-side rows are formed in the same
//     launch, so no side launch precedes it. The first workgroups of the
//     grid (dispatched first, on the CU slots the tiles leave free) each
//     take 64 tokens and a depth slice of 384: t = x . A (or u = dy . B^T)
//     as matrix-core steps, factor rows in the A role; f32 partials at
//     device scope, the last slice of a group sums them in order, stores
//     bf16(s . sum) (t for the caller, u for dA) and publishes the group's
//     ready flag stamped with the launch's epoch. A tile waits for its
//     groups' flags before its LoRA step (bounded: it never waits for a
//     workgroup that is not running, and a wait that runs out flags a
//     failure and uses NaN). The weight-side rows come from the raw factor
//     (B across its rows, divided by an fp8 weight scale; A's rows). The
//     last tile to finish clears the flags and advances the epoch;
//   - tile order: the tiles are cut into groups of up to eight token tiles
//     by all row tiles, token tile fastest, and each XCD (own L2) takes a
//     contiguous range, so an XCD's tiles share a few token tiles of the
//     activations and a band of weight rows.
// Edges: rows past M, E and the depth read zeros (buffer-resource bounds),
// the depth runs in whole rounds of four steps (the tail reads zeros), and
// outputs past M or E are not stored.

#include "lrq_common.h"
#include "lrq_kernels.h"
#include "lrq_tn.h"

namespace {

// device-scope accesses of the fold's cross-workgroup data (written through
// and read past the per-XCD L2s), as in lrq_skinny.hip
constexpr int MXSCOPE = __HIP_MEMORY_SCOPE_AGENT;
LRQ_DEV uint32_t madd_dev(uint32_t* c) { return __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, MXSCOPE); }
LRQ_DEV void mzero_dev(uint32_t* c) { __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, MXSCOPE); }
LRQ_DEV uint32_t mload_dev(const uint32_t* c) { return __hip_atomic_load(c, __ATOMIC_RELAXED, MXSCOPE); }
LRQ_DEV u32x4 mbload16_dev(rsrc_t r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16); }
LRQ_DEV void mstore16_dev(rsrc_t r, uint32_t off, const u32x4& v) { __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 16); }
LRQ_DEV void mstore8_dev(rsrc_t r, uint32_t off, const u32x2& v) { __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, 16); }
LRQ_DEV uint32_t mstamp(uint32_t ep) { return ep + 1 == 0 ? 1u : ep + 1; }
constexpr uint32_t MID_MAX_POLLS = 1u << 22;  // about 0.2 s of s_sleep 2
// the fold's counters: per 64-token group the slices' arrivals at [0, G)
// and the ready flags at [G, 2 G)

constexpr int MD = 64;    // depth per step (one 64 x 64 weight block)
constexpr int MR = 64;    // rows per tile: four wavefronts of 16
constexpr int MST = MID_MST;  // pipeline stages

// LDS chunk swizzle: rows r and r + 1 share a chunk order, so the 16 rows a
// quarter-wavefront reads at one logical chunk cover all 64 banks
LRQ_DEV int mswz(int r) { return (r >> 1) & 7; }

// FOLD: workgroup fw of the factor workgroups: 64-token group fw / fold_slices,
// depth slice fw % fold_slices, RT rank tiles of 16 (rp = 16 RT). Wavefront
// w takes tokens 16 w .. + 16 of the group; each of its lanes loads the
// group's token row 16 w + (l & 15) at depths 32 ss + 8 (l >> 4) .. + 8 of
// the slice (every load of the slice at once) and the factor fragments of
// the same depths for ranks 16 rt + (l & 15): forward A's rows staged
// transposed in LDS (rank tile rt's aT [16][FKT + 8] in lds[rt]), backward
// B's rows read directly. `want` is the launch's stamp.
template <bool BWD, int RT>
LRQ_DEV void mid_fold_slice(const GemmArgs& a, int fw, uint16_t* lds0, uint16_t* lds1, uint32_t want) {
  constexpr int FKT = MID_FOLD_KT, NSS = FKT / 32, AST = FKT + 8, RP = 16 * RT;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15, kq = lane >> 4;
  const int fs = a.fold_slices, g = fw / fs, sl = fw % fs;
  const int64_t M = a.m, D = a.l, Mp = (M + 63) / 64 * 64;
  const int r = a.r;
  const int64_t k0 = (int64_t)sl * FKT, k1 = k0 + FKT < D ? k0 + FKT : D;
  const int64_t tok = (int64_t)g * 64 + 16 * w + c16;
  const rsrc_t rx = make_rsrc(a.act, clamp_bytes(M * D * 2));
  const rsrc_t rf = make_rsrc(a.lact, clamp_bytes(D * r * 2));
  uint16_t* const lds[2] = {lds0, lds1};
  u32x4 xf[NSS], bf[RT][NSS];
#pragma unroll
  for (int ss = 0; ss < NSS; ++ss) {
    const int64_t k = k0 + 32 * ss + 8 * kq;
    xf[ss] = bload16(rx, opaque_u32(tok < M && k < k1 ? (uint32_t)((tok * D + k) * 2) : LRQ_OOB));
    if (BWD) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int j = 16 * rt + c16;
        bf[rt][ss] = bload16(rf, opaque_u32(j < r && k < k1 ? (uint32_t)(((int64_t)j * D + k) * 2) : LRQ_OOB));
      }
    }
  }
  if (!BWD) {
    // A [D][r] rows of the slice, 8 ranks per 16-byte run: pair i = tid +
    // 256 q is depth i / JB, ranks 8 (i % JB) ..; zeros past the rank or depth
    constexpr int JB = RP / 8, AQ = JB * FKT / 256;
    u32x4 av[AQ];
#pragma unroll
    for (int qq = 0; qq < AQ; ++qq) {
      const int i = tid + 256 * qq, dd = i / JB, j0 = 8 * (i % JB);
      av[qq] = bload16(rf, opaque_u32(k0 + dd < k1 && j0 < r ? (uint32_t)(((k0 + dd) * r + j0) * 2) : LRQ_OOB));
    }
#pragma unroll
    for (int qq = 0; qq < AQ; ++qq) {
      const int i = tid + 256 * qq, dd = i / JB, j0 = 8 * (i % JB);
      uint16_t* t = lds[j0 >> 4];
#pragma unroll
      for (int e = 0; e < 8; ++e) t[((j0 & 15) + e) * AST + dd] = (uint16_t)(av[qq][e >> 1] >> (16 * (e & 1)));
    }
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int ss = 0; ss < NSS; ++ss)
        bf[rt][ss] = *reinterpret_cast<const u32x4*>(lds[rt] + c16 * AST + 32 * ss + 8 * kq);
  }
  // C element v of lane (c16, kq) in rank tile rt: rank 16 rt + 4 kq + v,
  // token 16 w + c16
  f32x4 acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    acc[rt] = acc_zero4();
#pragma unroll
    for (int ss = 0; ss < NSS; ++ss) acc[rt] = mfma16(as_bf16x8(bf[rt][ss]), as_bf16x8(xf[ss]), acc[rt]);
  }
  const rsrc_t rp = make_rsrc(a.fpart, clamp_bytes((int64_t)fs * Mp * RP * 4));
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
    mstore16_dev(rp, opaque_u32((uint32_t)((((int64_t)sl * Mp + tok) * RP + 16 * rt + 4 * kq) * 4)),
                 __builtin_bit_cast(u32x4, acc[rt]));
  // counted once the partial is acknowledged; the last slice of the group
  // sums the slices in order, stores the factor and publishes the flag
  __builtin_amdgcn_s_waitcnt(0);
  __shared__ int last;
  __syncthreads();
  const int64_t G = (M + 63) / 64;
  if (tid == 0) {
    last = madd_dev(a.fcnt + g) + 1 == (uint32_t)fs;
    if (last) mzero_dev(a.fcnt + g);
  }
  __syncthreads();
  if (!last) return;
  // thread: token g 64 + tid / 4, ranks 16 rt + 4 (tid % 4) ..
  const int64_t tk = (int64_t)g * 64 + (tid >> 2);
  const rsrc_t ro = make_rsrc(a.fout, clamp_bytes(M * a.fout_ld * 2));
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int rq = 16 * rt + 4 * (tid & 3);
    f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < fs; s0 += 8) {
      u32x4 pv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        pv[u] = mbload16_dev(rp, opaque_u32(s0 + u < fs ? (uint32_t)((((int64_t)(s0 + u) * Mp + tk) * RP + rq) * 4) : LRQ_OOB));
#pragma unroll
      for (int u = 0; u < 8; ++u) sum += __builtin_bit_cast(f32x4, pv[u]);
    }
    if (a.fout && tk < M && rq < a.fout_ld) {
      const u32x2 o = {pack_bf16x2(a.fscale * sum[0], a.fscale * sum[1]), pack_bf16x2(a.fscale * sum[2], a.fscale * sum[3])};
      mstore8_dev(ro, opaque_u32((uint32_t)((tk * a.fout_ld + rq) * 2)), o);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) __hip_atomic_store(a.fcnt + G + g, want, __ATOMIC_RELAXED, MXSCOPE);
}

// FOLD: a reader of the ready flags is done with them (a tile after its
// LoRA step, a dA block after its wait). The last of the launch's `readers`
// clears the flags and advances the epoch. Every thread of the workgroup
// calls it.
LRQ_DEV void mid_flags_done(const GemmArgs& a, int readers) {
  __shared__ int fin;
  __syncthreads();
  if (threadIdx.x == 0) fin = madd_dev(a.fcnt + SK_DCNT) + 1 == (uint32_t)readers;
  __syncthreads();
  if (fin) {
    const int64_t G = (a.m + 63) / 64;
    for (int64_t i = threadIdx.x; i < G; i += 256) mzero_dev(a.fcnt + G + i);
    if (threadIdx.x == 0) {
      mzero_dev(a.fcnt + SK_DCNT);
      madd_dev(a.fcnt + SK_EPOCH);
    }
  }
}

// FOLD backward: weight-gradient block tb of the launch's tn jobs (after the
// tiles). A dA block first waits (bounded, as the tiles do) for the ready
// flags of the 64-token groups of its token slice, then reads u at device
// scope; a wait that runs out flags the failure and makes its sums NaN.
// The factor slice goes to sq, the combine buffer to sr (16 KiB each).
LRQ_DEV void mid_tn(const GemmArgs& a, int tb, uint32_t want, int readers, uint16_t* sq, uint16_t* sr) {
  const bool second = tb >= a.tj[0].blocks;
  const int ji = second ? 1 : 0;
  const TnArgs& j = a.tj[ji];
  const int bid = tb - (second ? a.tj[0].blocks : 0);
  float* const red = reinterpret_cast<float*>(sr);
  if (ji != a.tn_da) {
    if (a.rp == 32)
      tn_block<2, MID_TN_LDS, MID_TN_LDS, false>(j, bid, sq, red, false);
    else
      tn_block<1, MID_TN_LDS, MID_TN_LDS, false>(j, bid, sq, red, false);
    return;
  }
  __shared__ int bad;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int64_t G = (a.m + 63) / 64;
    const int64_t m_lo = (int64_t)(bid / j.tiles) * j.m_per;
    const int64_t m_hi = min(j.M, m_lo + j.m_per);
    const int64_t gi = m_lo / 64 + lane;
    const bool mine = gi < (m_hi + 63) / 64 && gi < G;
    uint32_t polls = 0;
    const uint32_t cap = a.fold < 0 ? 16u : MID_MAX_POLLS;  // the test hook: 16 polls
    bool ok = !mine || mload_dev(a.fcnt + G + gi) == want;
    while (!__all(ok) && polls < cap) {
      __builtin_amdgcn_s_sleep(2);
      ++polls;
      ok = !mine || mload_dev(a.fcnt + G + gi) == want;
    }
    if (lane == 0) {
      bad = __all(ok) ? 0 : 1;
      if (!__all(ok)) __hip_atomic_store(a.fcnt + SK_FAIL, 1u, __ATOMIC_RELAXED, MXSCOPE);
    }
  }
  __syncthreads();
  const bool poison = bad != 0;
  mid_flags_done(a, readers);
  if (a.rp == 32)
    tn_block<2, MID_TN_LDS, MID_TN_LDS, true>(j, bid, sq, red, poison);
  else
    tn_block<1, MID_TN_LDS, MID_TN_LDS, true>(j, bid, sq, red, poison);
}

template <bool BWD, int FMT, int TT, int SD, bool FOLD>
__global__ void __launch_bounds__(256, 2) k_mid(GemmArgs a, int tiles_m, int tiles_e, int group_m) {
  constexpr bool I4 = FMT == LRQ_FMT_INT4;
  constexpr bool I8 = FMT == LRQ_FMT_INT8;
  constexpr bool GS = I4 || I8;                    // group scales (int4, int8) or channel scales (fp8)
  // the main loop loads a scale per block unless nothing reads it (the fp8
  // forward applies its channel scales in the epilogue)
  constexpr bool USE_SC = BWD || GS;
  constexpr int T = 16 * TT;                       // tokens per tile
  constexpr int XB = T * MD * SD;                  // bf16 per stage: SD sub-tiles [T][64]
  constexpr int XL = T / 32;                       // activation copies per wavefront per step
  constexpr uint32_t blkb = I4 ? 2048u : 4096u;    // bytes per 64 x 64 block
  constexpr uint32_t rowb = I4 ? 32u : 64u;        // bytes per block row
  __shared__ __attribute__((aligned(16))) uint16_t sx0[XB];
  __shared__ __attribute__((aligned(16))) uint16_t sx1[XB];
  __shared__ __attribute__((aligned(16))) uint16_t sx2[XB];
  __shared__ __attribute__((aligned(16))) uint16_t sx3[XB];

  const int ntiles = tiles_m * tiles_e;
  // depth ranges per tile (msplit > 1: the tile's ranges are consecutive
  // units, the last to finish sums them; see the epilogue)
  const int S = a.msplit > 1 ? a.msplit : 1;
  const int nunits = ntiles * S;
  // FOLD: the launch's stamp, and the factor workgroups ahead of the tiles
  // (the test hook, a.fold < 0, makes the tiles wait for a stamp no
  // launch publishes)
  uint32_t want = 0;
  if (FOLD) {
    const uint32_t stamp = mstamp(mload_dev(a.fcnt + SK_EPOCH));
    if ((int)blockIdx.x < a.fold_wgs) {
      if ((int)blockIdx.x < a.fold_slices * (int)((a.m + 63) / 64)) {
        if (a.rp == 32)
          mid_fold_slice<BWD, 2>(a, (int)blockIdx.x, sx0, sx1, stamp);
        else
          mid_fold_slice<BWD, 1>(a, (int)blockIdx.x, sx0, sx1, stamp);
      }
      return;
    }
    want = stamp + (a.fold < 0 ? 0x40000000u : 0u);
    if constexpr (BWD) {
      if ((int)blockIdx.x >= a.fold_wgs + nunits) {
        static_assert(MID_TN_LDS <= XB * 2, "a weight-gradient block's LDS fits one stage buffer");
        const int nda = a.tn_da >= 0 ? a.tj[a.tn_da].blocks : 0;
        mid_tn(a, (int)blockIdx.x - a.fold_wgs - nunits, want, ntiles + nda, sx0, sx1);
        return;
      }
    }
  }
  const int vb = FOLD ? (int)blockIdx.x - a.fold_wgs : (int)blockIdx.x;
  const int lu = xcd_remap(vb, nunits);
  const int lt = lu / S, sp = lu % S;
  const int per = group_m * tiles_e;
  const int grp = lt / per, within = lt % per;
  const int gm = min(group_m, tiles_m - grp * group_m);
  const int tm = grp * group_m + within % gm, te = within / gm;
  const int64_t M = a.m, D = a.l, E = a.e;
  const int64_t m0 = (int64_t)tm * T, e0 = (int64_t)te * MR;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4, l16 = lane & 15;
  const int64_t KB = (D + 63) / 64;
  const int nk = (int)KB;
  // stages of SD blocks, in whole rounds of MST stages: the whole depth, or
  // range sp's a.mspl stages (a multiple of MST) from stage s0, the last
  // range rounded up past the depth (which reads zeros)
  const int nst = (nk + SD - 1) / SD;
  const int s0 = S > 1 ? sp * a.mspl : 0;
  const int nsp = (S > 1 && sp < S - 1) ? a.mspl : (nst - s0 + MST - 1) / MST * MST;

  // ---- weight: the tile's block row (64 rows = the tile), wavefront w's 16.
  // Each resource ends where this block row's data ends, so a step past the
  // depth reads zeros without a per-lane select.
  const int64_t rb = e0 / 64;
  const rsrc_t rw = make_rsrc(a.wdata + rb * KB * blkb, clamp_bytes(KB * blkb));
  const uint32_t woff = (uint32_t)(16 * w + l16) * rowb + (uint32_t)q * (I4 ? 8u : 16u);
  // forward int4 / int8: group scales [NB][Gp][64], this block row's slab;
  // lane quarter q's group at step kt is (64 kt + 16 q) >> gshift: the
  // step's first group, plus q / 2 for groups of 32
  const uint32_t Gp = (uint32_t)((KB * 64) >> a.gshift);
  // backward int4 / int8: ST [KGt][64 KB], row kg = output row >> gshift
  // (uniform over the wavefront's 16 rows: groups are 32 or more); lane l
  // of each 16-lane row loads the scale of depth 16 (l >> 4) + (l & 15).
  // backward fp8: the channel scale of each depth [n], or a scalar.
  const bool pc = !GS && a.per_channel;
  const int64_t NP = KB * 64;
  rsrc_t rs;
  uint32_t sbase = 0;
  if (!BWD) {
    rs = make_rsrc(a.wscale + (GS ? rb * Gp * 64 : 0), GS ? clamp_bytes((int64_t)Gp * 64 * 4) : 0u);
    sbase = (uint32_t)(16 * w + l16) * 4u + (a.gshift == 5 ? (uint32_t)(q >> 1) * 256u : 0u);
  } else if (GS) {
    rs = make_rsrc(a.wscale + ((e0 + 16 * w) >> a.gshift) * NP, clamp_bytes(NP * 4));
    sbase = (uint32_t)((16 * q + l16) * 4);
  } else {
    rs = make_rsrc(a.wscale, pc ? clamp_bytes(D * 4) : 0u);
    sbase = (uint32_t)((16 * q + l16) * 4);
  }
  const float s0add = (BWD && !GS && !pc) ? a.wscale[0] : 0.0f;

  // ---- activations: wavefront w copies token rows w T/4 .. +T/4; lane l of
  // copy c lands at row w T/4 + 8c + l/8, physical chunk l%8, fetching
  // logical chunk (l%8) ^ mswz(row) = (l%8) ^ ((4c' + l/16) & 7), c' the
  // row's 8-row group (its parity decides the pattern). A chunk at or past
  // the depth reads zeros: lim = D - 8 lc bounds the step's start (it also
  // ends the steps past the last block).
  const rsrc_t rx = make_rsrc(a.act + (m0 < M ? m0 : 0) * D, m0 < M ? clamp_bytes((M - m0) * D * 2) : 0u);
  const int xr0 = w * (T / 4);
  const int lc0 = (lane & 7) ^ ((lane >> 4) & 7), lc1 = (lane & 7) ^ (((lane >> 4) + 4) & 7);
  const uint32_t xo0 = (uint32_t)(((xr0 + (lane >> 3)) * D + lc0 * 8) * 2);
  const uint32_t xo1 = (uint32_t)(((xr0 + (lane >> 3)) * D + lc1 * 8) * 2);
  const int lim0 = (int)D - 8 * lc0, lim1 = (int)D - 8 * lc1;
  auto dma = [&](uint16_t* buf, int kt) {
    const int k0 = (kt + s0 * SD) * MD;
    const bool ok0 = k0 < lim0, ok1 = k0 < lim1;
    const uint32_t ko = (uint32_t)(k0 * 2);
    __attribute__((address_space(3))) char* base =
        (__attribute__((address_space(3))) char*)(lds_void*)(buf + xr0 * MD);
    const uint32_t o0 = opaque_u32(xo0) + ko, o1 = opaque_u32(xo1) + ko;
#pragma unroll
    for (int c = 0; c < XL; ++c) {
      // the row group of copy c is xr0/8 + c: xr0/8 is even (T/4 is a
      // multiple of 16), so its parity is c's
      const bool ok = (c & 1) ? ok1 : ok0;
      const uint32_t off = opaque_u32(ok ? ((c & 1) ? o1 : o0) + (uint32_t)(c * 8 * D * 2) : LRQ_OOB);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void*)(base + c * 8 * MD * 2), 16, off, 0, 0, 0);
    }
  };
  // B-role fragment of token tile j, sub-step kk: row 16j + l16, logical
  // chunk 2q + kk at physical chunk (2q + kk) ^ mswz(l16) (mswz(16j + l16) =
  // mswz(l16)); the tile offset is an immediate of the LDS read
  uint32_t xf[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
    xf[kk] = opaque_u32((uint32_t)((l16 * MD + (((2 * q + kk) ^ mswz(l16)) * 8)) * 2));
  auto xfrag = [&](const uint16_t* buf, int j, int kk) -> bf16x8 {
    return as_bf16x8(ld16(reinterpret_cast<const char*>(buf) + xf[kk] + (uint32_t)(j * 16 * MD * 2)));
  };

  // ---- weights: per stage and block the packed bytes and one scale, in
  // register sets; loaded one stage ahead of the activations, so a step can
  // dequantize the next stage while its matrix-core steps run
  u32x4 wv[MST][SD];
  float sv[MST][SD] = {};
  auto load_w = [&](int set, int st) {
#pragma unroll
    for (int d = 0; d < SD; ++d) {
      const uint32_t kt = (uint32_t)((st + s0) * SD + d);
      if (I4) {
        const u32x2 v = bload8(rw, opaque_u32(woff + kt * blkb));
        wv[set][d] = (u32x4){v[0], v[1], 0u, 0u};
      } else {
        wv[set][d] = bload16(rw, opaque_u32(woff + kt * blkb));
      }
      if (USE_SC) {
        const uint32_t so = !BWD ? ((kt * 64u) >> a.gshift) * 256u : kt * 256u;
        sv[set][d] = bloadf(rs, opaque_u32(sbase + so));
      }
    }
  };
  // A-role fragment of block d, sub-step kk from register set `set`
  auto wfrag = [&](int set, int d, int kk) -> bf16x8 {
    const u32x4 v = wv[set][d];
    const float sc = sv[set][d];
    if (!BWD) {
      if (I4) return as_bf16x8(dequant8_int4_bf16(v[kk], sc, a.nib));
      if (I8) return as_bf16x8(dequant8_int8_bf16((u32x2){v[2 * kk], v[2 * kk + 1]}, sc));
      const u32x2 lo = fp8x4_to_bf16(v[2 * kk]), hi = fp8x4_to_bf16(v[2 * kk + 1]);
      return as_bf16x8((u32x4){lo[0], lo[1], hi[0], hi[1]});
    }
    float f[8];
    if (I4) {
      int4x8_to_f32_div16(v[kk], f);  // q / 16, times 16 x the scale below
    } else if (I8) {
      int8x4_to_f32(v[2 * kk], f);
      int8x4_to_f32(v[2 * kk + 1], f + 4);
    } else {
      fp8x4_to_f32(v[2 * kk], f);
      fp8x4_to_f32(v[2 * kk + 1], f + 4);
    }
    const float S = I4 ? 16.0f * sc : sc + s0add;
    mul_row_bcast8(f, S, kk);
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
    return as_bf16x8(o);
  };

  f32x4 acc[TT];
#pragma unroll
  for (int j = 0; j < TT; ++j) acc[j] = acc_zero4();

  uint16_t* const bufs[MST] = {sx0, sx1, sx2, sx3};
  // A fragments of the current and the next stage
  bf16x8 fa[2][SD][2];
  // per-lane memory instructions of one stage: per block the activation
  // copies, the weight bytes and (USE_SC) the scale. The waits below count
  // them, so this must be exactly what a stage issues: a count one too high
  // lets a stage's last activation copy (8 token rows) still be in flight
  // when the fragment reads start
  constexpr int NST = SD * (XL + 1 + (USE_SC ? 1 : 0));
  // Stage st: activations in bufs[st % MST] (issued MST - 1 stages ahead),
  // weights in register set st % MST (MST stages ahead), A fragments in
  // fa[st % 2] (dequantized during stage st - 1).
  auto step = [&](const int b, const int st) {
    // nothing of one step moves into another
    __builtin_amdgcn_sched_barrier(0);
    // stage st's copies and stage st + 1's weights have landed (issued in
    // that order, then MST - 2 more stages); the newer ones may be in flight
    __builtin_amdgcn_s_waitcnt((((MST - 2) * NST) & 0xf) | ((((MST - 2) * NST) >> 4) << 14) | 0xf70);
    // a barrier without a memory fence: a fence would wait for every copy
    // in flight (the newer stages too). Each wavefront's own wait above
    // covers its copies of this stage, and the fragment reads of the last
    // step were consumed by its matrix-core steps before this point.
    __builtin_amdgcn_s_barrier();
    // every wavefront is done with the buffer of stage st - 1: refill it;
    // register set b (stage st's weights, dequantized last step) takes
    // stage st + MST's
    const int nb = (b + MST - 1) % MST;
#pragma unroll
    for (int d = 0; d < SD; ++d) dma(bufs[nb] + d * T * MD, (st + MST - 1) * SD + d);
    load_w(b, st + MST);
    __builtin_amdgcn_sched_barrier(0);
    const int cur = b & 1, nxt = cur ^ 1;
#pragma unroll
    for (int d = 0; d < SD; ++d)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
#pragma unroll
        for (int j = 0; j < TT; ++j) acc[j] = mfma16(fa[cur][d][kk], xfrag(bufs[b] + d * T * MD, j, kk), acc[j]);
        // the next stage's fragment, between this stage's matrix-core steps
        fa[nxt][d][kk] = wfrag((b + 1) % MST, d, kk);
      }
  };

  // FOLD: the weight-side factor rows of the LoRA step, fetched first (row
  // e0 + 16w + l16; ranks 8q .. + 8, up to the rank): forward B [r][E] across its
  // rows, backward A [E][r] as stored
  const int64_t frow = e0 + 16 * w + l16;
  u32x4 fla = zero4();
  if (FOLD) {
    const int fr_r = a.r;
    if (!BWD) {
      const rsrc_t rb = make_rsrc(a.lw, clamp_bytes((int64_t)fr_r * E * 2));
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const int j = 8 * q + e;
        const uint32_t lo = bload2(rb, opaque_u32(j < fr_r && frow < E ? (uint32_t)((j * E + frow) * 2) : LRQ_OOB));
        const uint32_t hi =
            bload2(rb, opaque_u32(j + 1 < fr_r && frow < E ? (uint32_t)(((j + 1) * E + frow) * 2) : LRQ_OOB));
        fla[e >> 1] = lo | (hi << 16);
      }
    } else {
      const rsrc_t ra = make_rsrc(a.lw, clamp_bytes(E * fr_r * 2));
      fla = bload16(ra, opaque_u32(8 * q < fr_r && frow < E ? (uint32_t)((frow * fr_r + 8 * q) * 2) : LRQ_OOB));
    }
  }
  // prologue: stage 0's weights, then stages 0 .. MST-2 of activations
  // each followed by the next stage's weights; stage 0 dequantized
  load_w(0, 0);
#pragma unroll
  for (int s = 0; s < MST - 1; ++s) {
#pragma unroll
    for (int d = 0; d < SD; ++d) dma(bufs[s] + d * T * MD, s * SD + d);
    load_w(s + 1, s + 1);
  }
  __builtin_amdgcn_s_waitcnt((((MST - 1) * NST) & 0xf) | ((((MST - 1) * NST) >> 4) << 14) | 0xf70);
#pragma unroll
  for (int d = 0; d < SD; ++d)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) fa[0][d][kk] = wfrag(0, d, kk);
  for (int st = 0; st < nsp; st += MST) {
#pragma unroll
    for (int b = 0; b < MST; ++b) step(b, st + b);
  }
  // the look-ahead copies past the depth read nothing (out of range), but
  // they are still in flight: drain them before LDS is released
  __builtin_amdgcn_s_waitcnt(0);

  // ---- depth ranges: every range stores its accumulators (f32, in their
  // own layout: unit (lt, range), token tile j, thread) at device scope and
  // counts itself at its tile once they are acknowledged; the last to
  // arrive sums the ranges in order (its own from registers) and goes on
  // with the epilogue, the others are done
  if (S > 1) {
    const int64_t pbytes = (int64_t)nunits * TT * 256 * 16;
    const rsrc_t rpp = make_rsrc(a.part, clamp_bytes(pbytes));
    auto poff = [&](int r, int j) { return (uint32_t)(((((int64_t)lt * S + r) * TT + j) * 256 + tid) * 16); };
#pragma unroll
    for (int j = 0; j < TT; ++j) mstore16_dev(rpp, opaque_u32(poff(sp, j)), __builtin_bit_cast(u32x4, acc[j]));
    __builtin_amdgcn_s_waitcnt(0);
    __shared__ int last_range;
    __syncthreads();
    if (tid == 0) {
      last_range = madd_dev(a.mcnt + lt) + 1 == (uint32_t)S;
      if (last_range) mzero_dev(a.mcnt + lt);
    }
    __syncthreads();
    if (!last_range) return;
    u32x4 pr[MID_MAX_SPLIT][TT];
#pragma unroll
    for (int r = 0; r < MID_MAX_SPLIT; ++r)
#pragma unroll
      for (int j = 0; j < TT; ++j) pr[r][j] = mbload16_dev(rpp, opaque_u32(r < S && r != sp ? poff(r, j) : LRQ_OOB));
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      f32x4 sum = sp == 0 ? acc[j] : __builtin_bit_cast(f32x4, pr[0][j]);
#pragma unroll
      for (int r = 1; r < MID_MAX_SPLIT; ++r)
        if (r < S) sum += r == sp ? acc[j] : __builtin_bit_cast(f32x4, pr[r][j]);
      acc[j] = sum;
    }
  }

  // ---- epilogue
  const int rp = a.rp;
  if (FOLD) {
    // wait for the token-side factor of the tile's 64-token groups (lane
    // i < T / 64 of wavefront 0 polls group m0 / 64 + i), bounded
    __shared__ int fold_bad;
    const int64_t G = (M + 63) / 64;
    if (w == 0) {
      const int64_t gi = m0 / 64 + lane;
      const bool mine = lane < T / 64 && gi < G;
      uint32_t polls = 0;
      const uint32_t cap = a.fold < 0 ? 16u : MID_MAX_POLLS;  // the test hook: 16 polls
      bool ok = !mine || mload_dev(a.fcnt + G + gi) == want;
      while (!__all(ok) && polls < cap) {
        __builtin_amdgcn_s_sleep(2);
        ++polls;
        ok = !mine || mload_dev(a.fcnt + G + gi) == want;
      }
      if (lane == 0) {
        fold_bad = __all(ok) ? 0 : 1;
        if (!__all(ok)) __hip_atomic_store(a.fcnt + SK_FAIL, 1u, __ATOMIC_RELAXED, MXSCOPE);
      }
    }
    __syncthreads();
    // the LoRA step: weight-side rows (A role) from the prefetched factor,
    // the tile's factor rows (B role) read past the L2s; forward fp8 rows
    // divided by the weight scale the epilogue multiplies by
    u32x4 la = fla;
    if (!BWD && !GS) {
      const float dv = a.per_channel ? (frow < E ? a.wscale[frow] : 1.0f) : a.wscale[0];
#pragma unroll
      for (int h = 0; h < 4; ++h)
        la[h] = (uint32_t)f32_to_bf16_bits(bf16_lo(la[h]) / dv) | ((uint32_t)f32_to_bf16_bits(bf16_hi(la[h]) / dv) << 16);
    }
    const rsrc_t rfo = make_rsrc(a.fout + (m0 < M ? m0 : 0) * a.fout_ld, m0 < M ? clamp_bytes((M - m0) * a.fout_ld * 2) : 0u);
    const bool bad = fold_bad != 0;
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      u32x4 lb = mbload16_dev(rfo, opaque_u32(8 * q < a.fout_ld ? (uint32_t)(((16 * j + l16) * a.fout_ld + 8 * q) * 2) : LRQ_OOB));
      if (bad) lb = (u32x4){0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u};
      acc[j] = mfma16(as_bf16x8(la), as_bf16x8(lb), acc[j]);
    }
  } else if (rp > 0) {
    // LoRA: A role = weight-side rows e0 + 16w + l16 (B^T forward, A
    // backward, [E][rp]), B role = token rows m0 + 16j + l16 (t or u,
    // [M][rp]); rank slots 32 ks + 8q .. +8, zero past rp
    const rsrc_t rfr = make_rsrc(a.lw + (e0 + 16 * w) * rp,
                                 e0 + 16 * w < E ? clamp_bytes((E - e0 - 16 * w) * rp * 2) : 0u);
    const rsrc_t rt = make_rsrc(a.lact + (m0 < M ? m0 : 0) * rp, m0 < M ? clamp_bytes((M - m0) * rp * 2) : 0u);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if (ks * 32 < rp) {
        const bool ok = 32 * ks + 8 * q < rp;
        const bf16x8 la = as_bf16x8(bload16(rfr, opaque_u32(ok ? (uint32_t)((l16 * rp + 32 * ks + 8 * q) * 2) : LRQ_OOB)));
#pragma unroll
        for (int j = 0; j < TT; ++j) {
          const bf16x8 lb = as_bf16x8(
              bload16(rt, opaque_u32(ok ? (uint32_t)(((16 * j + l16) * rp + 32 * ks + 8 * q) * 2) : LRQ_OOB)));
          acc[j] = mfma16(la, lb, acc[j]);
        }
      }
    }
  }
  // lane: output rows (columns of y / dx) n = e0 + 16w + 4q + v, v = 0..3,
  // token m0 + 16j + l16
  const int64_t n = e0 + 16 * w + 4 * q;
  const bool nok = n < E;  // E % 8 == 0: the four are in or out together
  f32x4 sc = {1.f, 1.f, 1.f, 1.f}, bv = {0.f, 0.f, 0.f, 0.f};
  if (!BWD) {
    if (!GS) {
      if (pc) {
        const rsrc_t rsc = make_rsrc(a.wscale, clamp_bytes(E * 4));
        const u32x4 s4 = bload16(rsc, opaque_u32(nok ? (uint32_t)(n * 4) : LRQ_OOB));
        sc = (f32x4){__uint_as_float(s4[0]), __uint_as_float(s4[1]), __uint_as_float(s4[2]), __uint_as_float(s4[3])};
      } else {
        const float s0 = a.wscale[0];
        sc = (f32x4){s0, s0, s0, s0};
      }
    }
    if (a.bias) {
      const rsrc_t rbi = make_rsrc(a.bias, clamp_bytes(E * 4));
      const u32x4 b4 = bload16(rbi, opaque_u32(nok ? (uint32_t)(n * 4) : LRQ_OOB));
      bv = (f32x4){__uint_as_float(b4[0]), __uint_as_float(b4[1]), __uint_as_float(b4[2]), __uint_as_float(b4[3])};
    }
  }
  const rsrc_t ry = make_rsrc(a.out + (m0 < M ? m0 : 0) * E, m0 < M ? clamp_bytes((M - m0) * E * 2) : 0u);
#pragma unroll
  for (int j = 0; j < TT; ++j) {
    const f32x4 c = acc[j];
    u32x2 o;
    o[0] = pack_bf16x2(__builtin_fmaf(c[0], sc[0], bv[0]), __builtin_fmaf(c[1], sc[1], bv[1]));
    o[1] = pack_bf16x2(__builtin_fmaf(c[2], sc[2], bv[2]), __builtin_fmaf(c[3], sc[3], bv[3]));
    const uint32_t off = nok ? (uint32_t)(((16 * j + l16) * E + n) * 2) : LRQ_OOB;
    __builtin_amdgcn_raw_buffer_store_b64(o, ry, opaque_u32(off), 0, 2);  // non-temporal, as the large tiles' output
  }
  if (FOLD) mid_flags_done(a, ntiles + ((BWD && a.tn_da >= 0) ? a.tj[a.tn_da].blocks : 0));
}

template <bool BWD, int FMT>
hipError_t run_mid(hipStream_t st, const GemmArgs& a, int variant) {
  const int T = variant == MID_64 ? 64 : 128;
  const int tiles_m = (int)((a.m + T - 1) / T);
  const int tiles_e = (int)((a.e + MR - 1) / MR);
  const int group_m = tiles_m < 8 ? tiles_m : 8;
  const int ntiles = tiles_m * tiles_e;
  const int S = a.msplit > 1 ? a.msplit : 1;
  // k_mid: two 64-wide blocks per stage with 64-token tiles, one with 128;
  // 64 KiB of LDS in every variant, two workgroups per CU; S units per tile
  // with depth ranges; with the fold, its workgroups first
  if (a.fold) {
    const unsigned grid = (unsigned)(ntiles * S + a.fold_wgs + (BWD ? a.tn_blocks : 0));
    if (variant == MID_128)
      hipLaunchKernelGGL((k_mid<BWD, FMT, 8, 1, true>), dim3(grid), dim3(256), 0, st, a, tiles_m, tiles_e, group_m);
    else
      hipLaunchKernelGGL((k_mid<BWD, FMT, 4, 2, true>), dim3(grid), dim3(256), 0, st, a, tiles_m, tiles_e, group_m);
  } else if (variant == MID_128) {
    hipLaunchKernelGGL((k_mid<BWD, FMT, 8, 1, false>), dim3(ntiles * S), dim3(256), 0, st, a, tiles_m, tiles_e, group_m);
  } else {
    hipLaunchKernelGGL((k_mid<BWD, FMT, 4, 2, false>), dim3(ntiles * S), dim3(256), 0, st, a, tiles_m, tiles_e, group_m);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_mid(hipStream_t st, int fmt, bool bwd, const GemmArgs& a, int variant) {
  if (a.m <= 0 || a.e <= 0) return hipSuccess;
  if (variant != MID_64 && variant != MID_128) return hipErrorInvalidValue;
  if (a.rp > 64 || a.rp % 16 != 0) return hipErrorInvalidValue;
  // depth ranges: at most MID_MAX_SPLIT, each whole rounds of stages, the
  // last one non-empty; partials for every unit and a counter per tile
  const int T = variant == MID_64 ? 64 : 128, SDv = variant == MID_64 ? 2 : 1;
  const int64_t ntiles = (a.m + T - 1) / T * ((a.e + MR - 1) / MR);
  const int S = a.msplit > 1 ? a.msplit : 1;
  if (S > 1) {
    const int64_t nst = ((a.l + 63) / 64 + SDv - 1) / SDv;
    if (S > MID_MAX_SPLIT || a.mspl <= 0 || a.mspl % MST != 0 || (int64_t)(S - 1) * a.mspl >= nst ||
        (int64_t)S * a.mspl < nst || !a.part || !a.mcnt ||
        (int64_t)S * ntiles * T * 64 * 4 >= ((int64_t)1 << 32))
      return hipErrorInvalidValue;
  }
  // the fold: ranks 8 to 32 (multiples of 8, padded to 16 or 32), both raw factors, its output, partials and
  // counters (groups' arrivals and flags within the counter area), and
  // enough factor workgroups, whole groups of eight
  if (a.fold) {
    const int64_t G = (a.m + 63) / 64;
    if ((a.rp != 16 && a.rp != 32) || a.r % 8 != 0 || a.r > a.rp || a.r <= a.rp - 16 || !a.lact || !a.lw ||
        !a.fout || a.fout_ld % 8 != 0 || a.fout_ld < a.r || a.fout_ld > a.rp || !a.fpart || !a.fcnt ||
        2 * G > SK_MAX_NB || a.fold_wgs % 8 != 0 ||
        a.fold_slices != (int)((a.l + MID_FOLD_KT - 1) / MID_FOLD_KT) || a.fold_wgs < a.fold_slices * G ||
        a.m * a.l * 2 >= ((int64_t)1 << 32) || a.m * a.fout_ld * 2 >= ((int64_t)1 << 32) ||
        (int64_t)a.fold_slices * G * 64 * a.rp * 4 >= ((int64_t)1 << 32))
      return hipErrorInvalidValue;
    // the weight gradients' jobs after the tiles (backward): each a whole
    // plan of token slices that fit MID_TN_LDS, over all the launch's
    // tokens, with its counters past the fold's and apart from the other's
    if (a.tn_blocks != 0) {
      if (!bwd || a.tn_blocks < 0 || a.tj[0].blocks + a.tj[1].blocks != a.tn_blocks || a.tn_da < -1 ||
          a.tn_da > 1 || (a.tn_da >= 0 && a.tj[a.tn_da].blocks == 0))
        return hipErrorInvalidValue;
      const uint32_t* lo = a.fcnt + 2 * G;
      if (S > 1 && a.mcnt + ntiles > lo) lo = a.mcnt + ntiles;
      for (int i = 0; i < 2; ++i) {
        const TnArgs& j = a.tj[i];
        if (j.blocks == 0) continue;
        if (j.C <= 0 || j.tiles != (j.C + 127) / 128 || j.splits < 1 || j.blocks != j.tiles * j.splits ||
            j.m_per <= 0 || j.m_per % 128 != 0 || a.rp * (j.m_per + 8) * 2 > MID_TN_LDS || j.M != a.m ||
            (int64_t)j.splits * j.m_per < j.M || (int64_t)(j.splits - 1) * j.m_per >= j.M || !j.p || !j.q ||
            !j.out || j.R < 1 || j.R > a.rp || j.ldq < j.R || (j.splits > 1 && !j.partial) || !j.cnt ||
            j.cnt < lo || j.cnt + TN_WAVES * j.tiles > a.fcnt + SK_MAX_NB ||
            j.m_per * j.C * 2 >= ((int64_t)1 << 31) || (int64_t)j.splits * j.C * a.rp * 4 >= ((int64_t)1 << 32))
          return hipErrorInvalidValue;
        if (i == a.tn_da && (j.ldq % 8 != 0 || (reinterpret_cast<uintptr_t>(j.q) & 15) != 0))
          return hipErrorInvalidValue;
        lo = j.cnt + TN_WAVES * j.tiles;
      }
    }
    // the tiles' range counters past the fold's
    if (S > 1 && (a.mcnt < a.fcnt + 2 * G || a.mcnt + ntiles > a.fcnt + SK_MAX_NB)) return hipErrorInvalidValue;
  } else if (a.tn_blocks != 0) {
    return hipErrorInvalidValue;
  }
  // 32-bit buffer offsets: one tile's activation rows and outputs, the depth
  // run of the weight's block row
  if ((int64_t)128 * a.l * 2 >= ((int64_t)1 << 31) || (int64_t)128 * a.e * 2 >= ((int64_t)1 << 31))
    return hipErrorInvalidValue;
  if (fmt == LRQ_FMT_INT4)
    return bwd ? run_mid<true, LRQ_FMT_INT4>(st, a, variant) : run_mid<false, LRQ_FMT_INT4>(st, a, variant);
  if (fmt == LRQ_FMT_INT8)
    return bwd ? run_mid<true, LRQ_FMT_INT8>(st, a, variant) : run_mid<false, LRQ_FMT_INT8>(st, a, variant);
  return bwd ? run_mid<true, LRQ_FMT_FP8>(st, a, variant) : run_mid<false, LRQ_FMT_FP8>(st, a, variant);
}
