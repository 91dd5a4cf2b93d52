// Input gradient of the quantized LoRA linear on gfx950 matrix cores:
//
//   dx[m, k] = dy[m, n] . bf16(dq(w))[n, k]  +  u[m, :] . A[k, :]^T
//
// (src/quant.rs:229-233 for the base product; the LoRA term is the autodiff
// of src/lora.rs:199-203, with u = s.dy.B^T computed by the skinny kernels.)
//
// A workgroup owns an RA x 256 output tile (RA k rows, 256 tokens in 4 token
// groups of 64). Each token group is served by WN wavefronts that split the
// RA rows; WN = 2 puts two wavefronts on each SIMD, so one's dequantization
// and LDS traffic overlap the other's matrix-core work:
//   - the reduction runs along n while the packed weight rows are contiguous
//     along k, so each thread reads a BN x 8 block of packed weights (BN
//     rows n, 8 columns k) from HBM/L2, dequantizes it in registers and
//     writes it transposed into a double-buffered LDS tile of bf16 [k][n];
//     a bf16 copy of the weight never exists in HBM;
//   - dy is copied global -> LDS by buffer loads with an LDS destination (no
//     register round trip), one reduction step ahead; each wavefront moves
//     and reads only its own 64 tokens, in XOR-swizzled 16-byte chunks;
//   - v_mfma_f32_32x32x16_bf16 with the weight as the A-role operand, so the
//     accumulators hold 4 consecutive k of one token and the epilogue writes
//     8-byte runs. The reduction index is permuted inside a step (lane group
//     g takes n = 32g + 8kk .. +8 in sub-step kk) so each lane's dy bytes are
//     64 contiguous bytes;
//   - the loop is unrolled by two steps so every buffer index is static and
//     the whole step is one basic block: buffer loads past a resource's size
//     return zeros, so edges need no branches (buffer descriptors are forced
//     scalar and selected offsets made opaque so the compiler cannot
//     reintroduce branches), the next tile's dequantization is interleaved
//     with the current tile's matrix-core work, and one barrier ends a step;
//   - the LoRA term is one more rank-wide step after the main loop (A staged
//     through LDS, u from global);
//   - int4 group scales vary along k, so each row of the 8 x BN block has its
//     own scale, applied during dequantization (fma(u, s, -8s) == q*s exactly);
//   - workgroup ids are remapped so each XCD (own L2) works on a contiguous
//     range of tiles.

#include "lrq_common.h"
#include "lrq_kernels.h"

namespace {

constexpr int BK = 64;      // reduction step
// LDS layouts (gfx950 LDS: 64 banks x 4 bytes; a 16-byte access serves 16
// lanes per pass, so each group of 16 lanes must cover distinct banks):
//   activation tile [rows][64] bf16, 128-byte rows (the buffer-load DMA
//     writes whole rows), 16-byte chunk c of row r stored at chunk
//     c ^ ((r >> 1) & 7);
//   weight tiles: 144-byte rows (8 bf16 of padding), no swizzle; 16
//     consecutive rows then cover all 64 banks, and every writer and reader
//     is mapped so that 16 consecutive lanes touch 16 consecutive rows at one
//     chunk, or (backward transposed writes) 8 lanes fill one whole row.
constexpr int LD = BK + 8;  // weight-tile row stride (bf16)
LRQ_DEV int swz(int r) { return (r >> 1) & 7; }
constexpr int MJ = 2;       // 32-token tiles per wavefront
constexpr int RB = 4 * 32 * MJ;  // tokens per workgroup (4 token groups of 64)

// WN wavefronts share each token group, splitting its RA k rows: WN = 2
// gives 8 wavefronts (two per SIMD) with half the accumulators each.
template <int FMT, int NI, int WN>
struct Cfg {
  static constexpr int NT = 256 * WN;  // threads per workgroup
  static constexpr int NIW = NI / WN;  // 32-row tiles per wavefront
  static constexpr int RA = 32 * NI;  // a multiple of 64 (whole weight blocks)
  // one BN (n) x 8 (k) block per thread; RA/8 k-chunks x 64/BN n-chunks
  // (BN = 4 with 8 wavefronts keeps 32 values per thread)
  static constexpr int KCH = RA / 8;
  static constexpr int BN = (WN == 2) ? 4 : 8;
  static constexpr int NCH = 64 / BN;
  static constexpr int WORDS = (FMT == LRQ_FMT_INT4) ? 1 : 2;  // dwords per 8 k of one row
  static constexpr int WBUF = RA * LD;                          // weight tile (bf16)
  static constexpr int XBUF = RB * BK;                          // activation tile (bf16)
  static constexpr int LDS_ELEMS = 2 * WBUF + 2 * XBUF + NT * 8;
  static_assert(NI % WN == 0, "whole row tiles per wavefront");
};

template <int FMT, int NI, int WN>
__global__ void __launch_bounds__(256 * WN) __attribute__((amdgpu_waves_per_eu(WN, WN)))
k_dx(GemmArgs a, int tiles_m) {
  using C = Cfg<FMT, NI, WN>;
  constexpr int RA = C::RA, NT = C::NT, NIW = C::NIW;
  __shared__ __attribute__((aligned(16))) uint16_t lds[C::LDS_ELEMS];
  uint16_t* const sW = lds;                     // [2][RA][LD]
  uint16_t* const sX = lds + 2 * C::WBUF;       // [2][256][64], 16-byte chunks XOR-swizzled by row
  uint16_t* const sDummy = sX + 2 * C::XBUF;    // per-thread slots for idle threads

  // XCD-contiguous logical order, then groups of GM token tiles walked
  // weight-tile by weight-tile: the 32 concurrent workgroups of an XCD cover
  // a GM x 8 block, so activation and weight slices are shared in its L2
  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int tiles_a = gridDim.x / tiles_m;
  constexpr int GM = 4;
  const int grp = logical / (GM * tiles_a), within = logical % (GM * tiles_a);
  const int gm = min(GM, tiles_m - grp * GM);
  const int tm = grp * GM + within % gm, ta = within / gm;
  const int64_t m0 = (int64_t)tm * RB, e0 = (int64_t)ta * RA;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t M = a.m, L = a.l, E = a.e, K = a.wk;
  const int g = lane >> 5, l32 = lane & 31;
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const int tw = wv & 3, rh = wv >> 2;  // token group, weight-row part

  // ---------------- dy: DMA into LDS, one reduction step ahead
  // The WN wavefronts of token group tw move its 64 token rows (8 KB per
  // step) with 8 buffer loads, 8/WN each, whose lanes cover 8 rows x 128
  // contiguous bytes each; lane l of load c lands at row c*8 + l/8, physical
  // chunk l%8, and fetches logical chunk (l%8) ^ swz(row). Rows past M read
  // zeros through the resource size.
  const int64_t mw = m0 + tw * (32 * MJ);
  const int64_t mrows = (M - mw) < (32 * MJ) ? (M - mw) : (32 * MJ);
  const rsrc_t ract = make_rsrc(a.act + (mw < M ? mw : 0) * L, clamp_bytes(mrows * L * 2));
  // (l%8) ^ swz(c*8 + l/8); swz(c*8 + l/8) = (4c + l/16) & 7 alternates with
  // the parity of c, so two offsets cover all eight loads.
  const int drow = lane >> 3;
  const int dq0 = (lane & 7) ^ ((lane >> 4) & 7), dq1 = (lane & 7) ^ (((lane >> 4) + 4) & 7);
  const uint32_t doff0 = (uint32_t)((drow * L + dq0 * 8) * 2), doff1 = (uint32_t)((drow * L + dq1 * 8) * 2);
  auto dma_act = [&](int buf, int64_t k0) {
    const bool kok0 = k0 + dq0 * 8 < L, kok1 = k0 + dq1 * 8 < L;  // L % 8 == 0
    const uint32_t koff = (uint32_t)(k0 * 2);
    lds_void* base = (lds_void*)(sX + buf * C::XBUF + tw * (32 * MJ) * BK);
#pragma unroll
    for (int cc = 0; cc < 4 * MJ / WN; ++cc) {
      const int c = rh * (4 * MJ / WN) + cc;
      const bool kok = (c & 1) ? kok1 : kok0;
      const uint32_t doff = (c & 1) ? doff1 : doff0;
      const uint32_t off = opaque_u32(kok ? doff + (uint32_t)(c * 8 * L * 2) + koff : LRQ_OOB);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ract, (lds_void*)((__attribute__((address_space(3))) char*)base + c * 8 * BK * 2),
                                               16, off, 0, 0, 0);
    }
  };
  // fragment of wave-local row j*32 + l32, logical chunk q: byte offset
  // (row * 128) ^ ((q ^ swz(l32)) * 16); swz(j*32 + l32) = swz(l32). The XOR
  // is done per read from an opaque base so the eight chunk addresses are not
  // all kept live in registers.
  const uint32_t xrow = (uint32_t)((tw * (32 * MJ) + l32) * BK * 2) | (uint32_t)(swz(l32) * 16);
  auto bfrag = [&](int buf, int j, int q) -> bf16x8 {
    const uint32_t off = (opaque_u32(xrow) ^ (uint32_t)(q * 16)) + (uint32_t)((buf * C::XBUF + j * 32 * BK) * 2);
    return as_bf16x8(ld16(reinterpret_cast<const char*>(sX) + off));
  };

  // ---------------- weight operand (blocked layout): packed loads, two register sets
  const int64_t KB = (K + 63) / 64;
  const uint32_t blkb = (FMT == LRQ_FMT_INT4) ? 2048u : 4096u;  // bytes per 64x64 block
  const uint32_t rowb = (FMT == LRQ_FMT_INT4) ? 32u : 64u;      // bytes per block row
  const uint32_t Gp = (FMT == LRQ_FMT_INT4) ? (uint32_t)((KB * 64) >> a.gshift) : 0u;
  int64_t wbytes, nsc;
  blocked_sizes_dev(FMT, L, K, &wbytes, &nsc, a.gshift);
  const rsrc_t rw = make_rsrc(a.wdata, clamp_bytes(wbytes));
  const rsrc_t rs = (FMT == LRQ_FMT_INT4) ? make_rsrc(a.wscale, clamp_bytes(nsc * 4))
                                          : make_rsrc(a.wscale, a.per_channel ? clamp_bytes(L * 4) : 4u);

  // thread mapping: nc = tid % NCH (BN n), kc = (tid / NCH) % KCH (8 k), so
  // the NCH lanes of one k-row group write one whole 128-byte tile row;
  // threads past NCH*KCH redo a block and write it to a private dummy slot
  const bool wthr_ok = tid < C::NCH * C::KCH;
  const int bnc = tid % C::NCH;
  const int bkc = (tid / C::NCH) % C::KCH;
  const int64_t bcol = e0 + bkc * 8;
  const bool bcol_ok = bcol < KB * 64;  // columns in [K, 64*KB) are zero padding
  const uint32_t bcolbyte = bcol_ok ? (uint32_t)((bcol >> 6) * blkb + ((FMT == LRQ_FMT_INT4) ? (bcol & 63) / 2 : (bcol & 63)))
                                    : LRQ_OOB;
  const uint32_t bscol = bcol_ok ? ((FMT == LRQ_FMT_INT4) ? (uint32_t)(bcol >> a.gshift) * 64u * 4u : 0u) : LRQ_OOB;

  // fp8: per-channel scale offsets, or the one scalar scale (loop invariant)
  const uint32_t fp8_pc_off = (a.per_channel && bcol_ok) ? 0u : LRQ_OOB;
  const float fp8_scalar = (FMT == LRQ_FMT_FP8 && !a.per_channel) ? bloadf(rs, bcol_ok ? 0u : LRQ_OOB) : 0.0f;

  uint32_t wb[2][C::BN * C::WORDS];  // BN rows x 8 k, packed
  float wbs[2][C::BN];               // row scales

  auto load_w = [&](int set, int kt) {
    // rows n = kt*64 + nc*BN + i: block row kt, in-block rows nc*BN + i
    const uint32_t rbase = (uint32_t)kt * (uint32_t)KB * blkb + (uint32_t)(bnc * C::BN) * rowb + bcolbyte;
#pragma unroll
    for (int i = 0; i < C::BN; ++i) {
      if (FMT == LRQ_FMT_INT4) {
        wb[set][i] = bload4(rw, rbase + (uint32_t)i * rowb);
      } else {
        const u32x2 v = bload8(rw, rbase + (uint32_t)i * rowb);
        wb[set][2 * i] = v[0];
        wb[set][2 * i + 1] = v[1];
      }
    }
    if (FMT == LRQ_FMT_INT4) {
      const uint32_t soff = ((uint32_t)kt * Gp * 64u + (uint32_t)(bnc * C::BN)) * 4u + bscol;
#pragma unroll
      for (int h = 0; h < C::BN / 4; ++h) {
        const u32x4 sv = bload16(rs, soff + 16u * h);
#pragma unroll
        for (int i = 0; i < 4; ++i) wbs[set][4 * h + i] = __uint_as_float(sv[i]);
      }
    } else {
      // per-channel rows read their scales; with one scalar scale the loads
      // fall outside the 4-byte resource (zeros) and the scalar is added
      const uint32_t soff = fp8_pc_off + (uint32_t)kt * 256u + (uint32_t)(bnc * C::BN * 4);
#pragma unroll
      for (int h = 0; h < C::BN / 4; ++h) {
        const u32x4 sv = bload16(rs, soff + 16u * h);
#pragma unroll
        for (int i = 0; i < 4; ++i) wbs[set][4 * h + i] = __uint_as_float(sv[i]) + fp8_scalar;
      }
    }
  };

  // dequantize one register set into weight buffer `buf`; `part` in 0..3 selects
  // a quarter of the work so it can be spread over the four MFMA sub-steps.
  uint32_t bpk[4 * C::BN];  // packed row pairs [pair][k]
  auto store_w = [&](int set, int buf, int part) {
    uint16_t* sA = sW + buf * C::WBUF;
    // BN = 8: rows 2*part, 2*part+1 -> 8 packed dwords (one per k).
    // BN = 4: row pair part/2, k half part%2 -> 4 packed dwords.
    // The transposed tile rows are written at part 3.
    const int pr = (C::BN == 8) ? part : (part >> 1);
    const int q0 = (C::BN == 8) ? 0 : 4 * (part & 1), nq = (C::BN == 8) ? 8 : 4;
    float f0[8], f1[8];
    if (FMT == LRQ_FMT_INT4) {
      dequant8_int4_f32(wb[set][2 * pr], wbs[set][2 * pr], f0, a.nib);
      dequant8_int4_f32(wb[set][2 * pr + 1], wbs[set][2 * pr + 1], f1, a.nib);
    } else {
      fp8x4_to_f32(wb[set][4 * pr], f0);
      fp8x4_to_f32(wb[set][4 * pr + 1], f0 + 4);
      fp8x4_to_f32(wb[set][4 * pr + 2], f1);
      fp8x4_to_f32(wb[set][4 * pr + 3], f1 + 4);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        f0[q] *= wbs[set][2 * pr];
        f1[q] *= wbs[set][2 * pr + 1];
      }
    }
#pragma unroll
    for (int q = q0; q < q0 + nq; ++q) bpk[pr * 8 + q] = pack_bf16x2(f0[q], f1[q]);
    if (part == 3) {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int R = bkc * 8 + q;
        uint16_t* dst = wthr_ok ? (sA + R * LD + bnc * C::BN) : (sDummy + tid * 8);
        if constexpr (C::BN == 8) {
          st16(dst, (u32x4){bpk[q], bpk[8 + q], bpk[16 + q], bpk[24 + q]});
        } else {
          st8(dst, (u32x2){bpk[q], bpk[8 + q]});
        }
      }
    }
  };

  f32x16 acc[NIW][MJ];
#pragma unroll
  for (int i = 0; i < NIW; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  // A-role fragment of row R, logical 8-column chunk c
  auto afrag = [&](const uint16_t* sA, int R, int c) -> bf16x8 {
    return as_bf16x8(ld16(sA + R * LD + c * 8));
  };

  // one reduction step on buffers `buf`; the dequantization of register set
  // `wset` into weight buffer `nbuf` rides along. Fragments of sub-step kk+1
  // are read while sub-step kk's matrix-core work runs, and the schedule
  // interleaves every matrix-core instruction with ~3 VALU (dequantization)
  // and spreads LDS writes and global loads between them.
  auto step = [&](int buf, int wset, int nbuf) {
    const uint16_t* sA = sW + buf * C::WBUF;
    bf16x8 fa[2][NIW], fb[2][MJ];
#pragma unroll
    for (int i = 0; i < NIW; ++i) fa[0][i] = afrag(sA, (rh * NIW + i) * 32 + l32, g * 4);
#pragma unroll
    for (int j = 0; j < MJ; ++j) fb[0][j] = bfrag(buf, j, g * 4);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int cur = kk & 1;
      if (kk < 3) {
#pragma unroll
        for (int i = 0; i < NIW; ++i) fa[cur ^ 1][i] = afrag(sA, (rh * NIW + i) * 32 + l32, g * 4 + kk + 1);
#pragma unroll
        for (int j = 0; j < MJ; ++j) fb[cur ^ 1][j] = bfrag(buf, j, g * 4 + kk + 1);
      }
#pragma unroll
      for (int i = 0; i < NIW; ++i)
#pragma unroll
        for (int j = 0; j < MJ; ++j) acc[i][j] = mfma32(fa[cur][i], fb[cur][j], acc[i][j]);
      store_w(wset, nbuf, kk);
    }
    constexpr int PS = NIW * MJ;                  // matrix-core instructions per sub-step
    constexpr int NM = 4 * PS;                    // ... per step
    constexpr int NW = 8;                         // LDS tile writes
    // VALU per step (dequantization + addressing), measured from the ISA:
    // ~215 for an 8x8 block
    constexpr int NV = 27 * C::BN;
    constexpr int VPM = (NV + NM - 1) / NM;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0);  // VALU
      if (m / PS < 3 && (m % PS) < NI + MJ) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // next sub-step's reads
      if ((m * NW) / NM != ((m + 1) * NW) / NM) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
      if (m % 5 == 2) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
    }
  };

  const int nk = (int)((L + BK - 1) / BK);
  auto kc_ = [&](int kt) -> int { return kt < nk ? kt : nk - 1; };

  // prologue: act(0) -> sX[0]; weight tile 0 -> sW[0]; tile 1 raw -> set 1
  dma_act(0, 0);
  load_w(0, 0);
  load_w(1, kc_(1));
#pragma unroll
  for (int part = 0; part < 4; ++part) store_w(0, 0, part);
  __syncthreads();

  int kt = 0;
  for (; kt + 1 < nk; kt += 2) {
    // even step: compute buffers 0; stage act(kt+1) and weight tile kt+1 into buffers 1
    dma_act(1, (int64_t)(kt + 1) * BK);
    load_w(0, kc_(kt + 2));
    step(0, 1, 1);
    __syncthreads();
    // odd step: compute buffers 1; stage act(kt+2) and weight tile kt+2 into buffers 0
    dma_act(0, (int64_t)kc_(kt + 2) * BK);
    load_w(1, kc_(kt + 3));
    step(1, 0, 0);
    __syncthreads();
  }
  if (kt < nk) {
    // last (even) step; what it stages is never read
    step(0, 1, 1);
    __syncthreads();
  }

  // LoRA: one rank-wide step. A-role rows: A [E, r] staged through weight
  // buffer 0; B-role: u [M, rp] (zero-padded, pre-scaled) from global.
  if (a.rp > 0) {
    uint16_t* sA = sW;
    const int rp = a.rp, r = a.r;
    // A[e0 + row][0 .. r) -> sA[row][0 .. rp), zero-padded
    for (int id = tid; id < RA * rp; id += NT) {
      const int row = id / rp, j = id % rp;
      const int64_t k = e0 + row;
      uint16_t v = 0;
      if (j < r && k < E) v = a.lw[k * r + j];
      sA[row * LD + j] = v;
    }
    __syncthreads();
    u32x4 lb[MJ][4];
#pragma unroll
    for (int j = 0; j < MJ; ++j) {
      const int64_t m = m0 + tw * (32 * MJ) + j * 32 + l32;
      const bool ok = m < M;
      const uint16_t* src = a.lact + (ok ? m : (M - 1)) * rp + g * 8;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        lb[j][kk] = zero4();
        if (kk * 16 < rp) {
          const u32x4 v = ld16(src + kk * 16);
          lb[j][kk] = ok ? v : zero4();
        }
      }
    }
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk * 16 < rp) {
#pragma unroll
        for (int i = 0; i < NIW; ++i) {
          const bf16x8 fa = afrag(sA, (rh * NIW + i) * 32 + l32, kk * 2 + g);
#pragma unroll
          for (int j = 0; j < MJ; ++j) acc[i][j] = mfma32(fa, as_bf16x8(lb[j][kk]), acc[i][j]);
        }
      }
    }
  }

  // epilogue: lane holds 4 consecutive k of one token
#pragma unroll
  for (int i = 0; i < NIW; ++i) {
#pragma unroll
    for (int vg = 0; vg < 4; ++vg) {
      const int64_t e = e0 + (rh * NIW + i) * 32 + 8 * vg + 4 * g;
      if (e >= E) continue;
#pragma unroll
      for (int j = 0; j < MJ; ++j) {
        const int64_t m = m0 + tw * (32 * MJ) + j * 32 + l32;
        if (m < M) {
          u32x2 o;
          o[0] = pack_bf16x2(acc[i][j][4 * vg + 0], acc[i][j][4 * vg + 1]);
          o[1] = pack_bf16x2(acc[i][j][4 * vg + 2], acc[i][j][4 * vg + 3]);
          *reinterpret_cast<u32x2*>(a.out + m * E + e) = o;
        }
      }
    }
  }
}

// ------------------------------------------------------------------ dispatch
int g_num_cus = 256;

// Pick the weight-side tile height (32*NI) minimizing rounds x tile work.
int pick_ni(int64_t extent, int64_t m, const int* cands, int ncands) {
  const int64_t tb = (m + RB - 1) / RB;
  int best = cands[0];
  double best_t = 1e300;
  for (int c = 0; c < ncands; ++c) {
    const int ni = cands[c];
    const int64_t ta = (extent + 32 * ni - 1) / (32 * ni);
    const int64_t rounds = (ta * tb + g_num_cus - 1) / g_num_cus;
    // larger tiles amortize the activation loads; 8% per step down in size
    const double eff = 1.0 + 0.08 * (8 - ni) / 2.0;
    const double t = (double)rounds * ni * eff;
    if (t < best_t - 1e-9) {
      best_t = t;
      best = ni;
    }
  }
  return best;
}

template <int FMT, int NI, int WN>
hipError_t run(hipStream_t st, const GemmArgs& a) {
  const int tiles_m = (int)((a.m + RB - 1) / RB);
  const int tiles_e = (int)((a.e + 32 * NI - 1) / (32 * NI));
  hipLaunchKernelGGL((k_dx<FMT, NI, WN>), dim3(tiles_m * tiles_e), dim3(256 * WN), 0, st, a, tiles_m);
  return hipGetLastError();
}

template <int FMT>
hipError_t dispatch(hipStream_t st, const GemmArgs& a) {
  // NI in {6, 4}: at most one 8x8 block per thread (NI = 8 exceeds the
  // register file). int4: two wavefronts per SIMD (4x8 blocks) hide the
  // dequantization; fp8: 8x8 blocks keep each row's 64 packed bytes in one load
  static const int cands[] = {6, 4};
  switch (pick_ni(a.e, a.m, cands, 2)) {
    case 6: return run<FMT, 6, (FMT == LRQ_FMT_INT4 ? 2 : 1)>(st, a);
    default: return run<FMT, 4, 1>(st, a);
  }
}

}  // namespace

void set_num_cus(int n) { g_num_cus = n > 0 ? n : 256; }
int get_num_cus() { return g_num_cus; }

hipError_t launch_dx(hipStream_t st, int fmt, const GemmArgs& a) {
  if (a.m == 0 || a.e == 0) return hipSuccess;
  return fmt == LRQ_FMT_INT4 ? dispatch<LRQ_FMT_INT4>(st, a) : dispatch<LRQ_FMT_FP8>(st, a);
}
