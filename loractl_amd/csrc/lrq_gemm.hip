// The two fused GEMMs of the quantized LoRA linear on gfx950 matrix cores.
//
//   forward   y[m, n]  = x[m, k] . bf16(dq(w))[n, k]^T  (+bias)  + t[m, :] . B[:, n]
//   backward dx[m, k]  = dy[m, n] . bf16(dq(w))[n, k]          + u[m, :] . A[k, :]^T
//
// (src/quant.rs:175-176 and :229-233 for the base products; the LoRA terms
// are the two small products of src/lora.rs:199-203 and their autodiff,
// with t = s.x.A and u = s.dy.B^T computed by the skinny kernels.)
//
// One kernel template serves both passes. A workgroup owns an RA x 256
// output tile (RA weight-side rows: n forward, k backward; 256 tokens in 4
// token groups of 64). Each token group is served by WN wavefronts that
// split the RA rows; WN = 2 (the large-tile forward) puts two wavefronts on
// each SIMD, so one's dequantization and LDS traffic overlap the other's
// matrix-core work:
//   - the packed weight tile of each 64-wide reduction step is read from
//     HBM/L2 in packed form (int4 nibbles or fp8 bytes), dequantized in
//     registers and written once per workgroup into a double-buffered LDS
//     tile of bf16; a bf16 copy of the weight never exists in HBM. In the
//     backward the reduction runs along n while the packed rows are
//     contiguous along k, so each thread dequantizes an 8x8 block and writes
//     it transposed (XOR-swizzled 16-byte chunks keep the LDS banks apart);
//   - the activation operand (x or dy) is copied global -> LDS by buffer
//     loads with an LDS destination (no register round trip), one reduction
//     step ahead; each wavefront moves and reads only its own 64 tokens, in
//     XOR-swizzled 16-byte chunks;
//   - v_mfma_f32_32x32x16_bf16 with the weight as the A-role operand, so the
//     accumulators hold 4 consecutive output features of one token and the
//     epilogue writes 8-byte runs. The reduction index is permuted inside a
//     step (lane group g takes k = 32g + 8kk .. +8 in sub-step kk) so each
//     lane's activation bytes are 64 contiguous bytes;
//   - the loop is unrolled by two steps so every buffer index is static and
//     the whole step is one basic block: buffer loads past a resource's size
//     return zeros, so edges need no branches (buffer descriptors are forced
//     scalar and selected offsets made opaque so the compiler cannot
//     reintroduce branches), the next tile's dequantization is interleaved
//     with the current tile's matrix-core work, and one barrier ends a step;
//   - the LoRA term is one more rank-wide step after the main loop (the
//     weight-side factor B or A staged through LDS, t or u from global);
//   - fp8 per-output-channel scales factor out of the forward reduction and
//     are applied to the f32 accumulators before the LoRA step; int4 group
//     scales vary along k and are applied during dequantization, exactly
//     (fma(u, s, -8s) == q*s);
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

// WN wavefronts share each token group, splitting its RA weight-side rows:
// WN = 2 gives 8 wavefronts (two per SIMD) with half the accumulators each.
template <bool BWD, int FMT, int NI, int WN>
struct Cfg {
  static constexpr int NT = 256 * WN;  // threads per workgroup
  static constexpr int NIW = NI / WN;  // 32-row tiles per wavefront
  static constexpr int RA = 32 * NI;  // a multiple of 64 (whole weight blocks)
  // forward: 16-byte chunks of the packed weight tile per step, per thread
  static constexpr int WPR = (FMT == LRQ_FMT_INT4) ? 2 : 4;  // chunks per block row (64 k)
  static constexpr int CH = RA * WPR / NT;
  // backward: one BN (n) x 8 (k) block per thread; RA/8 k-chunks x 64/BN
  // n-chunks (BN = 4 with 8 wavefronts keeps 32 values per thread)
  static constexpr int KCH = RA / 8;
  static constexpr int BN = (WN == 2) ? 4 : 8;
  static constexpr int NCH = 64 / BN;
  static constexpr int WORDS = (FMT == LRQ_FMT_INT4) ? 1 : 2;  // dwords per 8 k of one row
  static constexpr int WBUF = RA * LD;                          // weight tile (bf16)
  static constexpr int XBUF = RB * BK;                          // activation tile (bf16)
  static constexpr int LDS_ELEMS = 2 * WBUF + 2 * XBUF + (BWD ? NT * 8 : 0);
  static_assert(NI % WN == 0, "whole row tiles per wavefront");
  static_assert(BWD || CH * NT == RA * WPR, "whole 16-byte weight chunks per thread");
};

template <bool BWD, int FMT, int NI, int WN>
__global__ void __launch_bounds__(256 * WN) __attribute__((amdgpu_waves_per_eu(WN, WN)))
k_gemm(GemmArgs a, int tiles_m) {
  using C = Cfg<BWD, FMT, NI, WN>;
  constexpr int RA = C::RA, NT = C::NT, NIW = C::NIW;
  __shared__ __attribute__((aligned(16))) uint16_t lds[C::LDS_ELEMS];
  uint16_t* const sW = lds;                     // [2][RA][LD]
  uint16_t* const sX = lds + 2 * C::WBUF;       // [2][256][64], 16-byte chunks XOR-swizzled by row
  uint16_t* const sDummy = sX + 2 * C::XBUF;    // backward: per-thread slots for idle threads

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

  // ---------------- activation operand: DMA into LDS, one reduction step ahead
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
  blocked_sizes_dev(FMT, (BWD ? L : E), K, &wbytes, &nsc, a.gshift);
  // forward: resources based at the tile's first block row; backward: whole weight
  const int64_t nb0 = BWD ? 0 : e0 / 64;
  const rsrc_t rw = make_rsrc(a.wdata + nb0 * KB * blkb, clamp_bytes(wbytes - nb0 * KB * blkb));
  const rsrc_t rs = (FMT == LRQ_FMT_INT4)
                        ? make_rsrc(a.wscale + nb0 * Gp * 64, clamp_bytes((nsc - nb0 * Gp * 64) * 4))
                        : make_rsrc(a.wscale, a.per_channel ? clamp_bytes(L * 4) : 4u);

  // forward per-chunk constants: block bi, byte offset inside the block, row, part
  uint32_t fblk[BWD ? 1 : C::CH], finb[BWD ? 1 : C::CH], fsrow[BWD ? 1 : C::CH], fpart[BWD ? 1 : C::CH];
  if (!BWD) {
#pragma unroll
    for (int c = 0; c < C::CH; ++c) {
      const int id = tid + NT * c;
      const int per_blk = 64 * C::WPR;
      const int bi = id / per_blk, inb = id % per_blk;
      const int brow = inb % 64, bpart = inb / 64;  // 16 lanes: 16 rows, one chunk
      fblk[c] = (uint32_t)bi * (uint32_t)KB * blkb;
      finb[c] = (uint32_t)brow * rowb + (uint32_t)bpart * 16u;
      fsrow[c] = (uint32_t)bi * Gp * 64u + (uint32_t)brow;
      fpart[c] = (uint32_t)bpart;
    }
  }
  // backward mapping: nc = tid % NCH (BN n), kc = (tid / NCH) % KCH (8 k), so
  // the NCH lanes of one k-row group write one whole 128-byte tile row;
  // threads past NCH*KCH redo a block and write it to a private dummy slot
  const bool wthr_ok = BWD ? (tid < C::NCH * C::KCH) : true;
  const int bnc = BWD ? tid % C::NCH : 0;
  const int bkc = BWD ? (tid / C::NCH) % C::KCH : 0;
  const int64_t bcol = e0 + bkc * 8;
  const bool bcol_ok = bcol < KB * 64;  // columns in [K, 64*KB) are zero padding
  const uint32_t bcolbyte = bcol_ok ? (uint32_t)((bcol >> 6) * blkb + ((FMT == LRQ_FMT_INT4) ? (bcol & 63) / 2 : (bcol & 63)))
                                    : LRQ_OOB;
  const uint32_t bscol = bcol_ok ? ((FMT == LRQ_FMT_INT4) ? (uint32_t)(bcol >> a.gshift) * 64u * 4u : 0u) : LRQ_OOB;

  // backward fp8: per-channel scale offsets, or the one scalar scale (loop invariant)
  const uint32_t fp8_pc_off = (a.per_channel && bcol_ok) ? 0u : LRQ_OOB;
  const float fp8_scalar = (BWD && FMT == LRQ_FMT_FP8 && !a.per_channel) ? bloadf(rs, bcol_ok ? 0u : LRQ_OOB) : 0.0f;

  u32x4 wf[2][BWD ? 1 : C::CH];            // forward packed chunks
  float wfs[2][BWD ? 1 : C::CH];           // forward chunk scales (int4)
  uint32_t wb[2][BWD ? C::BN * C::WORDS : 1];  // backward BN rows x 8 k
  float wbs[2][BWD ? C::BN : 1];               // backward row scales

  auto load_w = [&](int set, int kt) {
    if (!BWD) {
#pragma unroll
      for (int c = 0; c < C::CH; ++c) {
        const uint32_t off = fblk[c] + (uint32_t)kt * blkb + finb[c];
        wf[set][c] = bload16(rw, off);
        if (FMT == LRQ_FMT_INT4) {
          const uint32_t j = ((uint32_t)kt * 64u + fpart[c] * 32u) >> a.gshift;
          wfs[set][c] = bloadf(rs, (fsrow[c] + j * 64u) * 4u);
        }
      }
    } else {
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
    }
  };

  // dequantize one register set into weight buffer `buf`; `part` in 0..3 selects
  // a quarter of the work so it can be spread over the four MFMA sub-steps.
  uint32_t bpk[BWD ? 4 * C::BN : 1];  // backward: packed row pairs [pair][k]
  u32x2 fp8_half[(!BWD && FMT == LRQ_FMT_FP8) ? C::CH : 1];  // forward fp8: pending half chunk
  auto store_w = [&](int set, int buf, int part) {
    uint16_t* sA = sW + buf * C::WBUF;
    if (!BWD) {
#pragma unroll
      for (int c = 0; c < C::CH; ++c) {
        const int id = tid + NT * c;
        const int per_blk = 64 * C::WPR;
        const int row = (id / per_blk) * 64 + (id % per_blk) % 64;
        const int pt = (id % per_blk) / 64;
        if (FMT == LRQ_FMT_INT4) {
          uint16_t* dst = sA + row * LD + pt * 32 + part * 8;
          st16(dst, dequant8_int4_bf16(wf[set][c][part], wfs[set][c], a.nib));
        } else {
          // two 4-value halves make one 16-byte write
          const u32x2 p = fp8x4_to_bf16(wf[set][c][part]);
          if (part & 1) {
            uint16_t* dst = sA + row * LD + pt * 16 + (part >> 1) * 8;
            st16(dst, (u32x4){fp8_half[c][0], fp8_half[c][1], p[0], p[1]});
          } else {
            fp8_half[c] = p;
          }
        }
      }
    } else {
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
    constexpr int NW = BWD ? 8 : 4 * C::CH;       // LDS tile writes
    // VALU per step (dequantization + addressing), measured from the ISA:
    // ~105 per 16-byte chunk forward, ~215 for the backward 8x8 block
    constexpr int NV = BWD ? 27 * C::BN : 106 * C::CH;
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

  // fp8 forward: the per-output-channel scale factors out of the k reduction
  if (!BWD && FMT == LRQ_FMT_FP8) {
#pragma unroll
    for (int i = 0; i < NIW; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t n = e0 + (rh * NIW + i) * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
        const float s = (n < E) ? (a.per_channel ? a.wscale[n] : a.wscale[0]) : 0.0f;
#pragma unroll
        for (int j = 0; j < MJ; ++j) acc[i][j][v] *= s;
      }
  }

  // LoRA: one rank-wide step. A-role rows: B^T (forward, B is [r, E]) or A
  // (backward, A is [E, r]) staged through weight buffer 0; B-role: t or u
  // [M, rp] (zero-padded, pre-scaled) from global.
  if (a.rp > 0) {
    uint16_t* sA = sW;
    const int rp = a.rp, r = a.r;
    if (!BWD) {
      // B[j][e0 + c*8 .. +8] -> sA[(c*8 + q) * LD + j]
      const int cpr = RA / 8;
      for (int id = tid; id < rp * cpr; id += NT) {
        const int j = id / cpr, c = id % cpr;
        const int64_t n = e0 + c * 8;
        u32x4 v = zero4();
        if (j < r && n < E) v = ld16(a.lw + (int64_t)j * E + n);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          sA[(c * 8 + 2 * q) * LD + j] = (uint16_t)(v[q] & 0xffffu);
          sA[(c * 8 + 2 * q + 1) * LD + j] = (uint16_t)(v[q] >> 16);
        }
      }
    } else {
      // A[e0 + row][0 .. r) -> sA[row][swizzled chunks], zero-padded to rp
      for (int id = tid; id < RA * rp; id += NT) {
        const int row = id / rp, j = id % rp;
        const int64_t k = e0 + row;
        uint16_t v = 0;
        if (j < r && k < E) v = a.lw[k * r + j];
        sA[row * LD + j] = v;
      }
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

  // epilogue: lane holds 4 consecutive weight-side rows (n or k) of one token
#pragma unroll
  for (int i = 0; i < NIW; ++i) {
#pragma unroll
    for (int vg = 0; vg < 4; ++vg) {
      const int64_t e = e0 + (rh * NIW + i) * 32 + 8 * vg + 4 * g;
      if (e >= E) continue;
      f32x4 bv = {0.0f, 0.0f, 0.0f, 0.0f};
      if (!BWD && a.bias) bv = *reinterpret_cast<const f32x4*>(a.bias + e);
#pragma unroll
      for (int j = 0; j < MJ; ++j) {
        const int64_t m = m0 + tw * (32 * MJ) + j * 32 + l32;
        if (m < M) {
          u32x2 o;
          o[0] = pack_bf16x2(acc[i][j][4 * vg + 0] + bv[0], acc[i][j][4 * vg + 1] + bv[1]);
          o[1] = pack_bf16x2(acc[i][j][4 * vg + 2] + bv[2], acc[i][j][4 * vg + 3] + bv[3]);
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

template <bool BWD, int FMT, int NI, int WN>
hipError_t run(hipStream_t st, const GemmArgs& a) {
  const int tiles_m = (int)((a.m + RB - 1) / RB);
  const int tiles_e = (int)((a.e + 32 * NI - 1) / (32 * NI));
  hipLaunchKernelGGL((k_gemm<BWD, FMT, NI, WN>), dim3(tiles_m * tiles_e), dim3(256 * WN), 0, st, a, tiles_m);
  return hipGetLastError();
}

template <bool BWD, int FMT>
hipError_t dispatch(hipStream_t st, const GemmArgs& a) {
  // forward tiles: NI in {8, 4} (whole 16-byte chunks per thread), two
  // wavefronts per token group where the chunks divide (int4 NI = 4 has one);
  // backward: NI in {6, 4} (at most one 8x8
  // block per thread), one wavefront per token group (NI = 8 exceeds the
  // register file). fp8 keeps to the smaller forward tile: its wider raw
  // chunks and the channel-scale epilogue do not fit at NI = 8.
  static const int fwd_c[] = {8, 4};
  static const int bwd_c[] = {6, 4};
  const int skip = (FMT == LRQ_FMT_FP8) ? 1 : 0;
  if constexpr (BWD) {
    switch (pick_ni(a.e, a.m, bwd_c, 2)) {
      // int4: two wavefronts per SIMD (4x8 blocks) hide the dequantization;
      // fp8: 8x8 blocks keep each row's 64 packed bytes in one load
      case 6: return run<BWD, FMT, 6, (FMT == LRQ_FMT_INT4 ? 2 : 1)>(st, a);
      default: return run<BWD, FMT, 4, 1>(st, a);
    }
  } else {
    switch (pick_ni(a.e, a.m, fwd_c, 2)) {
      case 8: return run<BWD, FMT, 8, 2>(st, a);
      default: return run<BWD, FMT, 4, (FMT == LRQ_FMT_FP8 ? 2 : 1)>(st, a);
    }
  }
}

}  // namespace

void set_num_cus(int n) { g_num_cus = n > 0 ? n : 256; }
int get_num_cus() { return g_num_cus; }

hipError_t launch_gemm(hipStream_t st, bool bwd, int fmt, const GemmArgs& a) {
  if (a.m == 0 || a.e == 0) return hipSuccess;
  if (bwd) return fmt == LRQ_FMT_INT4 ? dispatch<true, LRQ_FMT_INT4>(st, a) : dispatch<true, LRQ_FMT_FP8>(st, a);
  return fmt == LRQ_FMT_INT4 ? dispatch<false, LRQ_FMT_INT4>(st, a) : dispatch<false, LRQ_FMT_FP8>(st, a);
}
