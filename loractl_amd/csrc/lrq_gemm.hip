// The two large GEMMs of the quantized LoRA linear (m > 16 tokens), with the
// weight operand dequantized straight into matrix-core registers:
//
//   forward   y[m, n]  = x[m, k]  . bf16(dq(w))[n, k]^T (+bias) + t[m, :] . B[:, n]
//   backward  dx[m, k] = dy[m, n] . bf16(dq(w))[n, k]            + u[m, :] . A[k, :]^T
//
// (src/quant.rs:175-176 and :229-233 for the base products; the LoRA terms
// are the two small products of src/lora.rs:199-203 and their autodiff, with
// t = bf16(s . x . A), u = bf16(s . dy . B^T) and the weight-side factor
// rows (B^T or A, [rows][rp]) prepared by the LoRA side kernels.)
//
// One kernel template serves both passes. Call the output columns "rows"
// (n forward, k backward) and the reduction index "depth" (k forward, n
// backward). Output tiles are RA rows x 256 tokens; a persistent grid of one
// workgroup per CU walks its tiles, and four wavefronts (one per SIMD) each
// own two 32-row tiles of a tile:
//   - RA = 256: rows 64w .. 64w+63, both row tiles for all 256 tokens;
//   - RA = 192 (when it fills the CUs better, e.g. 3072 output rows): row
//     tile 0 = rows 32w .. +32 for all 256 tokens, row tile 1 = rows
//     128 + 32(w/2) .. +32 for one 128-token half (h = w%2): two wavefronts
//     share that row tile, split by tokens. Those wavefronts see the token
//     tiles rotated by four (local tile j = token tile (j + 4h) % 8), so
//     their half is always local tiles 0..3 and no register index depends on
//     the wavefront.
// Accumulators: v_mfma_f32_32x32x16_bf16, weight rows in the A role, tokens
// in the B role, 2 x 8 tiles of 16 f32 per lane.
//   - weight (A role): each lane loads the packed bytes of its own row from
//     the blocked layout (int4: 16 bytes = 32 depth of one row, fp8: 32
//     bytes), dequantizes them in registers to the exact bf16 operand and
//     feeds the matrix cores. The depth index is permuted inside a 64-wide
//     step: lane group g (lanes 32g .. 32g+31) takes depth 32g + 8kk .. +8 in
//     sub-step kk, so a lane's packed bytes are contiguous. The forward reads
//     the row section (rows n, int4 nibbles q+8, one group scale per lane and
//     step: fma(u, s, -8s) == q*s exactly, then bf16; fp8: the exact e4m3
//     value, its scale applied to the accumulators). The backward reads the
//     transposed section (rows k, depth n): each of a lane's 8 values has its
//     own scale (int4: scale of row n and group k/group; fp8: channel scale of
//     n). Lane l of each 16-lane row holds the scale of depth 32g + 16p + l
//     (p = kk/2, one register per half step) and a DPP row broadcast hands
//     value 8(kk%2) + e to every lane: q (sign-extended nibble, or the e4m3
//     value) times that scale, rounded to bf16 -- the same bf16(q * s) the
//     forward's operand holds;
//   - activations (B role): the 256 x 64 token tile of a step is copied
//     global -> LDS by buffer loads with an LDS destination (each wavefront
//     moves 64 token rows) and read by all four wavefronts;
//   - the pipeline: token tiles in two LDS buffers and packed weights in two
//     register sets, one step ahead, continuing across tiles: the last steps
//     of a tile prefetch the first steps of the workgroup's next tile, so
//     that tile's loads are in flight while this tile's epilogue (LoRA step,
//     bias, stores) runs, and the stores drain under the next tile's
//     matrix-core work. The one barrier of a step sits between its third and
//     fourth sub-steps, after the last fragment reads of the current buffer;
//   - edges: buffer loads past a resource's size return zeros (partial token
//     and weight tiles, the depth tail and the zero step that rounds a tile's
//     steps up to an even count); padding weight rows and depth columns hold
//     q = 0;
//   - epilogue: the LoRA term is one rank-wide matrix-core step (the tile's
//     token-side and weight-side factor rows, copied into LDS while the
//     tile's main loop runs); then forward fp8 channel scales (they factor
//     out of the depth reduction; B^T arrives divided by them) and the bias;
//     each wavefront then passes its bf16 output rows through LDS so that
//     every store writes whole 128-byte (RA = 256) or 64-byte row segments;
//   - tile order: workgroup b's i-th tile is virtual tile b + i*G, mapped so
//     each XCD (own L2) works on a contiguous range of tiles, grouped four
//     token tiles deep;
//   - split depth: with fewer tiles than CUs (few tokens, or a narrow output)
//     the depth range of every tile is cut into S ranges of whole steps; a
//     work unit is (tile, range), the persistent grid walks units as it walks
//     tiles, each unit writes its f32 accumulators to a partial buffer
//     [S][m][e] (range 0 adds the LoRA term), and k_split_reduce sums the S
//     partials in range order, applies the forward fp8 scales and bias and
//     rounds once to bf16.

#include "lrq_common.h"
#include "lrq_kernels.h"

namespace {

constexpr int BK = 64;         // reduction step
constexpr int MJ = 8;          // 32-token tiles per wavefront (row tile 0)
constexpr int RB = MJ * 32;    // tokens per tile (256)
constexpr int XBUF = RB * BK;  // bf16 per activation buffer (32 KB)
constexpr int GM = 4;          // token tiles per group of the tile order
constexpr int NBUF = 2;        // pipeline depth (LDS buffers, register sets)

// activation LDS tile [256 rows][64] bf16: 128-byte rows, 16-byte chunk c of
// row r at chunk c ^ swz(r), so the 16 lanes of a read pass (16 rows at one
// logical chunk) cover all 64 banks
LRQ_DEV int swz(int r) { return (r >> 1) & 7; }

// Per-unit load sources: the activation rows of wavefront w's DMA share, the
// weight block row(s) (data; forward int4 scales), backward int4 the byte
// offsets of the two row tiles' group rows in the transposed scale table,
// and the unit's first step and depth range.
struct TileSrc {
  int64_t m0, e0;
  rsrc_t act, wd, ws;
  uint32_t sk0, sk1;
  int k0, sp;
};

template <bool BWD, int FMT, bool R192, bool SPLIT>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
k_gemm(GemmArgs a, int tiles_m, int ntiles) {
  constexpr bool I4 = FMT == LRQ_FMT_INT4;
  constexpr bool I8 = FMT == LRQ_FMT_INT8;
  constexpr bool GS = I4 || I8;         // group scales (int4, int8) or channel scales (fp8)
  constexpr int WV = I4 ? 1 : 2;        // 16-byte packed loads per row tile per step
  constexpr int RA = R192 ? 192 : 256;  // rows per tile
  constexpr int MJ1 = R192 ? 4 : MJ;    // token tiles of row tile 1
  constexpr int NSC = GS ? 2 : 1;       // backward scale registers: per row tile (int4, int8) or shared (fp8)
  __shared__ __attribute__((aligned(16))) uint16_t sX0[XBUF];
  __shared__ __attribute__((aligned(16))) uint16_t sX1[XBUF];
  // epilogue region: the tile's LoRA operands (token rows, then weight-side
  // rows, [256][rp] each) copied in during the tile, then each wavefront's
  // output rows
  __shared__ __attribute__((aligned(16))) uint16_t sE[4 * 128 * 64];
  // forward: the tile's bias [256] and fp8 channel scales [256], f32
  __shared__ __attribute__((aligned(16))) float sAux[BWD ? 4 : 2 * 256];

  const int G = gridDim.x;
  const int S = SPLIT ? a.splits : 1;
  const int nunits = ntiles * S;
  int vb = blockIdx.x;
  if (vb >= nunits) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int H = R192 ? (w & 1) : 0;  // token-half rotation of this wavefront
  const int64_t M = a.m, K = a.l, E = a.e;
  const int tiles_a = ntiles / tiles_m;
  // rows (within the tile) of the wavefront's two row tiles
  const int ro0 = R192 ? 32 * w : 64 * w;
  const int ro1 = R192 ? 128 + 32 * (w >> 1) : 64 * w + 32;

  const int64_t KB = (K + 63) / 64;
  constexpr uint32_t blkb = I4 ? 2048u : 4096u;  // bytes per 64x64 block
  constexpr uint32_t rowb = I4 ? 32u : 64u;      // bytes per block row
  const uint32_t Gp = (GS && !BWD) ? (uint32_t)((KB * 64) >> a.gshift) : 0u;
  int64_t wbytes, nsc;
  blocked_sizes_dev(FMT, E, K, &wbytes, &nsc, a.gshift);
  const int nk = (int)KB;
  // steps per unit: the whole depth rounded up to whole pipeline rounds, or
  // one split range (a multiple of NBUF; the last range may run past nk)
  const int nkp = SPLIT ? a.spl : (nk + NBUF - 1) / NBUF * NBUF;

  // backward scales: int4 and int8 ST [KGt][64*KB] (row n = depth, group kg
  // of the output row k); fp8 the channel scales [n] or one scalar
  const int64_t NP = KB * 64;
  const int64_t KGt = (BWD && GS) ? (((E + 63) / 64 * 64 + (1 << a.gshift) - 1) >> a.gshift) : 0;
  const bool pc = !GS && a.per_channel;
  const rsrc_t rbs = BWD ? (GS ? make_rsrc(a.wscale, clamp_bytes(KGt * NP * 4))
                               : make_rsrc(a.wscale, pc ? clamp_bytes(K * 4) : 0u))
                         : make_rsrc(a.wscale, 0u);
  // fp8 with one scalar scale: the per-channel loads read zeros, plus this
  const float s0add = (BWD && !GS && !pc) ? a.wscale[0] : 0.0f;

  // sources of virtual unit v (zero-size resources when v is past the grid);
  // the S ranges of a tile are consecutive units
  auto tile_src = [&](int v) -> TileSrc {
    TileSrc t;
    const bool ok = v < nunits;
    const int lu = xcd_remap(ok ? v : 0, nunits);
    const int logical = SPLIT ? lu / S : lu;
    t.sp = SPLIT ? lu % S : 0;
    t.k0 = t.sp * nkp;
    const int grp = logical / (GM * tiles_a), within = logical % (GM * tiles_a);
    const int gm = min(GM, tiles_m - grp * GM);
    const int tm = grp * GM + within % gm, ta = within / gm;
    t.m0 = (int64_t)tm * RB;
    t.e0 = (int64_t)ta * RA;
    const int64_t mw = t.m0 + 64 * w;
    const int64_t mrows = ok ? ((M - mw) < 64 ? (M - mw) : 64) : 0;
    t.act = make_rsrc(a.act + (mw < M ? mw : 0) * K, clamp_bytes(mrows * K * 2));
    // block row of the resource base: the wavefront's own (RA = 256) or the tile's first
    const int64_t nb = t.e0 / 64 + (R192 ? 0 : w);
    t.wd = make_rsrc(a.wdata + nb * KB * blkb, ok ? clamp_bytes(wbytes - nb * KB * blkb) : 0u);
    t.ws = make_rsrc(a.wscale + ((GS && !BWD) ? nb * Gp * 64 : 0),
                     (GS && !BWD && ok) ? clamp_bytes((nsc - nb * Gp * 64) * 4) : 0u);
    t.sk0 = (BWD && GS) ? (uint32_t)(((t.e0 + ro0) >> a.gshift) * NP * 4) : 0u;
    t.sk1 = (BWD && GS) ? (uint32_t)(((t.e0 + ro1) >> a.gshift) * NP * 4) : 0u;
    return t;
  };

  // ---------------- activation DMA: wavefront w moves token rows 64w .. +64
  // 8 buffer loads per step; lane l of load c lands at row 64w + 8c + l/8,
  // physical chunk l%8, and fetches logical chunk (l%8) ^ swz(row), where
  // swz(64w + 8c + l/8) = (4c + l/16) & 7 alternates with the parity of c.
  const int drow = lane >> 3;
  const int dq0 = (lane & 7) ^ ((lane >> 4) & 7), dq1 = (lane & 7) ^ (((lane >> 4) + 4) & 7);
  const uint32_t doff0 = (uint32_t)((drow * K + dq0 * 8) * 2), doff1 = (uint32_t)((drow * K + dq1 * 8) * 2);
  auto dma = [&](uint16_t* buf, const rsrc_t& ract, int kt) {
    const int64_t k0 = (int64_t)kt * BK;
    const bool kok0 = k0 + dq0 * 8 < K, kok1 = k0 + dq1 * 8 < K;  // K % 8 == 0
    const uint32_t koff = (uint32_t)(k0 * 2);
    __attribute__((address_space(3))) char* base =
        (__attribute__((address_space(3))) char*)(lds_void*)(buf + 64 * w * BK);
    // the per-load offsets are formed here from opaque bases each step, so
    // the compiler does not keep 16 hoisted copies live across the loop
    const uint32_t o0 = opaque_u32(doff0) + koff, o1 = opaque_u32(doff1) + koff;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const bool kok = (c & 1) ? kok1 : kok0;
      const uint32_t off = opaque_u32(kok ? ((c & 1) ? o1 : o0) + (uint32_t)(c * 8 * K * 2) : LRQ_OOB);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ract, (lds_void*)(base + c * 8 * BK * 2), 16, off, 0, 0, 0);
    }
  };
  // B-role fragment of local token tile j in sub-step kk: token tile
  // j' = (j + 4H) % 8, row 32j' + l32, logical chunk 4g + kk, stored at chunk
  // (4g + kk) ^ swz(l32) (swz(32j' + l32) = swz(l32)). The per-lane chunk
  // bases are fixed (xk: local tiles 0..3, xq: 4..7); tile and buffer offsets
  // are immediates of the LDS read.
  const uint32_t xrow = (uint32_t)(l32 * BK * 2) | (uint32_t)(swz(l32) * 16);
  constexpr uint32_t HALF = 4 * 32 * BK * 2;  // bytes of four token tiles
  uint32_t xk[4], xq[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const uint32_t c = xrow ^ (uint32_t)((4 * g + kk) * 16);
    xk[kk] = opaque_u32(c + (uint32_t)H * HALF);
    xq[kk] = R192 ? opaque_u32(c + (uint32_t)(1 - H) * HALF) : 0u;
  }
  auto xfrag = [&](const uint16_t* buf, int j, int kk) -> bf16x8 {
    const char* b = reinterpret_cast<const char*>(buf);
    if (!R192 || j < 4) return as_bf16x8(ld16(b + xk[kk] + (uint32_t)(j * 32 * BK * 2)));
    return as_bf16x8(ld16(b + xq[kk] + (uint32_t)((j - 4) * 32 * BK * 2)));
  };

  // ---------------- weight: offsets from the resource's block row: the
  // lane's part (row l32 of a row tile, lane group g's 16 (int4) or 32 (fp8,
  // int8) bytes; group scale of row l32) plus a wavefront-uniform part per row tile
  // (a constant for RA = 256, so it folds into the loads' immediates)
  const uint32_t woff = (uint32_t)l32 * rowb + (uint32_t)g * (I4 ? 16u : 32u);
  const uint32_t soff = (uint32_t)l32 * 4u;
  auto wrow = [&](int i) -> uint32_t {  // uniform data offset of row tile i
    if (!R192) return (uint32_t)i * 32u * rowb;
    const int ro = i ? ro1 : ro0;
    return (uint32_t)(ro >> 6) * (uint32_t)KB * blkb + (uint32_t)(ro & 63) * rowb;
  };
  auto srow = [&](int i) -> uint32_t {  // uniform group-scale offset of row tile i
    if (!R192) return (uint32_t)i * 128u;
    const int ro = i ? ro1 : ro0;
    return ((uint32_t)(ro >> 6) * Gp * 64u + (uint32_t)(ro & 63)) * 4u;
  };
  // backward: lane l of a 16-lane row holds the scale of depth 32g + 16p + l%16
  const uint32_t bsoff = (uint32_t)(32 * g + (lane & 15)) * 4u;
  u32x4 wp[NBUF][2 * WV];   // packed weight bytes per register set
  float wsc[NBUF][2];       // forward int4 / int8 group scales per register set
  float bsc[NBUF][NSC][2];  // backward per-depth scales, two halves of a step
  auto load_w = [&](int set, const TileSrc& t, int kt) {
    // steps past the tile's last one read zeros (bytes and scales)
    const uint32_t kb = opaque_u32(kt < nk ? (uint32_t)kt * blkb : LRQ_OOB);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int h = 0; h < WV; ++h) wp[set][i * WV + h] = bload16(t.wd, kb + woff + wrow(i) + 16u * h);
    if (!BWD && GS) {
      const uint32_t j = ((uint32_t)kt * 64u + (uint32_t)g * 32u) >> a.gshift;
      const uint32_t so = opaque_u32(kt < nk ? (j * 64u) * 4u : LRQ_OOB);
#pragma unroll
      for (int i = 0; i < 2; ++i) wsc[set][i] = bloadf(t.ws, so + soff + srow(i));
    }
    if (BWD) {
      const uint32_t sb = opaque_u32(kt < nk ? (uint32_t)kt * 256u + bsoff : LRQ_OOB);
      if (GS) {
        bsc[set][0][0] = bloadf(rbs, sb + t.sk0);
        bsc[set][0][1] = bloadf(rbs, sb + t.sk0 + 64u);
        bsc[set][NSC - 1][0] = bloadf(rbs, sb + t.sk1);
        bsc[set][NSC - 1][1] = bloadf(rbs, sb + t.sk1 + 64u);
      } else {
        bsc[set][0][0] = bloadf(rbs, sb) + s0add;
        bsc[set][0][1] = bloadf(rbs, sb + 64u) + s0add;
      }
    }
  };
  // A-role fragment of row tile i, sub-step kk, from register set `set`
  auto wfrag = [&](int set, int i, int kk) -> bf16x8 {
    if (!BWD) {
      if (I4) return as_bf16x8(dequant8_int4_bf16(wp[set][i][kk], wsc[set][i], a.nib));
      const u32x4 v = wp[set][i * WV + (kk >> 1)];
      if (I8) return as_bf16x8(dequant8_int8_bf16((u32x2){v[2 * (kk & 1)], v[2 * (kk & 1) + 1]}, wsc[set][i]));
      const u32x2 lo = fp8x4_to_bf16(v[2 * (kk & 1)]), hi = fp8x4_to_bf16(v[2 * (kk & 1) + 1]);
      return as_bf16x8((u32x4){lo[0], lo[1], hi[0], hi[1]});
    }
    float f[8];
    const float S = bsc[set][GS ? i : 0][kk >> 1];
    if (I4) {
      const uint32_t d = wp[set][i][kk];
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = (float)((int)(d << (28 - 4 * e)) >> 28);
    } else if (I8) {
      const u32x4 v = wp[set][i * WV + (kk >> 1)];
      int8x4_to_f32(v[2 * (kk & 1)], f);
      int8x4_to_f32(v[2 * (kk & 1) + 1], f + 4);
    } else {
      const u32x4 v = wp[set][i * WV + (kk >> 1)];
      fp8x4_to_f32(v[2 * (kk & 1)], f);
      fp8x4_to_f32(v[2 * (kk & 1) + 1], f + 4);
    }
    mul_row_bcast8(f, S, kk & 1);
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(f[2 * q], f[2 * q + 1]);
    return as_bf16x8(o);
  };

  f32x16 acc[2][MJ];
  auto zero_acc = [&]() {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < MJ; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
  };

  uint16_t* const bufs[2] = {sX0, sX1};
  bf16x8 fa[2][2], fb[2][MJ];

  // One step on LDS buffer `b` and register set `b` (b = step % 2; the
  // unrolled loop makes both static). On entry fa[0] and fb[0] hold sub-step
  // 0's fragments; on exit they hold the next step's. After the barrier the
  // step refills buffer and set b with step `lkt` of tile `ls`.
  auto step = [&](const int b, const TileSrc& ls, const int lkt) {
    const uint16_t* buf = bufs[b];
    const int nb_ = (b + 1) % NBUF;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int cur = kk & 1;
      if (kk < 3) {
#pragma unroll
        for (int j = 0; j < MJ; ++j) fb[cur ^ 1][j] = xfrag(buf, j, kk + 1);
#pragma unroll
        for (int i = 0; i < 2; ++i) fa[cur ^ 1][i] = wfrag(b, i, kk + 1);
      } else {
        // every read of buffer b is issued: one barrier, then refill buffer
        // and register set b, and read the next step's first fragments from
        // buffer nb_ while sub-step 3 runs
        __syncthreads();
        dma(bufs[b], ls.act, lkt);
        load_w(b, ls, lkt);
#pragma unroll
        for (int j = 0; j < MJ; ++j) fb[cur ^ 1][j] = xfrag(bufs[nb_], j, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i) fa[cur ^ 1][i] = wfrag(nb_, i, 0);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < (i == 0 ? MJ : MJ1); ++j) acc[i][j] = mfma32(fa[cur][i], fb[cur][j], acc[i][j]);
    }
  };

  const int rp = a.rp;
  // LoRA operands of a tile: token rows [m0, m0+256) and weight-side rows
  // [e0, e0+256) (only RA of them used), 256 * rp bf16 each, contiguous in
  // global memory (rows past M or E read zeros); copied to sE as [256][rp]
  // each, 16 bytes per lane per load
  const rsrc_t rbt = make_rsrc(a.lw, rp > 0 ? clamp_bytes(E * rp * 2) : 0u);
  const rsrc_t rt = make_rsrc(a.lact, rp > 0 ? clamp_bytes(M * rp * 2) : 0u);
  const int lora_loads = rp / 8;  // 16-byte loads per lane per operand: 256*rp*2 / (256*16)
  const bool has_bias = !BWD && a.bias != nullptr;
  const bool fpc = !BWD && pc;  // forward fp8 channel scales in the epilogue
  const rsrc_t rbias = make_rsrc(a.bias, has_bias ? clamp_bytes(E * 4) : 0u);
  const rsrc_t rsc = make_rsrc(a.wscale, fpc ? clamp_bytes(E * 4) : 0u);
  // copies for the tile at (m0, e0), issued at its start: LoRA operands to sE,
  // forward bias and fp8 channel scales of its output columns to sAux
  // (columns past E read zeros)
  auto dma_aux = [&](int64_t m0, int64_t e0) {
    __attribute__((address_space(3))) char* base = (__attribute__((address_space(3))) char*)(lds_void*)sE;
    const uint32_t tb = (uint32_t)(m0 * rp * 2), bb = (uint32_t)(e0 * rp * 2);
    for (int c = 0; c < lora_loads; ++c) {
      const uint32_t o = (uint32_t)((c * 256 + w * 64) * 16);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rt, (lds_void*)(base + o), 16, opaque_u32(tb + o + lane * 16), 0, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rbt, (lds_void*)(base + 256 * rp * 2 + o), 16,
                                               opaque_u32(bb + o + lane * 16), 0, 0, 0);
    }
    if (!BWD) {
      __attribute__((address_space(3))) char* abase = (__attribute__((address_space(3))) char*)(lds_void*)sAux;
      const uint32_t co = opaque_u32((uint32_t)(e0 * 4 + lane * 16));
      if (w == 0 && has_bias) __builtin_amdgcn_raw_ptr_buffer_load_lds(rbias, (lds_void*)abase, 16, co, 0, 0, 0);
      if (w == 1 && fpc) __builtin_amdgcn_raw_ptr_buffer_load_lds(rsc, (lds_void*)(abase + 256 * 4), 16, co, 0, 0, 0);
    }
  };

  // epilogue of the tile at (m0, e0). Its per-lane values are derived from
  // an opaque copy of the lane id, so the compiler recomputes them per tile
  // instead of hoisting them out of the tile loop (where they would only be
  // spilled: the main loop holds the registers).
  auto epilogue = [&](int64_t m0, int64_t e0) {
    const int lane = (int)opaque_u32((uint32_t)threadIdx.x & 63u);
    const int g = lane >> 5, l32 = lane & 31;
    // LoRA: one rank-wide step from sE; A role = weight-side rows ro_i + l32,
    // B role = token rows 32 ((j + 4H) % 8) + l32, rank columns 16kk + 8g .. +8
    if (rp > 0) {
      const uint16_t* sT = sE;
      const uint16_t* sBt = sE + 256 * rp;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (kk * 16 < rp) {
          bf16x8 la[2];
          la[0] = as_bf16x8(ld16(sBt + (ro0 + l32) * rp + kk * 16 + g * 8));
          la[1] = as_bf16x8(ld16(sBt + (ro1 + l32) * rp + kk * 16 + g * 8));
#pragma unroll
          for (int j = 0; j < MJ; ++j) {
            const int tj = R192 ? ((j + 4 * H) & 7) : j;
            const bf16x8 lb = as_bf16x8(ld16(sT + (32 * tj + l32) * rp + kk * 16 + g * 8));
            acc[0][j] = mfma32(la[0], lb, acc[0][j]);
            if (j < MJ1) acc[1][j] = mfma32(la[1], lb, acc[1][j]);
          }
        }
      }
    }
    // keep the accumulators in AGPRs here: the packing below then copies one
    // tile at a time to VGPRs, instead of the whole set before the LoRA step
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < MJ; ++j) asm volatile("" : "+a"(acc[i][j]));
    // every wavefront's LoRA reads are done before sE takes output rows
    __syncthreads();
    // output: per half of the local tokens, the wavefront's [128 tokens][64]
    // bf16 staging rows (columns 0..31 row tile 0, 32..63 row tile 1) go to
    // its sE slice (16-byte chunk c of row r at c ^ swz(r)), then back out in
    // row segments, 8 rows per store
    uint16_t* sO = sE + w * 128 * 64;
    const float s0 = (!BWD && !GS && !pc) ? a.wscale[0] : 1.0f;
    // output rows of this tile: a resource from row m0, so rows past M fall
    // outside it
    const rsrc_t ry = make_rsrc(a.out + m0 * E, clamp_bytes((M - m0) * E * 2));
    const int rr = lane >> 3, cc = lane & 7;
    // staging chunk cc: column 8cc of row tile 0 (cc < 4) or 8(cc-4) of row
    // tile 1; RA = 256 keeps the two row tiles adjacent
    const int64_t ncol = e0 + (R192 ? ((cc < 4) ? ro0 + 8 * cc : ro1 + 8 * (cc - 4)) : ro0 + 8 * cc);
    const uint32_t ybase0 = (uint32_t)(ncol * 2);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int row = 32 * jj + l32;
        // one 32-token tile at a time, so few accumulators are in flight
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          if (R192 && i == 1 && h == 1) continue;  // row tile 1 covers local tokens 0..127
#pragma unroll
          for (int vg = 0; vg < 4; ++vg) {
            const int ro = i ? ro1 : ro0;
            const f32x4 bv = has_bias ? *reinterpret_cast<const f32x4*>(sAux + ro + 8 * vg + 4 * g)
                                      : (f32x4){0.f, 0.f, 0.f, 0.f};
            // forward fp8: the per-output-channel scale factors out of the
            // depth reduction (the LoRA operand bt arrives divided by it);
            // per-channel scales of columns past E are zero (not stored)
            const f32x4 sv = (BWD || GS) ? (f32x4){1.f, 1.f, 1.f, 1.f}
                                         : (pc ? *reinterpret_cast<const f32x4*>(sAux + 256 + ro + 8 * vg + 4 * g)
                                               : (f32x4){s0, s0, s0, s0});
            const f32x16& c = acc[i][4 * h + jj];
            u32x2 o;
            o[0] = pack_bf16x2(__builtin_fmaf(c[4 * vg + 0], sv[0], bv[0]), __builtin_fmaf(c[4 * vg + 1], sv[1], bv[1]));
            o[1] = pack_bf16x2(__builtin_fmaf(c[4 * vg + 2], sv[2], bv[2]), __builtin_fmaf(c[4 * vg + 3], sv[3], bv[3]));
            const int chunk = (4 * i + vg) ^ swz(row);
            st8(sO + row * 64 + chunk * 8 + g * 4, o);
          }
        }
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wavefront's rows are in LDS
      // local half h holds tokens m0 + 128 (h ^ H) ..
      const uint32_t ybase = ybase0 + (uint32_t)(128 * (h ^ H) * E * 2);
      const bool cok = ncol < E && !(R192 && h == 1 && cc >= 4);
#pragma unroll
      for (int p = 0; p < 16; ++p) {
        const int row = 8 * p + rr;
        const u32x4 v = ld16(sO + row * 64 + (cc ^ swz(row)) * 8);
        // columns past E (and the unused half of row tile 1) are skipped
        // (offset past the resource); rows past M are past it already
        const uint32_t off = cok ? ybase + (uint32_t)(row * E * 2) : LRQ_OOB;
        // non-temporal (aux bit 1): the output is not read again in this
        // launch, and streaming it past the caches keeps the activation and
        // weight tiles there (the north-star step 0.9% faster)
        __builtin_amdgcn_raw_buffer_store_b128(v, ry, opaque_u32(off), 0, 2);
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // reads done before the next half's writes
    }
  };

  // split-depth epilogue: range 0 adds the LoRA term; every range stores
  // its f32 accumulators to part[range][m][e], four consecutive e per 16-byte
  // store (rows past M fall outside the resource, columns past E are skipped)
  auto epilogue_partial = [&](const TileSrc& u) {
    const int lane = (int)opaque_u32((uint32_t)threadIdx.x & 63u);
    const int g = lane >> 5, l32 = lane & 31;
    if (rp > 0 && u.sp == 0) {
      const uint16_t* sT = sE;
      const uint16_t* sBt = sE + 256 * rp;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        if (kk * 16 < rp) {
          bf16x8 la[2];
          la[0] = as_bf16x8(ld16(sBt + (ro0 + l32) * rp + kk * 16 + g * 8));
          la[1] = as_bf16x8(ld16(sBt + (ro1 + l32) * rp + kk * 16 + g * 8));
#pragma unroll
          for (int j = 0; j < MJ; ++j) {
            const int tj = R192 ? ((j + 4 * H) & 7) : j;
            const bf16x8 lb = as_bf16x8(ld16(sT + (32 * tj + l32) * rp + kk * 16 + g * 8));
            acc[0][j] = mfma32(la[0], lb, acc[0][j]);
            if (j < MJ1) acc[1][j] = mfma32(la[1], lb, acc[1][j]);
          }
        }
      }
    }
    const rsrc_t rp_ = make_rsrc(a.part + ((int64_t)u.sp * M + u.m0) * E, clamp_bytes((M - u.m0) * E * 4));
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < (i == 0 ? MJ : MJ1); ++j) {
        const int tj = R192 ? ((j + 4 * H) & 7) : j;
        const uint32_t rowoff = (uint32_t)((32 * tj + l32) * E * 4);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int vg = 0; vg < 4; ++vg) {
          const int64_t e = u.e0 + (i ? ro1 : ro0) + 8 * vg + 4 * g;
          const f32x16& c = acc[i][j];
          const u32x4 v = {__float_as_uint(c[4 * vg]), __float_as_uint(c[4 * vg + 1]), __float_as_uint(c[4 * vg + 2]),
                           __float_as_uint(c[4 * vg + 3])};
          const uint32_t off = e < E ? rowoff + (uint32_t)(e * 4) : LRQ_OOB;
          __builtin_amdgcn_raw_buffer_store_b128(v, rp_, opaque_u32(off), 0, 0);
        }
      }
  };

  // prologue: the first tile's first two steps in flight
  TileSrc cur = tile_src(vb);
#pragma unroll
  for (int b = 0; b < NBUF; ++b) {
    dma(bufs[b], cur.act, cur.k0 + b);
    load_w(b, cur, cur.k0 + b);
  }
  dma_aux(cur.m0, cur.e0);
  zero_acc();
  __syncthreads();
#pragma unroll
  for (int j = 0; j < MJ; ++j) fb[0][j] = xfrag(bufs[0], j, 0);
#pragma unroll
  for (int i = 0; i < 2; ++i) fa[0][i] = wfrag(0, i, 0);

  for (;;) {
    int kt = 0;
    for (; kt + NBUF < nkp; kt += NBUF) {
#pragma unroll
      for (int b = 0; b < NBUF; ++b) step(b, cur, cur.k0 + kt + NBUF + b);
    }
    // last two steps: prefetch the next unit's first steps
    const TileSrc nxt = tile_src(vb + G);
#pragma unroll
    for (int b = 0; b < NBUF; ++b) step(b, nxt, nxt.k0 + b);
    if (SPLIT)
      epilogue_partial(cur);
    else
      epilogue(cur.m0, cur.e0);
    vb += G;
    if (vb >= nunits) break;
    zero_acc();
    cur = nxt;
    // every wavefront's output reads of sE are done before the next tile's
    // LoRA operands land there
    __syncthreads();
    dma_aux(cur.m0, cur.e0);
  }
  // drain the look-ahead copies before the workgroup ends
  __builtin_amdgcn_s_waitcnt(0);
}

template <bool BWD, int FMT, bool R192, bool SPLIT>
hipError_t run(hipStream_t st, const GemmArgs& a) {
  constexpr int RA = R192 ? 192 : 256;
  const int tiles_m = (int)((a.m + RB - 1) / RB);
  const int tiles_e = (int)((a.e + RA - 1) / RA);
  const int ntiles = tiles_m * tiles_e;
  const int nunits = ntiles * (SPLIT ? a.splits : 1);
  const int grid = nunits < get_num_cus() ? nunits : get_num_cus();
  hipLaunchKernelGGL((k_gemm<BWD, FMT, R192, SPLIT>), dim3(grid), dim3(256), 0, st, a, tiles_m, ntiles);
  return hipGetLastError();
}

// 192-row tiles when they fill the CUs in fewer rounds of work: a tile round
// of RA = 192 costs about 0.8 of a 256-row round (3/4 of the matrix-core
// work, with a larger dequantization share).
bool use_r192(int64_t m, int64_t e) {
  const int64_t tm = (m + RB - 1) / RB, cus = get_num_cus();
  const int64_t r256 = ((e + 255) / 256 * tm + cus - 1) / cus;
  const int64_t r192 = ((e + 191) / 192 * tm + cus - 1) / cus;
  return 0.8 * (double)r192 < (double)r256 - 1e-9;
}

// out[m, e] = bf16(sc(e) * sum over ranges (in order) of part[s][m][e] +
// bias(e)); sc = the forward fp8 channel scale or scalar, else 1. Four
// consecutive e per thread (e % 4 == 0).
__global__ void __launch_bounds__(256) k_split_reduce(const float* __restrict__ part, int S, int64_t M, int64_t E,
                                                      const float* __restrict__ scale, int per_channel,
                                                      const float* __restrict__ bias, uint16_t* __restrict__ out) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (q >= M * E / 4) return;
  const int64_t e = (q * 4) % E;
  f32x4 sum = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < S; ++s) {
    const f32x4 v = reinterpret_cast<const f32x4*>(part + (int64_t)s * M * E)[q];
#pragma unroll
    for (int i = 0; i < 4; ++i) sum[i] += v[i];
  }
  f32x4 sc = {1.f, 1.f, 1.f, 1.f}, bv = {0.f, 0.f, 0.f, 0.f};
  if (scale) sc = per_channel ? *reinterpret_cast<const f32x4*>(scale + e) : (f32x4){scale[0], scale[0], scale[0], scale[0]};
  if (bias) bv = *reinterpret_cast<const f32x4*>(bias + e);
  u32x2 o;
  o[0] = pack_bf16x2(__builtin_fmaf(sum[0], sc[0], bv[0]), __builtin_fmaf(sum[1], sc[1], bv[1]));
  o[1] = pack_bf16x2(__builtin_fmaf(sum[2], sc[2], bv[2]), __builtin_fmaf(sum[3], sc[3], bv[3]));
  reinterpret_cast<u32x2*>(out)[q] = o;
}

// Depth ranges: with fewer output tiles than CUs, as many ranges as fill the
// CUs once, of at least four steps each (at most 16 ranges).
struct SplitPlan {
  bool r192;
  int S, spl;
};
SplitPlan plan_split(int64_t m, int64_t e, int64_t depth) {
  SplitPlan p{};
  p.r192 = use_r192(m, e);
  const int64_t RA = p.r192 ? 192 : 256;
  const int64_t tiles = (m + RB - 1) / RB * ((e + RA - 1) / RA), cus = get_num_cus();
  const int64_t nk = (depth + 63) / 64;
  int64_t S = 1;
  if (tiles > 0 && tiles < cus) {
    S = cus / tiles;
    if (S > nk / 4) S = nk / 4;
    if (S > 16) S = 16;
    if (S < 1) S = 1;
  }
  int64_t spl = (nk + S - 1) / S;
  spl = (spl + NBUF - 1) / NBUF * NBUF;
  p.spl = (int)spl;
  p.S = (int)((nk + spl - 1) / spl);  // every range holds at least one step
  return p;
}


template <bool BWD, bool SPLIT>
hipError_t run_fmt(hipStream_t st, int fmt, bool r192, const GemmArgs& a) {
  if (fmt == LRQ_FMT_INT4)
    return r192 ? run<BWD, LRQ_FMT_INT4, true, SPLIT>(st, a) : run<BWD, LRQ_FMT_INT4, false, SPLIT>(st, a);
  if (fmt == LRQ_FMT_INT8)
    return r192 ? run<BWD, LRQ_FMT_INT8, true, SPLIT>(st, a) : run<BWD, LRQ_FMT_INT8, false, SPLIT>(st, a);
  return r192 ? run<BWD, LRQ_FMT_FP8, true, SPLIT>(st, a) : run<BWD, LRQ_FMT_FP8, false, SPLIT>(st, a);
}

// Which GEMM kernel a shape takes: the 256-token tiles above (split in
// depth when they are too few), or lrq_gemm_mid.hip's 64-row tiles of 64 or
// 128 tokens over the whole depth, two workgroups per CU. The choice is the
// smaller modelled time, in microseconds, with constants measured on MI355X
// (fwd and input gradient of the C1, C3, C5 and north-star shapes, every
// path forced in turn):
//   - a 256 x 256 x 64 step of the large tiles takes 1.86 us (0.8 of that
//     for 192-row tiles); a split shape adds its f32 partials, written and
//     read once at about 4 TB/s, and the reduction launch;
//   - a 64-wide depth block of a mid tile takes MID_T1 us when its
//     workgroup has the CU to itself and MID_T2 us each when two share it
//     (64 tokens: 0.342 / 0.423, 128 tokens: 0.441 / 0.696); the tiles are
//     dealt over the CUs, two at a time;
//   - a mid tile may split its depth into S <= MID_MAX_SPLIT ranges (one
//     workgroup each, whole rounds of MID_MST stages) when its tiles leave
//     CUs idle; the ranges' accumulators meet in the launch, about
//     MID_FINISH_US more, and S > 1 must model at least a tenth faster.
constexpr double LARGE_STEP_US = 1.86;
// per variant MID_64, MID_128: tile tokens, block us alone and shared, and
// a fixed cost per round of tiles
constexpr int MID_T[3] = {0, 64, 128};
constexpr double MID_T1[3] = {0, 0.342, 0.441}, MID_T2[3] = {0, 0.423, 0.696};
constexpr double MID_FIX[3] = {0, 2.0, 2.0};
constexpr int MID_SD[3] = {0, 2, 1};  // 64-deep blocks per pipeline stage
constexpr double MID_FINISH_US = 5.0;
// lrq_debug_gemm_path: 0 planned, 1 large tiles, 2 + (variant - 1) a mid
// variant, 4 + (variant - 1) a mid variant with at least two depth ranges
// where the depth has them
int g_gemm_path = 0;

double large_us(int64_t m, int64_t e, int64_t depth) {
  const SplitPlan p = plan_split(m, e, depth);
  const int64_t cus = get_num_cus();
  const int64_t RA = p.r192 ? 192 : 256;
  const int64_t tiles = (m + RB - 1) / RB * ((e + RA - 1) / RA);
  const double f = p.r192 ? 0.8 : 1.0;
  if (p.S <= 1) return (double)((tiles + cus - 1) / cus) * (double)((depth + 63) / 64) * LARGE_STEP_US * f + 3.0;
  const double part = 4.0 * (double)p.S * (double)m * (double)e;
  return (double)p.spl * LARGE_STEP_US * f + 2.0 * part / 4.0e6 + 8.0;
}

// stages per range (whole rounds) for S ranges of a depth, and the ranges
// that gives
int mid_spl(int64_t depth, int v, int S) {
  const int64_t nst = ((depth + 63) / 64 + MID_SD[v] - 1) / MID_SD[v];
  return (int)(((nst + S - 1) / S + MID_MST - 1) / MID_MST * MID_MST);
}
int mid_ranges(int64_t depth, int v, int S) {
  const int64_t nst = ((depth + 63) / 64 + MID_SD[v] - 1) / MID_SD[v];
  const int spl = mid_spl(depth, v, S);
  return (int)((nst + spl - 1) / spl);
}

double mid_us(int64_t m, int64_t e, int64_t depth, int v, int S = 1) {
  const int64_t T = MID_T[v], cus = get_num_cus();
  const int64_t tiles = (m + T - 1) / T * ((e + 63) / 64) * S;
  const int64_t n = (tiles + cus - 1) / cus;
  const int64_t nb = S > 1 ? std::min<int64_t>((int64_t)mid_spl(depth, v, S) * MID_SD[v], (depth + 63) / 64)
                           : (depth + 63) / 64;
  return (double)nb * ((double)(n / 2) * MID_T2[v] + (double)(n % 2) * MID_T1[v]) +
         MID_FIX[v] * (double)((n + 1) / 2) + (S > 1 ? MID_FINISH_US : 0.0);
}

struct MidChoice {
  int v, S, spl;
  double us;
};

// the best number of depth ranges for variant v (forced: at least two
// where the depth has them)
MidChoice mid_best_split(int64_t m, int64_t e, int64_t depth, int v, bool force_split) {
  MidChoice best{v, 1, 0, mid_us(m, e, depth, v, 1)};
  MidChoice alt{v, 1, 0, 1e30};
  for (int S = 2; S <= MID_MAX_SPLIT; ++S) {
    const int R = mid_ranges(depth, v, S);
    if (R < 2 || R != S) continue;  // (S that rounding turns into fewer ranges are covered by those)
    const double t = mid_us(m, e, depth, v, S);
    if (t < alt.us) alt = MidChoice{v, S, mid_spl(depth, v, S), t};
  }
  if (alt.S > 1 && (force_split || alt.us < 0.9 * best.us)) return alt;
  return best;
}

// the mid variant and its depth ranges a shape takes (v = MID_NONE: the
// large tiles)
MidChoice mid_choice(int64_t m, int64_t e, int64_t depth) {
  const MidChoice none{MID_NONE, 1, 0, 0.0};
  if (m <= 0 || e <= 0 || g_gemm_path == 1) return none;
  if (g_gemm_path >= 2) return mid_best_split(m, e, depth, (g_gemm_path - 2) % 2 + 1, g_gemm_path >= 4);
  MidChoice pick = none;
  pick.us = large_us(m, e, depth);
  for (int v : {MID_64, MID_128}) {
    const MidChoice c = mid_best_split(m, e, depth, v, false);
    if (c.us < pick.us) pick = c;
  }
  return pick;
}

// MID_NONE (the large tiles) or the mid variant a shape takes
int mid_plan(int64_t m, int64_t e, int64_t depth) { return mid_choice(m, e, depth).v; }

template <bool BWD>
hipError_t dispatch(hipStream_t st, int fmt, const GemmArgs& a) {
  if (a.m == 0 || a.e == 0) return hipSuccess;
  const MidChoice mc = mid_choice(a.m, a.e, a.l);
  if (mc.v != MID_NONE) {
    if (mc.S <= 1) return launch_mid(st, fmt, BWD, a, mc.v);
    if (!a.part || !a.mcnt) return hipErrorInvalidValue;
    GemmArgs b = a;
    b.msplit = mc.S;
    b.mspl = mc.spl;
    return launch_mid(st, fmt, BWD, b, mc.v);
  }
  const SplitPlan p = plan_split(a.m, a.e, a.l);
  if (p.S <= 1) return run_fmt<BWD, false>(st, fmt, p.r192, a);
  if (!a.part) return hipErrorInvalidValue;
  GemmArgs b = a;
  b.splits = p.S;
  b.spl = p.spl;
  hipError_t err = run_fmt<BWD, true>(st, fmt, p.r192, b);
  if (err != hipSuccess) return err;
  // forward fp8: channel scales (or the scalar) and the bias in the reduction
  const bool f8 = !BWD && fmt == LRQ_FMT_FP8;
  const int64_t quads = a.m * a.e / 4;
  hipLaunchKernelGGL(k_split_reduce, dim3((unsigned)((quads + 255) / 256)), dim3(256), 0, st, a.part, p.S, a.m, a.e,
                     f8 ? a.wscale : nullptr, a.per_channel, BWD ? nullptr : a.bias, a.out);
  return hipGetLastError();
}

}  // namespace

int g_num_cus_ = 256;  // compute units of the context's device (the persistent grid)
void set_num_cus(int n) { g_num_cus_ = n > 0 ? n : 256; }
int get_num_cus() { return g_num_cus_; }

hipError_t launch_fwd(hipStream_t st, int fmt, const GemmArgs& a) { return dispatch<false>(st, fmt, a); }
MidSplit mid_split_plan(int64_t m, int64_t e, int64_t depth) {
  const MidChoice mc = mid_choice(m, e, depth);
  if (mc.v == MID_NONE || mc.S <= 1) return MidSplit{1, 0, 0, 0};
  const int64_t T = MID_T[mc.v], tiles = (m + T - 1) / T * ((e + 63) / 64);
  return MidSplit{mc.S, mc.spl, tiles, (int64_t)mc.S * tiles * T * 64};
}

int64_t gemm_split_floats(int64_t m, int64_t e, int64_t depth) {
  if (m <= 0 || e <= 0) return 0;
  if (mid_plan(m, e, depth)) return mid_split_plan(m, e, depth).floats;  // the mid tiles' depth ranges
  const SplitPlan p = plan_split(m, e, depth);
  return p.S > 1 ? (int64_t)p.S * m * e : 0;
}
hipError_t launch_bwd(hipStream_t st, int fmt, const GemmArgs& a) { return dispatch<true>(st, fmt, a); }
int gemm_mid_tokens(int64_t m, int64_t e, int64_t depth) { return MID_T[mid_plan(m, e, depth)]; }
void set_gemm_path(int path) { g_gemm_path = path; }
