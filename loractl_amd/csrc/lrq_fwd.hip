// Forward GEMM of the quantized LoRA linear for m > 16 tokens, with the
// weight operand dequantized straight into matrix-core registers:
//
//   y[m, n] = x[m, k] . bf16(dq(w))[n, k]^T (+bias) + t[m, :] . B[:, n]
//
// (src/quant.rs:175-176 for the base product, src/lora.rs:199-203 for the
// LoRA term; t = bf16(s . x . A) comes from the LoRA side kernels.)
//
// A workgroup of four wavefronts (one per SIMD) owns a 256 (n) x 256 (token)
// output tile. Wavefront w owns weight rows 64w .. 64w+63 of it for all 256
// tokens: 2 x 8 accumulator tiles of v_mfma_f32_32x32x16_bf16 (256 f32 per
// lane). The design keeps LDS traffic and dequantization work per
// matrix-core instruction small:
//   - weight (A role): each lane loads the packed bytes of its own row
//     straight from the blocked layout (int4: 16 bytes = 32 k of one row,
//     fp8: 32 bytes), dequantizes in registers to the exact bf16 operand
//     (int4 fma(u, s, -8s) == q*s, then bf16; fp8 the exact e4m3 value) and
//     feeds the matrix cores. The reduction index is permuted inside a
//     64-wide step: lane group g (lanes 32g .. 32g+31) takes k = 32g + 8kk ..
//     +8 in sub-step kk, so a lane's packed bytes are contiguous. No weight
//     row is shared between wavefronts, so each weight element is
//     dequantized once per workgroup, and the weight never passes LDS;
//   - activations (B role): the 256 x 64 x-tile of a step is copied global ->
//     LDS by buffer loads with an LDS destination (each wavefront moves 64
//     token rows) and read by all four wavefronts: 1/64 byte of LDS reads per
//     flop, half of what a shared dequantized weight tile would add;
//   - the pipeline: x tiles in NBUF LDS buffers, packed weights in NBUF
//     register sets, both NBUF-1 steps ahead. The one barrier of a step sits
//     between its third and fourth sub-steps, after the last fragment reads of
//     the current buffer: the fourth sub-step's matrix-core work then covers
//     the barrier and the next step's first fragment reads;
//   - edges: buffer loads past a resource's size return zeros (partial token
//     and weight tiles, the k tail, and the zero steps that pad the unrolled
//     loop); padding weight rows hold q = 0 with scale 0;
//   - epilogue: fp8 per-channel scales multiply the f32 accumulators (they
//     factor out of the k reduction), then the LoRA term is one more
//     rank-wide matrix-core step (B^T staged in LDS at the start, t from
//     global), then bias and 8-byte bf16 stores;
//   - workgroup ids are remapped so each XCD (own L2) works on a contiguous
//     range of tiles, grouped four token tiles deep.

#include "lrq_common.h"
#include "lrq_kernels.h"

namespace {

constexpr int BK = 64;              // reduction step
constexpr int NWV = 4;              // wavefronts per workgroup (one per SIMD)
constexpr int NIW = 2;              // 32-row weight tiles per wavefront
constexpr int MJ = 8;               // 32-token tiles per wavefront
constexpr int RA = NWV * NIW * 32;  // weight rows per workgroup (256)
constexpr int RB = MJ * 32;         // tokens per workgroup (256)
constexpr int XBUF = RB * BK;       // bf16 per activation buffer (32 KB)
constexpr int LDL = 72;             // staged B^T row stride (bf16): 144-byte rows

// activation LDS tile [256 rows][64] bf16: 128-byte rows, 16-byte chunk c of
// row r at chunk c ^ swz(r), so the 16 lanes of a read pass (16 rows at one
// logical chunk) cover all 64 banks
LRQ_DEV int swz(int r) { return (r >> 1) & 7; }

template <int FMT, int NBUF>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
k_fwd(GemmArgs a, int tiles_m) {
  constexpr bool I4 = FMT == LRQ_FMT_INT4;
  constexpr int WV = I4 ? 1 : 2;  // 16-byte packed loads per row tile per step
  __shared__ __attribute__((aligned(16))) uint16_t sX0[XBUF];
  __shared__ __attribute__((aligned(16))) uint16_t sX1[XBUF];
  __shared__ __attribute__((aligned(16))) uint16_t sX2[NBUF > 2 ? XBUF : 8];
  __shared__ __attribute__((aligned(16))) uint16_t sB[RA * LDL];  // B^T [256 n][rp]

  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int tiles_a = gridDim.x / tiles_m;
  constexpr int GM = 4;
  const int grp = logical / (GM * tiles_a), within = logical % (GM * tiles_a);
  const int gm = min(GM, tiles_m - grp * GM);
  const int tm = grp * GM + within % gm, ta = within / gm;
  const int64_t m0 = (int64_t)tm * RB, e0 = (int64_t)ta * RA;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int64_t M = a.m, K = a.l, E = a.e;

  // ---------------- B^T staging for the LoRA step (read after the main loop)
  const int rp = a.rp, r = a.r;
  if (rp > 0) {
    // B[j][e0 + c*8 .. +8] -> sB[(c*8 + q) * LDL + j]
    constexpr int cpr = RA / 8;
    for (int id = tid; id < rp * cpr; id += 256) {
      const int j = id / cpr, c = id % cpr;
      const int64_t n = e0 + c * 8;
      u32x4 v = zero4();
      if (j < r && n < E) v = ld16(a.lw + (int64_t)j * E + n);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        sB[(c * 8 + 2 * q) * LDL + j] = (uint16_t)(v[q] & 0xffffu);
        sB[(c * 8 + 2 * q + 1) * LDL + j] = (uint16_t)(v[q] >> 16);
      }
    }
  }

  // ---------------- activation DMA: wavefront w moves token rows 64w .. +64
  // 8 buffer loads per step; lane l of load c lands at row 64w + 8c + l/8,
  // physical chunk l%8, and fetches logical chunk (l%8) ^ swz(row), where
  // swz(64w + 8c + l/8) = (4c + l/16) & 7 alternates with the parity of c.
  const int64_t mw = m0 + 64 * w;
  const int64_t mrows = (M - mw) < 64 ? (M - mw) : 64;
  const rsrc_t ract = make_rsrc(a.act + (mw < M ? mw : 0) * K, clamp_bytes(mrows * K * 2));
  const int drow = lane >> 3;
  const int dq0 = (lane & 7) ^ ((lane >> 4) & 7), dq1 = (lane & 7) ^ (((lane >> 4) + 4) & 7);
  const uint32_t doff0 = (uint32_t)((drow * K + dq0 * 8) * 2), doff1 = (uint32_t)((drow * K + dq1 * 8) * 2);
  auto dma = [&](uint16_t* buf, int kt) {
    const int64_t k0 = (int64_t)kt * BK;
    const bool kok0 = k0 + dq0 * 8 < K, kok1 = k0 + dq1 * 8 < K;  // K % 8 == 0
    const uint32_t koff = (uint32_t)(k0 * 2);
    __attribute__((address_space(3))) char* base =
        (__attribute__((address_space(3))) char*)(lds_void*)(buf + 64 * w * BK);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const bool kok = (c & 1) ? kok1 : kok0;
      const uint32_t doff = (c & 1) ? doff1 : doff0;
      const uint32_t off = opaque_u32(kok ? doff + (uint32_t)(c * 8 * K * 2) + koff : LRQ_OOB);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ract, (lds_void*)(base + c * 8 * BK * 2), 16, off, 0, 0, 0);
    }
  };
  // B-role fragment of token tile j in sub-step kk: row 32j + l32, logical
  // chunk 4g + kk, stored at chunk (4g + kk) ^ swz(l32) (swz(32j + l32) =
  // swz(l32)). The four per-lane chunk bases are fixed; tile and buffer
  // offsets are immediates of the LDS read.
  const uint32_t xrow = (uint32_t)(l32 * BK * 2) | (uint32_t)(swz(l32) * 16);
  uint32_t xk[4];
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) xk[kk] = opaque_u32(xrow ^ (uint32_t)((4 * g + kk) * 16));
  auto xfrag = [&](const uint16_t* buf, int j, int kk) -> bf16x8 {
    return as_bf16x8(ld16(reinterpret_cast<const char*>(buf) + xk[kk] + (uint32_t)(j * 32 * BK * 2)));
  };

  // ---------------- weight: this wavefront's block row of the blocked layout
  const int64_t KB = (K + 63) / 64;
  constexpr uint32_t blkb = I4 ? 2048u : 4096u;  // bytes per 64x64 block
  constexpr uint32_t rowb = I4 ? 32u : 64u;      // bytes per block row
  const uint32_t Gp = I4 ? (uint32_t)((KB * 64) >> a.gshift) : 0u;
  int64_t wbytes, nsc;
  blocked_sizes_dev(FMT, E, K, &wbytes, &nsc, a.gshift);
  const int64_t nb = e0 / 64 + w;
  const rsrc_t rw = make_rsrc(a.wdata + nb * KB * blkb, clamp_bytes(wbytes - nb * KB * blkb));
  const rsrc_t rs = make_rsrc(a.wscale + (I4 ? nb * Gp * 64 : 0), I4 ? clamp_bytes((nsc - nb * Gp * 64) * 4) : 0u);
  // lane offsets: row tile i at row 32i + l32 of the block, lane group g's
  // 16 (int4) or 32 (fp8) bytes
  const uint32_t woff = (uint32_t)l32 * rowb + (uint32_t)g * (I4 ? 16u : 32u);
  const uint32_t soff = (uint32_t)l32 * 4u;
  const int nk = (int)KB;

  u32x4 wp[NBUF][NIW * WV];  // packed weight bytes per register set
  float wsc[NBUF][NIW];      // int4 group scales per register set
  auto load_w = [&](int set, int kt) {
    // steps past the last one read zeros (bytes and scales): they add nothing
    const uint32_t kb = opaque_u32(kt < nk ? (uint32_t)kt * blkb : LRQ_OOB);
#pragma unroll
    for (int i = 0; i < NIW; ++i)
#pragma unroll
      for (int h = 0; h < WV; ++h) wp[set][i * WV + h] = bload16(rw, kb + woff + (uint32_t)i * 32u * rowb + 16u * h);
    if (I4) {
      const uint32_t j = ((uint32_t)kt * 64u + (uint32_t)g * 32u) >> a.gshift;
      const uint32_t so = opaque_u32(kt < nk ? (j * 64u) * 4u + soff : LRQ_OOB);
#pragma unroll
      for (int i = 0; i < NIW; ++i) wsc[set][i] = bloadf(rs, so + (uint32_t)i * 128u);
    }
  };
  // A-role fragment of row tile i, sub-step kk, from register set `set`
  auto wfrag = [&](int set, int i, int kk) -> bf16x8 {
    if (I4) return as_bf16x8(dequant8_int4_bf16(wp[set][i][kk], wsc[set][i], a.nib));
    const u32x4 v = wp[set][i * WV + (kk >> 1)];
    const u32x2 lo = fp8x4_to_bf16(v[2 * (kk & 1)]), hi = fp8x4_to_bf16(v[2 * (kk & 1) + 1]);
    return as_bf16x8((u32x4){lo[0], lo[1], hi[0], hi[1]});
  };

  f32x16 acc[NIW][MJ];
#pragma unroll
  for (int i = 0; i < NIW; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  uint16_t* const bufs[3] = {sX0, sX1, sX2};
  bf16x8 fa[2][NIW], fb[2][MJ];

  // One step on LDS buffer `b` and register set `b` (b = kt % NBUF; the
  // unrolled loop makes both static). On entry fa[0] and fb[0] hold sub-step
  // 0's fragments; on exit they hold the next step's.
  auto step = [&](const int b, const int kt) {
    const uint16_t* buf = bufs[b];
    const int nb_ = (b + 1) % NBUF;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int cur = kk & 1;
      if (kk < 3) {
#pragma unroll
        for (int j = 0; j < MJ; ++j) fb[cur ^ 1][j] = xfrag(buf, j, kk + 1);
#pragma unroll
        for (int i = 0; i < NIW; ++i) fa[cur ^ 1][i] = wfrag(b, i, kk + 1);
      } else {
        // every read of buffer b is issued: one barrier, then refill it
        // (NBUF steps ahead) and register set b, and read the next step's
        // first fragments from buffer nb_ while sub-step 3 runs
        __syncthreads();
        dma(bufs[b], kt + NBUF);
        load_w(b, kt + NBUF);
#pragma unroll
        for (int j = 0; j < MJ; ++j) fb[cur ^ 1][j] = xfrag(bufs[nb_], j, 0);
#pragma unroll
        for (int i = 0; i < NIW; ++i) fa[cur ^ 1][i] = wfrag(nb_, i, 0);
      }
#pragma unroll
      for (int i = 0; i < NIW; ++i)
#pragma unroll
        for (int j = 0; j < MJ; ++j) acc[i][j] = mfma32(fa[cur][i], fb[cur][j], acc[i][j]);
    }
  };

  // prologue: NBUF steps of x and packed weights in flight
#pragma unroll
  for (int b = 0; b < NBUF; ++b) {
    dma(bufs[b], b);
    load_w(b, b);
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < MJ; ++j) fb[0][j] = xfrag(bufs[0], j, 0);
#pragma unroll
  for (int i = 0; i < NIW; ++i) fa[0][i] = wfrag(0, i, 0);

  for (int kt = 0; kt < nk; kt += NBUF) {
#pragma unroll
    for (int b = 0; b < NBUF; ++b) step(b, kt + b);
  }

  // drain the look-ahead copies before the epilogue reads LDS
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // fp8 forward: the per-output-channel scale factors out of the k reduction
  if (!I4) {
#pragma unroll
    for (int i = 0; i < NIW; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t n = e0 + 64 * w + 32 * i + 8 * (v >> 2) + 4 * g + (v & 3);
        const float s = (n < E) ? (a.per_channel ? a.wscale[n] : a.wscale[0]) : 0.0f;
#pragma unroll
        for (int j = 0; j < MJ; ++j) acc[i][j][v] *= s;
      }
  }

  // LoRA: one rank-wide step; A role = B^T rows from LDS, B role = t [M, rp]
  // (zero-padded, pre-scaled) from global
  if (rp > 0) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk * 16 < rp) {
        bf16x8 la[NIW];
#pragma unroll
        for (int i = 0; i < NIW; ++i)
          la[i] = as_bf16x8(ld16(sB + (64 * w + 32 * i + l32) * LDL + kk * 16 + g * 8));
#pragma unroll
        for (int j = 0; j < MJ; ++j) {
          const int64_t m = m0 + 32 * j + l32;
          const u32x4 v = ld16(a.lact + (m < M ? m : (M - 1)) * rp + kk * 16 + g * 8);
          const bf16x8 lb = as_bf16x8(m < M ? v : zero4());
#pragma unroll
          for (int i = 0; i < NIW; ++i) acc[i][j] = mfma32(la[i], lb, acc[i][j]);
        }
      }
    }
  }

  // epilogue: lane holds 4 consecutive n of one token per accumulator group
#pragma unroll
  for (int i = 0; i < NIW; ++i) {
#pragma unroll
    for (int vg = 0; vg < 4; ++vg) {
      const int64_t n = e0 + 64 * w + 32 * i + 8 * vg + 4 * g;
      if (n >= E) continue;
      f32x4 bv = {0.0f, 0.0f, 0.0f, 0.0f};
      if (a.bias) bv = *reinterpret_cast<const f32x4*>(a.bias + n);
#pragma unroll
      for (int j = 0; j < MJ; ++j) {
        const int64_t m = m0 + 32 * j + l32;
        if (m < M) {
          u32x2 o;
          o[0] = pack_bf16x2(acc[i][j][4 * vg + 0] + bv[0], acc[i][j][4 * vg + 1] + bv[1]);
          o[1] = pack_bf16x2(acc[i][j][4 * vg + 2] + bv[2], acc[i][j][4 * vg + 3] + bv[3]);
          *reinterpret_cast<u32x2*>(a.out + m * E + n) = o;
        }
      }
    }
  }
}

template <int FMT, int NBUF>
hipError_t run(hipStream_t st, const GemmArgs& a) {
  const int tiles_m = (int)((a.m + RB - 1) / RB);
  const int tiles_e = (int)((a.e + RA - 1) / RA);
  hipLaunchKernelGGL((k_fwd<FMT, NBUF>), dim3(tiles_m * tiles_e), dim3(256), 0, st, a, tiles_m);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_fwd(hipStream_t st, int fmt, const GemmArgs& a) {
  if (a.m == 0 || a.e == 0) return hipSuccess;
  return fmt == LRQ_FMT_INT4 ? run<LRQ_FMT_INT4, 2>(st, a) : run<LRQ_FMT_FP8, 2>(st, a);
}
