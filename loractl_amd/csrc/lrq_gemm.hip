// The two fused GEMMs of the quantized LoRA linear on gfx950 matrix cores.
//
//   forward   y[m, n]  = x[m, k] . bf16(dq(w))[n, k]^T  (+bias)  + t[m, :] . bt[n, :]^T
//   backward dx[m, k]  = dy[m, n] . bf16(dq(w))[n, k]          + u[m, :] . ap[k, :]^T
//
// (src/quant.rs:175-176 and :229-233 for the base products; the LoRA terms
// are the two small products of src/lora.rs:199-203 and their autodiff,
// with t = s.x.A and u = s.dy.B^T computed by the skinny kernels.)
//
// Design (one workgroup of 4 wavefronts per CU, 2x2 wave grid):
//   - the packed weight is read straight from HBM/L2 in its packed form and
//     dequantized in registers into an LDS tile of bf16; a bf16 copy of the
//     weight never exists in HBM, in either pass;
//   - activations are staged into LDS with 16-byte loads;
//   - LDS is double-buffered and the next tile's global loads are issued
//     before the current tile's matrix-core work, one barrier per k-step;
//   - v_mfma_f32_32x32x16_bf16 with the weight as the A-role operand, so each
//     lane's accumulators hold 4 consecutive output features of one token and
//     the epilogue writes 8-byte runs;
//   - the LoRA term is one more (rank-wide) k-step over LDS after the main
//     loop, so x.A is never recomputed per output tile;
//   - fp8 per-output-channel scales factor out of the forward reduction and
//     are applied to the f32 accumulators; int4 group scales vary along k
//     and are applied during dequantization (exactly: fma(u, s, -8s) == q*s);
//   - in the backward the reduction runs along n while the packed weight is
//     contiguous along k, so each thread dequantizes an 8x8 block and writes
//     it transposed into LDS (XOR-swizzled 16-byte chunks against bank
//     conflicts);
//   - workgroup ids are remapped so each XCD (own L2) works on a contiguous
//     range of tiles.
#include "lrq_common.h"
#include "lrq_kernels.h"

namespace {

constexpr int BK = 64;       // reduction step
constexpr int LD = BK + 8;   // LDS row stride in bf16 (144 bytes)
constexpr int NT = 256;      // threads per workgroup

LRQ_DEV int xcd_remap(int bid, int nblk) {
  const int q = nblk / 8, r = nblk % 8;
  const int x = bid % 8, i = bid / 8;
  return x * q + min(x, r) + i;
}

// ------------------------------------------------------------------ forward
template <int FMT, int NI, int MJ>
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 1)))
k_fwd_main(FwdArgs a, int tiles_m) {
  constexpr int RA = 64 * NI;  // weight rows (n) per tile
  constexpr int RB = 64 * MJ;  // token rows (m) per tile
  constexpr int BUF = (RA + RB) * LD;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * BUF];

  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int tm = logical % tiles_m, tn = logical / tiles_m;
  const int64_t m0 = (int64_t)tm * RB, n0 = (int64_t)tn * RA;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wa = wave >> 1, wb = wave & 1;
  const int64_t M = a.m, N = a.n, K = a.k;

  // X loader: chunk c covers row c*32 + tid/8, 8 bf16 at column (tid%8)*8
  constexpr int XC = RB / 32;
  const int xrow = tid >> 3, xcol = (tid & 7) * 8;
  const uint16_t* xbase = a.x + (m0 + xrow) * K + xcol;
  // W loader
  constexpr int WPR = (FMT == LRQ_FMT_INT4) ? 2 : 4;  // 16-byte chunks per weight row per k-step
  constexpr int WC = (RA * WPR + NT - 1) / NT;
  const int kgroups = (FMT == LRQ_FMT_INT4) ? (int)(K / a.group) : 0;

  u32x4 xr[XC];
  u32x4 wr[WC];
  float wsc[WC];

  auto gload = [&](int64_t k0) {
#pragma unroll
    for (int c = 0; c < XC; ++c) {
      const bool ok = (m0 + c * 32 + xrow < M) && (k0 + xcol < K);
      xr[c] = ld16_pred(xbase + (int64_t)c * 32 * K + k0, ok);
    }
#pragma unroll
    for (int c = 0; c < WC; ++c) {
      const int id = tid + NT * c;
      const int row = id / WPR, part = id % WPR;
      const int64_t n = n0 + row;
      if (FMT == LRQ_FMT_INT4) {
        const int64_t kk = k0 + part * 32;
        const bool ok = (id < RA * WPR) && (n < N) && (kk < K);
        wr[c] = ld16_pred(a.wdata + n * (K / 2) + kk / 2, ok);
        wsc[c] = ok ? a.wscale[n * kgroups + kk / a.group] : 0.0f;
      } else {
        const int64_t kk = k0 + part * 16;
        const bool ok = (id < RA * WPR) && (n < N) && (kk < K);
        wr[c] = ld16_pred(a.wdata + n * K + kk, ok);
      }
    }
  };

  auto lstore = [&](int buf) {
    uint16_t* sA = lds + buf * BUF;
    uint16_t* sB = sA + RA * LD;
#pragma unroll
    for (int c = 0; c < XC; ++c) st16(sB + (c * 32 + xrow) * LD + xcol, xr[c]);
#pragma unroll
    for (int c = 0; c < WC; ++c) {
      const int id = tid + NT * c;
      if (id < RA * WPR) {
        const int row = id / WPR, part = id % WPR;
        if (FMT == LRQ_FMT_INT4) {
          uint16_t* dst = sA + row * LD + part * 32;
#pragma unroll
          for (int d = 0; d < 4; ++d) st16(dst + d * 8, dequant8_int4_bf16(wr[c][d], wsc[c]));
        } else {
          uint16_t* dst = sA + row * LD + part * 16;
          u32x2 p0 = fp8x4_to_bf16(wr[c][0]), p1 = fp8x4_to_bf16(wr[c][1]);
          u32x2 p2 = fp8x4_to_bf16(wr[c][2]), p3 = fp8x4_to_bf16(wr[c][3]);
          u32x4 o0 = {p0[0], p0[1], p1[0], p1[1]};
          u32x4 o1 = {p2[0], p2[1], p3[0], p3[1]};
          st16(dst, o0);
          st16(dst + 8, o1);
        }
      }
    }
  };

  f32x16 acc[NI][MJ];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int arow = wa * (NI * 32) + (lane & 31);
  const int brow = wb * (MJ * 32) + (lane & 31);
  const int kq = (lane >> 5) * 8;

  auto compute = [&](int buf, int nsub) {
    const uint16_t* sA = lds + buf * BUF;
    const uint16_t* sB = sA + RA * LD;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk < nsub) {
        bf16x8 fa[NI], fb[MJ];
#pragma unroll
        for (int i = 0; i < NI; ++i) fa[i] = as_bf16x8(ld16(sA + (arow + i * 32) * LD + kk * 16 + kq));
#pragma unroll
        for (int j = 0; j < MJ; ++j) fb[j] = as_bf16x8(ld16(sB + (brow + j * 32) * LD + kk * 16 + kq));
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
          for (int j = 0; j < MJ; ++j) acc[i][j] = mfma32(fa[i], fb[j], acc[i][j]);
      }
    }
  };

  const int nk = (int)((K + BK - 1) / BK);
  gload(0);
  lstore(0);
  if (nk > 1) gload(BK);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) lstore(cur ^ 1);
    if (kt + 2 < nk) gload((int64_t)(kt + 2) * BK);
    compute(cur, 4);
    __syncthreads();
  }

  // fp8: the per-output-channel scale factors out of the k reduction
  if (FMT == LRQ_FMT_FP8) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int64_t n = n0 + wa * (NI * 32) + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        const float s = (n < N) ? (a.per_channel ? a.wscale[n] : a.wscale[0]) : 0.0f;
#pragma unroll
        for (int j = 0; j < MJ; ++j) acc[i][j][v] *= s;
      }
  }

  // LoRA: one rank-wide k-step, t [m, rp] against bt [n, rp]
  if (a.rp > 0) {
    uint16_t* sA = lds;
    uint16_t* sB = lds + RA * LD;
    const int cpr = a.rp / 8;
    for (int id = tid; id < RB * cpr; id += NT) {
      const int row = id / cpr, ch = id % cpr;
      const int64_t m = m0 + row;
      st16(sB + row * LD + ch * 8, ld16_pred(a.t + m * a.rp + ch * 8, m < M));
    }
    for (int id = tid; id < RA * cpr; id += NT) {
      const int row = id / cpr, ch = id % cpr;
      const int64_t n = n0 + row;
      st16(sA + row * LD + ch * 8, ld16_pred(a.bt + n * a.rp + ch * 8, n < N));
    }
    __syncthreads();
    compute(0, a.rp / 16);
  }

  // epilogue: lane holds 4 consecutive n for one m per (i, j, v>>2)
#pragma unroll
  for (int i = 0; i < NI; ++i) {
#pragma unroll
    for (int vg = 0; vg < 4; ++vg) {
      const int64_t n = n0 + wa * (NI * 32) + i * 32 + 8 * vg + 4 * (lane >> 5);
      if (n >= N) continue;
      f32x4 bv = {0.0f, 0.0f, 0.0f, 0.0f};
      if (a.bias) bv = *reinterpret_cast<const f32x4*>(a.bias + n);
#pragma unroll
      for (int j = 0; j < MJ; ++j) {
        const int64_t m = m0 + wb * (MJ * 32) + j * 32 + (lane & 31);
        if (m < M) {
          u32x2 o;
          o[0] = pack_bf16x2(acc[i][j][4 * vg + 0] + bv[0], acc[i][j][4 * vg + 1] + bv[1]);
          o[1] = pack_bf16x2(acc[i][j][4 * vg + 2] + bv[2], acc[i][j][4 * vg + 3] + bv[3]);
          *reinterpret_cast<u32x2*>(a.y + m * N + n) = o;
        }
      }
    }
  }
}

// ------------------------------------------------------------------ backward dx
template <int FMT, int NI, int MJ>
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 1)))
k_bwd_dx(BwdArgs a, int tiles_m) {
  constexpr int RA = 64 * NI;  // output k columns per tile (A-role rows)
  constexpr int RB = 64 * MJ;  // token rows per tile
  constexpr int BUF = (RA + RB) * LD;
  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * BUF];

  const int logical = xcd_remap(blockIdx.x, gridDim.x);
  const int tm = logical % tiles_m, tk = logical / tiles_m;
  const int64_t m0 = (int64_t)tm * RB, kq0 = (int64_t)tk * RA;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wa = wave >> 1, wb = wave & 1;
  const int64_t M = a.m, N = a.n, K = a.k;

  // dY loader (reduction dim n contiguous), same mapping as the forward X loader
  constexpr int XC = RB / 32;
  const int xrow = tid >> 3, xcol = (tid & 7) * 8;
  const uint16_t* ybase = a.dy + (m0 + xrow) * N + xcol;
  // W loader: 8 (n) x 8 (k) blocks; RA/8 k-chunks x 8 n-chunks per k-step
  constexpr int KCH = RA / 8;
  constexpr int WC = (8 * KCH + NT - 1) / NT;
  const int kgroups = (FMT == LRQ_FMT_INT4) ? (int)(K / a.group) : 0;

  u32x4 yr[XC];
  uint32_t wr[WC][FMT == LRQ_FMT_INT4 ? 8 : 16];
  float wsc[WC][8];

  auto gload = [&](int64_t nb) {
#pragma unroll
    for (int c = 0; c < XC; ++c) {
      const bool ok = (m0 + c * 32 + xrow < M) && (nb + xcol < N);
      yr[c] = ld16_pred(ybase + (int64_t)c * 32 * N + nb, ok);
    }
#pragma unroll
    for (int c = 0; c < WC; ++c) {
      const int id = tid + NT * c;
      const int kc = id % KCH, nc = id / KCH;
      const int64_t k = kq0 + kc * 8;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int64_t n = nb + nc * 8 + i;
        const bool ok = (id < 8 * KCH) && (n < N) && (k < K);
        if (FMT == LRQ_FMT_INT4) {
          wr[c][i] = ok ? *reinterpret_cast<const uint32_t*>(a.wdata + n * (K / 2) + k / 2) : 0x88888888u;
          wsc[c][i] = ok ? a.wscale[n * kgroups + k / a.group] : 0.0f;
        } else {
          u32x2 v = {0u, 0u};
          if (ok) v = *reinterpret_cast<const u32x2*>(a.wdata + n * K + k);
          wr[c][2 * i] = v[0];
          wr[c][2 * i + 1] = v[1];
          wsc[c][i] = ok ? (a.per_channel ? a.wscale[n] : a.wscale[0]) : 0.0f;
        }
      }
    }
  };

  auto lstore = [&](int buf) {
    uint16_t* sA = lds + buf * BUF;
    uint16_t* sB = sA + RA * LD;
#pragma unroll
    for (int c = 0; c < XC; ++c) st16(sB + (c * 32 + xrow) * LD + xcol, yr[c]);
#pragma unroll
    for (int c = 0; c < WC; ++c) {
      const int id = tid + NT * c;
      if (id < 8 * KCH) {
        const int kc = id % KCH, nc = id / KCH;
        float f[8][8];  // [n row i][k offset]
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (FMT == LRQ_FMT_INT4) {
            dequant8_int4_f32(wr[c][i], wsc[c][i], f[i]);
          } else {
            fp8x4_to_f32(wr[c][2 * i], f[i]);
            fp8x4_to_f32(wr[c][2 * i + 1], f[i] + 4);
#pragma unroll
            for (int j = 0; j < 8; ++j) f[i][j] *= wsc[c][i];
          }
        }
#pragma unroll
        for (int kk = 0; kk < 8; ++kk) {
          const int R = kc * 8 + kk;
          const int phys = nc ^ ((R >> 3) & 7);
          u32x4 o;
          o[0] = pack_bf16x2(f[0][kk], f[1][kk]);
          o[1] = pack_bf16x2(f[2][kk], f[3][kk]);
          o[2] = pack_bf16x2(f[4][kk], f[5][kk]);
          o[3] = pack_bf16x2(f[6][kk], f[7][kk]);
          st16(sA + R * LD + phys * 8, o);
        }
      }
    }
  };

  f32x16 acc[NI][MJ];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < MJ; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

  const int arow = wa * (NI * 32) + (lane & 31);
  const int brow = wb * (MJ * 32) + (lane & 31);
  const int kq = (lane >> 5) * 8;

  auto compute = [&](int buf, int nsub) {
    const uint16_t* sA = lds + buf * BUF;
    const uint16_t* sB = sA + RA * LD;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      if (kk < nsub) {
        bf16x8 fa[NI], fb[MJ];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const int R = arow + i * 32;
          const int phys = (kk * 2 + (lane >> 5)) ^ ((R >> 3) & 7);
          fa[i] = as_bf16x8(ld16(sA + R * LD + phys * 8));
        }
#pragma unroll
        for (int j = 0; j < MJ; ++j) fb[j] = as_bf16x8(ld16(sB + (brow + j * 32) * LD + kk * 16 + kq));
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
          for (int j = 0; j < MJ; ++j) acc[i][j] = mfma32(fa[i], fb[j], acc[i][j]);
      }
    }
  };

  const int nk = (int)((N + BK - 1) / BK);
  gload(0);
  lstore(0);
  if (nk > 1) gload(BK);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) lstore(cur ^ 1);
    if (kt + 2 < nk) gload((int64_t)(kt + 2) * BK);
    compute(cur, 4);
    __syncthreads();
  }

  // LoRA: u [m, rp] against ap [k, rp] (A-role rows swizzled like the weight)
  if (a.rp > 0) {
    uint16_t* sA = lds;
    uint16_t* sB = lds + RA * LD;
    const int cpr = a.rp / 8;
    for (int id = tid; id < RB * cpr; id += NT) {
      const int row = id / cpr, ch = id % cpr;
      const int64_t m = m0 + row;
      st16(sB + row * LD + ch * 8, ld16_pred(a.u + m * a.rp + ch * 8, m < M));
    }
    for (int id = tid; id < RA * cpr; id += NT) {
      const int row = id / cpr, ch = id % cpr;
      const int64_t k = kq0 + row;
      const int phys = ch ^ ((row >> 3) & 7);
      st16(sA + row * LD + phys * 8, ld16_pred(a.ap + k * a.rp + ch * 8, k < K));
    }
    __syncthreads();
    compute(0, a.rp / 16);
  }

#pragma unroll
  for (int i = 0; i < NI; ++i) {
#pragma unroll
    for (int vg = 0; vg < 4; ++vg) {
      const int64_t k = kq0 + wa * (NI * 32) + i * 32 + 8 * vg + 4 * (lane >> 5);
      if (k >= K) continue;
#pragma unroll
      for (int j = 0; j < MJ; ++j) {
        const int64_t m = m0 + wb * (MJ * 32) + j * 32 + (lane & 31);
        if (m < M) {
          u32x2 o;
          o[0] = pack_bf16x2(acc[i][j][4 * vg + 0], acc[i][j][4 * vg + 1]);
          o[1] = pack_bf16x2(acc[i][j][4 * vg + 2], acc[i][j][4 * vg + 3]);
          *reinterpret_cast<u32x2*>(a.dx + m * K + k) = o;
        }
      }
    }
  }
}

// ------------------------------------------------------------------ dispatch
struct Cfg {
  int ni, mj;
  float penalty;
};
constexpr Cfg kCfgs[] = {{4, 4, 1.00f}, {3, 4, 1.08f}, {2, 4, 1.20f}, {2, 2, 1.60f}};

int g_num_cus = 256;

int pick_cfg(int64_t extent_a, int64_t m, int first = 0) {
  int best = first;
  double best_t = 1e300;
  for (int c = first; c < (int)(sizeof(kCfgs) / sizeof(kCfgs[0])); ++c) {
    const int64_t ta = (extent_a + 64 * kCfgs[c].ni - 1) / (64 * kCfgs[c].ni);
    const int64_t tb = (m + 64 * kCfgs[c].mj - 1) / (64 * kCfgs[c].mj);
    const int64_t tiles = ta * tb;
    const int64_t rounds = (tiles + g_num_cus - 1) / g_num_cus;
    const double t = (double)rounds * 64.0 * kCfgs[c].ni * 64.0 * kCfgs[c].mj * kCfgs[c].penalty;
    if (t < best_t - 1e-9) {
      best_t = t;
      best = c;
    }
  }
  return best;
}

template <int FMT, int NI, int MJ>
hipError_t run_fwd(hipStream_t st, const FwdArgs& a) {
  const int tiles_m = (int)((a.m + 64 * MJ - 1) / (64 * MJ));
  const int tiles_n = (int)((a.n + 64 * NI - 1) / (64 * NI));
  hipLaunchKernelGGL((k_fwd_main<FMT, NI, MJ>), dim3(tiles_m * tiles_n), dim3(NT), 0, st, a, tiles_m);
  return hipGetLastError();
}

template <int FMT, int NI, int MJ>
hipError_t run_bwd(hipStream_t st, const BwdArgs& a) {
  const int tiles_m = (int)((a.m + 64 * MJ - 1) / (64 * MJ));
  const int tiles_k = (int)((a.k + 64 * NI - 1) / (64 * NI));
  hipLaunchKernelGGL((k_bwd_dx<FMT, NI, MJ>), dim3(tiles_m * tiles_k), dim3(NT), 0, st, a, tiles_m);
  return hipGetLastError();
}

template <int FMT>
hipError_t fwd_fmt(hipStream_t st, const FwdArgs& a) {
  // fp8 forward: the 256- and 192-row weight tiles exceed the register file
  // (the epilogue channel scaling spills), so fp8 uses the 128-row tiles.
  const int first = (FMT == LRQ_FMT_FP8) ? 2 : 0;
  switch (pick_cfg(a.n, a.m, first)) {
    case 0: return run_fwd<FMT, (FMT == LRQ_FMT_FP8 ? 2 : 4), 4>(st, a);
    case 1: return run_fwd<FMT, (FMT == LRQ_FMT_FP8 ? 2 : 3), 4>(st, a);
    case 2: return run_fwd<FMT, 2, 4>(st, a);
    default: return run_fwd<FMT, 2, 2>(st, a);
  }
}

template <int FMT>
hipError_t bwd_fmt(hipStream_t st, const BwdArgs& a) {
  switch (pick_cfg(a.k, a.m)) {
    case 0: return run_bwd<FMT, 4, 4>(st, a);
    case 1: return run_bwd<FMT, 3, 4>(st, a);
    case 2: return run_bwd<FMT, 2, 4>(st, a);
    default: return run_bwd<FMT, 2, 2>(st, a);
  }
}

}  // namespace

void set_num_cus(int n) { g_num_cus = n > 0 ? n : 256; }

hipError_t launch_fwd_main(hipStream_t st, int fmt, const FwdArgs& a, int* kid) {
  *kid = KID_FWD_MAIN;
  if (a.m == 0 || a.n == 0) return hipSuccess;
  return fmt == LRQ_FMT_INT4 ? fwd_fmt<LRQ_FMT_INT4>(st, a) : fwd_fmt<LRQ_FMT_FP8>(st, a);
}

hipError_t launch_bwd_dx(hipStream_t st, int fmt, const BwdArgs& a, int* kid) {
  *kid = KID_BWD_DX;
  if (a.m == 0 || a.k == 0) return hipSuccess;
  return fmt == LRQ_FMT_INT4 ? bwd_fmt<LRQ_FMT_INT4>(st, a) : bwd_fmt<LRQ_FMT_FP8>(st, a);
}
