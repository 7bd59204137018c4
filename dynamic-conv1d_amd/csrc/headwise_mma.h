// Headwise dynamic convolution backward on gfx950 matrix cores, for head
// sizes 8, 16, 32 and 64 at 9 <= W <= 32 (bf16 / fp16).
//
// Reference: headwise.py:105-215 (causal_conv1d_bwd_kernel), any W
// (headwise.py:226).  With h the head of channel d, hs its size:
//   dx[t,d]      = sum_k dy[t+k,d] * (w[t+k,h,k] + sw[k,d])  (+ dy[t,d])
//   dw[t,h,k]    = sum_{d in h} dy[t,d] * x[t-k,d]
//   dsw[k,d]     = sum_t dy[t,d] * x[t-k,d]
//
// At wide W and head sizes of 16 and more, the per-head parts are products of
// matrices.  Over a tile of 16 rows t0 .. t0+15 and one head:
//   * dw: C[t][s] = sum_{d in h} dy[t,d] x[s,d] (K = the head's channels) and
//     dw[t,h,k] = C[t][t-k]: a 16x16x32 MFMA per 16-row block of s (16x16x16 at
//     head size 16, two chained at 64), whose operands are 16-byte pieces of
//     rows as they lie in memory (lane (q, n): row n, channels 8q .. 8q+7).  The
//     reference sums the same exact products in fp32 (headwise.py:149-153).
//   * the head weights' part of dx: dx[t,d] = sum_s Wm[t][s] dy[s,d] with the
//     banded Wm[t][s] = w[s,h,s-t] (0 <= s-t < W): a 16x16x16 MFMA per 16-row
//     block of s and 16 channels, dy by column from LDS (transposing reads).
// Head size 8: a 16-channel block holds two heads.  In the dw product lane
// quarter q's channels 4q..4q+3 lie in head 4q/8 of the block, so each head's
// product takes A with the other head's quarters zeroed; in the dx (and the
// forward's y) product the output column is the channel, so each head adds its
// banded Wm times dy with the other head's columns zeroed.  Twice the products
// of head size 16, on a pipe these kernels leave mostly idle.
// The static filter is per channel: dx[t,d] += sum_k dy[t+k,d] sw[k,d] and
// dsw[k,d] += sum_t dy[t,d] x[t-k,d] stay on the vector units, two products
// per instruction (v_dot2c_f32_bf16 / _f16 on row pairs of one channel, which
// the transposing LDS reads deliver packed), fp32 accumulation.
//
// Layout.  A wavefront owns 64 channels (whole heads) and walks a run of
// 16-row tiles of one sequence.  Its LDS holds rings of row blocks: x of the
// tile and the NB blocks before it (the look-back of W-1 <= 31 rows), dy and
// the heads' weight rows of the tile and the NB blocks after it (the dx
// look-ahead); each tile loads one new block of each while it computes.  In the
// vector phase lane (q, n) owns channel 16q+n of the tile's 16 rows (its
// dstatic_w sums stay in registers over the run); dx is summed there and
// stored a row at a time.  dw goes through a staging tile in LDS and is
// stored as 16-byte pieces of the rows (whole pieces: checked on the host).
// dstatic_w: one fp32 partial per wavefront, summed by reduce_partials in a
// fixed order (deterministic).
#pragma once

#include "headwise_fast.h"  // Dot2: two 16-bit products into an fp32 accumulator
#include "lowrank_mfma.h"

namespace dc {

constexpr int kHwMmaMinW = 9, kHwMmaMaxW = 32;

struct HwMmaArgs {
  int Tn;       // sequence length
  int D;        // channels (a multiple of 64)
  int H;        // heads
  int nwc;      // D / 64 wavefront columns
  int nspb;     // runs per sequence: run i of a sequence holds tiles [i*ntile/nspb, (i+1)*ntile/nspb)
  int nseg;     // B * nspb
  int nblk;     // nseg * nwc (one wavefront per workgroup)
  int residual;
};

// LDS bytes of one backward wavefront (HwMmaGeom::BYTES), for the host's launch size.
constexpr int hw_mma_bwd_lds_bytes(int W, int HS) {
  const int NB = (W - 1 + 15) / 16, WP2 = (W + 1) / 2, NGY = (WP2 + 9) / 2;
  const int NBY = (4 * NGY - 16 + 15) / 16, NR = NB + 1, NRY = NBY + 1;
  const int WPB = (64 / HS) * W * 2, BLK = 16 * (64 * 2 + 16);
  return NR * BLK + NRY * BLK + NRY * 16 * WPB + 16 * WPB + 16 + 64 * (16 * 4 + 16) + 16;
}

// LDS geometry of one wavefront (bytes): row blocks of 16 rows.
template <typename T, int W, int HS>
struct HwMmaGeom {
  static constexpr int NB = (W - 1 + 15) / 16;      // x look-back blocks (1 or 2): rows t0-W+1 ..
  static constexpr int WP2 = (W + 1) / 2;           // static-filter tap pairs
  // dy rows the vector phase reads: t0 .. t0+4*NGY-1 (the odd-aligned pairs of
  // the last tap pair reach row t0+14+2*WP2)
  static constexpr int NGY = (WP2 + 9) / 2;
  static constexpr int NBY = (4 * NGY - 16 + 15) / 16;  // dy / weight look-ahead blocks (>= NB)
  static constexpr int NR = NB + 1;                 // x ring slots
  static constexpr int NRY = NBY + 1;               // dy / weight ring slots
  static constexpr int NHW = 64 / HS;               // heads per wavefront
  static constexpr int XP = 64 * 2 + 16;            // x / dy row pitch: 64 channels + 16 bytes of pad
  static constexpr int WPB = NHW * W * 2;           // weight row of the wavefront's heads (16-byte multiple)
  static constexpr int BLK = 16 * XP;               // an x / dy block
  static constexpr int WBLK = 16 * WPB;             // a weight block
  static constexpr int DXP = 16 * 4 + 16;           // dx staging: a channel's 16 fp32 rows + pad
  static constexpr int X0 = 0;
  static constexpr int Y0 = X0 + NR * BLK;
  static constexpr int W0 = Y0 + NRY * BLK;
  static constexpr int DW0 = W0 + NRY * WBLK;       // dw staging: 16 rows of WPB
  static constexpr int DX0 = DW0 + 16 * WPB + 16;   // dx staging (16 bytes of dummy slot before it)
  static constexpr int Z0 = DX0 + 64 * DXP;         // 16 zero bytes
  static constexpr int BYTES = Z0 + 16;
  static_assert(WPB % 16 == 0, "whole 16-byte pieces of the heads' weight rows");
  static_assert(NBY >= NB && 4 * NGY <= 16 * NRY, "the dy ring holds the look-ahead rows");
  static_assert(BYTES == hw_mma_bwd_lds_bytes(W, HS), "the host's LDS size of the backward");
};

// The pair of 16-bit elements (2i+1, 2i+2) of a packed row sequence v (pair i
// holds elements 2i, 2i+1): the odd-aligned pairs of the dot products.
__device__ __forceinline__ uint32_t odd_pair(uint32_t lo, uint32_t hi) { return __builtin_amdgcn_alignbit(hi, lo, 16); }

template <typename T, int W, int HS, bool STATIC>
__global__ __launch_bounds__(64) void hw_bwd_mma(const T* __restrict__ x, const T* __restrict__ wt,
                                                 const T* __restrict__ sw, const T* __restrict__ dy,
                                                 T* __restrict__ dx, T* __restrict__ dwt, float* __restrict__ part,
                                                 HwMmaArgs a) {
  typedef HwMmaGeom<T, W, HS> G;
  constexpr int NB = G::NB, NBY = G::NBY, NR = G::NR, NRY = G::NRY, NHW = G::NHW, XP = G::XP, WPB = G::WPB;
  constexpr int NXQ = (W - 1 + 3) / 4;         // 4-row groups of x look-back
  constexpr int NGX = NXQ + 4;                 // x column groups: rows t0-4*NXQ .. t0+15
  constexpr int NGY = G::NGY;                  // dy column groups: rows t0 .. t0+4*NGY-1
  constexpr int WP2 = G::WP2;
  constexpr int WPC = WPB / 16;                // 16-byte pieces of a weight row
  constexpr int WPIECES = 16 * WPC;            // pieces of a weight block
  constexpr int NWP = (WPIECES + 63) / 64;     // a lane's pieces of a weight block
  static_assert(4 * NXQ <= 16 * NB, "x columns within the ring");
  __shared__ __attribute__((aligned(16))) uint8_t lds[G::BYTES];

  const int lane = threadIdx.x;
  const int q = lane >> 4, n = lane & 15;
  // consecutive blocks take consecutive runs of one 64-channel slab: their halo
  // rows meet in the same L2
  const int lb = xcd_remap(blockIdx.x, a.nblk);
  const int s = lb % a.nseg, wc = lb / a.nseg;
  const int Tn = a.Tn, D = a.D;
  const int b = s / a.nspb;
  const int ntile = (Tn + 15) >> 4;
  const int ri = s - b * a.nspb;  // runs split the sequence's tiles evenly (lengths differ by at most one)
  const int m0 = (int)((int64_t)ri * ntile / a.nspb), m1 = (int)((int64_t)(ri + 1) * ntile / a.nspb);
  const int c0 = wc * 64;
  const int rb = run_base_row(m0);  // resources from the run's first tile less 32 rows
  const int64_t row0 = (int64_t)b * Tn;
  const int rowb = D * 2, wrowb = a.H * W * 2;
  const rsrc_t rx = run_rsrc(x + (row0 + rb) * D, Tn - rb, rowb);
  const rsrc_t rdy = run_rsrc(dy + (row0 + rb) * D, Tn - rb, rowb);
  const rsrc_t rdx = run_rsrc(dx + (row0 + rb) * D, Tn - rb, rowb);
  const int64_t wrow0 = (row0 + rb) * a.H * W;
  const rsrc_t rw = run_rsrc(wt + wrow0, Tn - rb, wrowb);
  const rsrc_t rdw = run_rsrc(dwt + wrow0, Tn - rb, wrowb);
  const int wseg = (c0 / HS) * W * 2;  // the wavefront's heads in a weight row (bytes)

  // ---- block loads (16 rows): x / dy as 128 pieces of 16 bytes (8 lanes per
  // row), weights as WPIECES pieces; rows outside the run's resource read 0
  struct Blk {
    u32x4 v[2];
    u32x4 w[NWP];
  };
  const int prow = lane >> 3, pcol = (c0 + 8 * (lane & 7)) * 2;  // piece (row, byte column) of lane, +8 rows for v[1]
  auto load_xy = [&](rsrc_t r, int blk, Blk& o) {  // rows 16*blk .. +15
#pragma unroll
    for (int h = 0; h < 2; ++h) o.v[h] = bload128(r, (16 * blk + prow + 8 * h - rb) * rowb + pcol);
  };
  auto load_w = [&](int blk, Blk& o) {
#pragma unroll
    for (int i = 0; i < NWP; ++i) {
      const int p = i * 64 + lane, r = p / WPC, pc = p - r * WPC;
      o.w[i] = bload128(rw, p < WPIECES ? (16 * blk + r - rb) * wrowb + wseg + pc * 16 : kOobLane);
    }
  };
  // ring slots of row block blk (blk >= -4: the look-back of the first tiles)
  auto xslot = [&](int blk) { return (blk + 4 * NR) % NR; };
  auto yslot = [&](int blk) { return blk % NRY; };
  auto store_xy = [&](int base, int slot, const Blk& o) {
    uint8_t* p = lds + base + slot * G::BLK;
#pragma unroll
    for (int h = 0; h < 2; ++h) *reinterpret_cast<u32x4*>(p + (prow + 8 * h) * XP + 16 * (lane & 7)) = o.v[h];
  };
  auto store_w = [&](int blk, const Blk& o) {
    uint8_t* p = lds + G::W0 + yslot(blk) * G::WBLK;
#pragma unroll
    for (int i = 0; i < NWP; ++i) {
      const int pi = i * 64 + lane;
      if (pi < WPIECES) *reinterpret_cast<u32x4*>(p + pi * 16) = o.w[i];
    }
  };
  // LDS address of row r (absolute) of the x / dy ring, byte column cb
  // (r >> 4 floors, r & 15 wraps, for the negative rows of the first tiles' look-back)
  auto xa = [&](int r, int cb) { return G::X0 + xslot(r >> 4) * G::BLK + (r & 15) * XP + cb; };
  auto ya = [&](int r, int cb) { return G::Y0 + yslot(r >> 4) * G::BLK + (r & 15) * XP + cb; };
  auto wa = [&](int r, int e) { return G::W0 + yslot(r >> 4) * G::WBLK + (r & 15) * WPB + 2 * e; };

  // ---- static filter of the lane's channel 16q+n, packed tap pairs; dstatic_w sums
  const int cl = 16 * q + n;  // the lane's channel in the vector phase
  uint32_t swp[STATIC ? WP2 : 1];
  float dsw[STATIC ? W : 1];
  if constexpr (STATIC) {
    const rsrc_t rs = make_rsrc(sw, (int64_t)W * D * 2);
    uint32_t e[2 * WP2];
#pragma unroll
    for (int k = 0; k < 2 * WP2; ++k) e[k] = k < W ? bload16(rs, (k * D + c0 + cl) * 2) : 0u;
#pragma unroll
    for (int p = 0; p < WP2; ++p) swp[p] = (e[2 * p] & 0xFFFFu) | (e[2 * p + 1] << 16);
#pragma unroll
    for (int k = 0; k < W; ++k) dsw[k] = 0.f;
  }

  // ---- prologue: x blocks m0-NB .. m0, dy / weight blocks m0 .. m0+NBY
  {
    Blk t;
#pragma unroll
    for (int j = 0; j <= NB; ++j) {
      load_xy(rx, m0 - NB + j, t);
      store_xy(G::X0, xslot(m0 - NB + j), t);
    }
#pragma unroll
    for (int j = 0; j <= NBY; ++j) {
      load_xy(rdy, m0 + j, t);
      load_w(m0 + j, t);
      store_xy(G::Y0, yslot(m0 + j), t);
      store_w(m0 + j, t);
    }
    // the dw staging tile's dummy slot and the zero bytes
    if (lane < 4) *reinterpret_cast<uint32_t*>(lds + G::Z0 + 4 * lane) = 0u;
  }
  __syncthreads();

  for (int m = m0; m < m1; ++m) {
    const int t0 = 16 * m;
    // next tile's blocks, in flight during this one
    Blk nx;
    load_xy(rx, m + 1, nx);
    Blk ny;
    load_xy(rdy, m + 1 + NBY, ny);
    load_w(m + 1 + NBY, ny);

    // ---- dw: C[t][s] over K = the head's channels; dw[t,h,k] = C[t][t-k]
    {
      f32x4 c[NHW][NB + 1];
      if constexpr (HS < 16) {
        constexpr int HPG = 16 / HS;  // heads per 16-channel block
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int be = 0; be <= NB; ++be) {
            const u32x2 av = *reinterpret_cast<const u32x2*>(lds + ya(t0 + n, (g * 16 + 4 * q) * 2));
            const u32x2 bv = *reinterpret_cast<const u32x2*>(lds + xa(t0 - 16 * be + n, (g * 16 + 4 * q) * 2));
#pragma unroll
            for (int hh = 0; hh < HPG; ++hh) {
              const u32x2 am = (4 * q) / HS == hh ? av : u32x2{0u, 0u};  // K = channels 4q..4q+3
              c[g * HPG + hh][be] = Mma16<T>::run(am, bv, f32x4{0.f, 0.f, 0.f, 0.f});
            }
          }
      } else {
#pragma unroll
      for (int h = 0; h < NHW; ++h) {
#pragma unroll
        for (int be = 0; be <= NB; ++be) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
          if constexpr (HS == 16) {
            const u32x2 av = *reinterpret_cast<const u32x2*>(lds + ya(t0 + n, (h * 16 + 4 * q) * 2));
            const u32x2 bv = *reinterpret_cast<const u32x2*>(lds + xa(t0 - 16 * be + n, (h * 16 + 4 * q) * 2));
            acc = Mma16<T>::run(av, bv, acc);
          } else {
#pragma unroll
            for (int kc = 0; kc < HS / 32; ++kc) {
              const int cb = (h * HS + 32 * kc + 8 * q) * 2;
              const u32x4 av = *reinterpret_cast<const u32x4*>(lds + ya(t0 + n, cb));
              const u32x4 bv = *reinterpret_cast<const u32x4*>(lds + xa(t0 - 16 * be + n, cb));
              acc = Mma32<T>::run(av, bv, acc);
            }
          }
          c[h][be] = acc;
        }
      }
      }
      // lane (q, n) holds C[4q+i][n] of block be: t = t0+4q+i, s = t0-16be+n, k = 4q+i-n+16be
#pragma unroll
      for (int h = 0; h < NHW; ++h)
#pragma unroll
        for (int be = 0; be <= NB; ++be)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int k = 4 * q + i - n + 16 * be;
            const int off = (k >= 0 && k < W) ? G::DW0 + (4 * q + i) * WPB + (h * W + k) * 2 : G::DW0 + 16 * WPB;
            const T v = (T)c[h][be][i];
            *reinterpret_cast<T*>(lds + off) = v;
          }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < NWP; ++i) {
        const int p = i * 64 + lane, r = p / WPC, pc = p - r * WPC;
        const u32x4 v = *reinterpret_cast<const u32x4*>(lds + G::DW0 + (p < WPIECES ? p : 0) * 16);
        bstore128<true>(v, rdw, p < WPIECES ? (t0 + r - rb) * wrowb + wseg + pc * 16 : kOobLane);
      }
    }

    // ---- dx from the head weights: C = Wm dy per head and 16 channels, K = s blocks
    if constexpr (HS < 16) {
      constexpr int HPG = 16 / HS;
      f32x4 c[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) c[g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int be = 0; be <= NB; ++be) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int L = lane & 15;
          const u32x2 bv0 = lds_read_tr16(lds + ya(t0 + 16 * be + 4 * q + (L >> 2), (g * 16 + 4 * (L & 3)) * 2));
#pragma unroll
          for (int hh = 0; hh < HPG; ++hh) {
            const int h = g * HPG + hh;
            uint32_t e4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int k = 16 * be + 4 * q + e - n;
              const int addr = (k >= 0 && k < W) ? wa(t0 + 16 * be + 4 * q + e, h * W + k) : G::Z0;
              e4[e] = *reinterpret_cast<const uint16_t*>(lds + addr);
            }
            const u32x2 av = {e4[0] | (e4[1] << 16), e4[2] | (e4[3] << 16)};
            const u32x2 bv = n / HS == hh ? bv0 : u32x2{0u, 0u};  // column n = channel g*16+n
            c[g] = Mma16<T>::run(av, bv, c[g]);
          }
        }
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) *reinterpret_cast<f32x4*>(lds + G::DX0 + (g * 16 + n) * G::DXP + 16 * q) = c[g];
    } else {
      f32x4 c[NHW][HS / 16];
#pragma unroll
      for (int h = 0; h < NHW; ++h)
#pragma unroll
        for (int j = 0; j < HS / 16; ++j) c[h][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int be = 0; be <= NB; ++be) {
#pragma unroll
        for (int h = 0; h < NHW; ++h) {
          // A[n][4q+e] = w[s, h, s-t0-n] with s = t0+16be+4q+e (0 outside the band)
          uint32_t e4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int k = 16 * be + 4 * q + e - n;
            const int addr = (k >= 0 && k < W) ? wa(t0 + 16 * be + 4 * q + e, h * W + k) : G::Z0;
            e4[e] = *reinterpret_cast<const uint16_t*>(lds + addr);
          }
          const u32x2 av = {e4[0] | (e4[1] << 16), e4[2] | (e4[3] << 16)};
#pragma unroll
          for (int j = 0; j < HS / 16; ++j) {
            // B[4q+e][n] = dy[t0+16be+4q+e][channel h*HS+16j+n]: a transposing read
            // (lane a+4i addresses row 4q+i, channels +4a .. +4a+3 of the group)
            const int L = lane & 15;
            const u32x2 bv = lds_read_tr16(lds + ya(t0 + 16 * be + 4 * q + (L >> 2), (h * HS + 16 * j + 4 * (L & 3)) * 2));
            c[h][j] = Mma16<T>::run(av, bv, c[h][j]);
          }
        }
      }
      // lane (q, n): rows t0+4q .. +3 of channel h*HS+16j+n, to the transposed staging tile
#pragma unroll
      for (int h = 0; h < NHW; ++h)
#pragma unroll
        for (int j = 0; j < HS / 16; ++j)
          *reinterpret_cast<f32x4*>(lds + G::DX0 + (h * HS + 16 * j + n) * G::DXP + 16 * q) = c[h][j];
    }
    __syncthreads();

    // ---- vector phase: lane = channel cl of the tile's rows
    {
      // dy rows t0 .. t0+4*NGY-1 and x rows t0-4*NXQ .. t0+15 of channel cl, packed row
      // pairs (transposing reads: lane a+4i of a group addresses row R0+i, channels 4a .. 4a+3)
      const int L = lane & 15;
      const int cb = (16 * q + 4 * (L & 3)) * 2;
      uint32_t yc[2 * NGY], xc[2 * NGX];
#pragma unroll
      for (int g = 0; g < NGY; ++g) {
        const u32x2 v = lds_read_tr16(lds + ya(t0 + 4 * g + (L >> 2), cb));
        yc[2 * g] = v[0];
        yc[2 * g + 1] = v[1];
      }
#pragma unroll
      for (int g = 0; g < NGX; ++g) {
        const u32x2 v = lds_read_tr16(lds + xa(t0 - 4 * NXQ + 4 * g + (L >> 2), cb));
        xc[2 * g] = v[0];
        xc[2 * g + 1] = v[1];
      }
      const f32x4* dd = reinterpret_cast<const f32x4*>(lds + G::DX0 + cl * G::DXP);
      float dxv[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 v = dd[g];
#pragma unroll
        for (int i = 0; i < 4; ++i) dxv[4 * g + i] = v[i];
      }
      // residual: + dy[t]
      if (a.residual) {
#pragma unroll
        for (int r = 0; r < 16; ++r) dxv[r] += Mma16<T>::to_f(r & 1 ? yc[r >> 1] >> 16 : yc[r >> 1] & 0xFFFFu);
      }
      if constexpr (STATIC) {
        // dx[t0+r] += sum_k dy[t0+r+k] sw[k]: pairs (dy[t0+r+2p], dy[t0+r+2p+1]) . (sw[2p], sw[2p+1])
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
          for (int p = 0; p < WP2; ++p) {
            const int j = r + 2 * p;  // first row of the pair, from t0
            const uint32_t yp = (j & 1) ? odd_pair(yc[j >> 1], yc[(j >> 1) + 1]) : yc[j >> 1];
            dxv[r] = Dot2<T>::run(yp, swp[p], dxv[r]);
          }
        // dsw[k] += sum_r dy[t0+r] x[t0+r-k]: pairs of rows (2u, 2u+1)
#pragma unroll
        for (int k = 0; k < W; ++k)
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int j = 2 * u - k + 4 * NXQ;  // first x row of the pair, from t0-4*NXQ
            const uint32_t xp = (j & 1) ? odd_pair(xc[j >> 1], xc[(j >> 1) + 1]) : xc[j >> 1];
            dsw[k] = Dot2<T>::run(yc[u], xp, dsw[k]);
          }
      }
      // dx rows t0 .. t0+15 of channel c0+cl (rows past T are out of range)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const T v = (T)dxv[r];
        uint16_t bits;
        __builtin_memcpy(&bits, &v, 2);
        __builtin_amdgcn_raw_buffer_store_b16(bits, rdx, (t0 + r - rb) * rowb + (c0 + cl) * 2, 0, kNt);
      }
    }
    __syncthreads();  // every read of the slots the next blocks replace is done
    store_xy(G::X0, xslot(m + 1), nx);
    store_xy(G::Y0, yslot(m + 1 + NBY), ny);
    store_w(m + 1 + NBY, ny);
    __syncthreads();
  }

  if constexpr (STATIC) {
    // one fp32 partial per run, the wavefronts of its slabs writing their
    // channels: part[s][k * D + c0 + cl]
    float* pp = part + (int64_t)s * W * D;
#pragma unroll
    for (int k = 0; k < W; ++k) pp[(int64_t)k * D + c0 + cl] = dsw[k];
  }
}

}  // namespace dc

namespace dc {

// ------------------------------------------------------------------ forward
//   y[t,d] = sum_k (w[t,h,k] + sw[k,d]) x[t-k,d]  (+ x[t,d])     headwise.py:24-91
// Over a tile of 16 rows, per head: y = Wf x with the banded Wf[t][s] =
// w[t,h,t-s] (0 <= t-s < W) from the tile's own weight rows, a 16x16x16 MFMA per
// 16-row block of s and 16 channels (x by column from LDS: transposing reads);
// the static filter and the residual by row pairs on v_dot2c, lane = channel,
// after the MFMA sums pass through a transposed staging tile.  LDS: a ring of x
// blocks (the tile and the NBF blocks before it, which hold row t0-W: the
// padding tap of odd W), the tile's weight rows, the staging tile.
template <typename T, int W, int HS>
struct HwMmaFwdGeom {
  static constexpr int NBF = (W + 15) / 16;         // x look-back blocks
  static constexpr int NR = NBF + 1;
  static constexpr int NHW = 64 / HS;
  static constexpr int XP = 64 * 2 + 16;
  static constexpr int WPB = NHW * W * 2;
  static constexpr int BLK = 16 * XP;
  static constexpr int DXP = 16 * 4 + 16;
  static constexpr int X0 = 0;
  static constexpr int W0 = X0 + NR * BLK;          // the tile's weight rows
  static constexpr int Y0 = W0 + 16 * WPB;          // staging: 64 channels x 16 fp32 rows
  static constexpr int Z0 = Y0 + 64 * DXP;          // 16 zero bytes
  static constexpr int BYTES = Z0 + 16;
  static_assert(WPB % 16 == 0, "whole 16-byte pieces of the heads' weight rows");
};

template <typename T, int W, int HS, bool STATIC>
__global__ __launch_bounds__(64) void hw_fwd_mma(const T* __restrict__ x, const T* __restrict__ wt,
                                                 const T* __restrict__ sw, T* __restrict__ y, HwMmaArgs a) {
  typedef HwMmaFwdGeom<T, W, HS> G;
  constexpr int NBF = G::NBF, NR = G::NR, NHW = G::NHW, XP = G::XP, WPB = G::WPB;
  constexpr int NB = (W - 1 + 15) / 16;        // MFMA blocks of s before the tile's own
  constexpr int NXQ = (W + 3) / 4;             // 4-row groups of the x columns before t0 (row t0-W included)
  constexpr int NGX = NXQ + 4;                 // x column groups: rows t0-4*NXQ .. t0+15
  constexpr int WP2 = (W + 1) / 2;
  constexpr int WPC = WPB / 16;
  constexpr int WPIECES = 16 * WPC;
  constexpr int NWP = (WPIECES + 63) / 64;
  static_assert(4 * NXQ <= 16 * NBF && NB <= NBF, "x look-back within the ring");
  __shared__ __attribute__((aligned(16))) uint8_t lds[G::BYTES];

  const int lane = threadIdx.x;
  const int q = lane >> 4, n = lane & 15;
  const int lb = xcd_remap(blockIdx.x, a.nblk);
  const int s = lb % a.nseg, wc = lb / a.nseg;  // consecutive blocks: consecutive runs of one slab
  const int Tn = a.Tn, D = a.D;
  const int b = s / a.nspb;
  const int ntile = (Tn + 15) >> 4;
  const int ri = s - b * a.nspb;  // runs split the sequence's tiles evenly (lengths differ by at most one)
  const int m0 = (int)((int64_t)ri * ntile / a.nspb), m1 = (int)((int64_t)(ri + 1) * ntile / a.nspb);
  const int c0 = wc * 64;
  const int rb = run_base_row(m0);
  const int64_t row0 = (int64_t)b * Tn;
  const int rowb = D * 2, wrowb = a.H * W * 2;
  const rsrc_t rx = run_rsrc(x + (row0 + rb) * D, Tn - rb, rowb);
  const rsrc_t ry = run_rsrc(y + (row0 + rb) * D, Tn - rb, rowb);
  const rsrc_t rw = run_rsrc(wt + (row0 + rb) * a.H * W, Tn - rb, wrowb);
  const int wseg = (c0 / HS) * W * 2;

  struct Blk {
    u32x4 v[2];
    u32x4 w[NWP];
  };
  const int prow = lane >> 3, pcol = (c0 + 8 * (lane & 7)) * 2;
  auto load_x = [&](int blk, Blk& o) {
#pragma unroll
    for (int h = 0; h < 2; ++h) o.v[h] = bload128(rx, (16 * blk + prow + 8 * h - rb) * rowb + pcol);
  };
  auto load_w = [&](int blk, Blk& o) {
#pragma unroll
    for (int i = 0; i < NWP; ++i) {
      const int p = i * 64 + lane, r = p / WPC, pc = p - r * WPC;
      o.w[i] = bload128(rw, p < WPIECES ? (16 * blk + r - rb) * wrowb + wseg + pc * 16 : kOobLane);
    }
  };
  auto xslot = [&](int blk) { return (blk + 4 * NR) % NR; };
  auto store_x = [&](int blk, const Blk& o) {
    uint8_t* p = lds + G::X0 + xslot(blk) * G::BLK;
#pragma unroll
    for (int h = 0; h < 2; ++h) *reinterpret_cast<u32x4*>(p + (prow + 8 * h) * XP + 16 * (lane & 7)) = o.v[h];
  };
  auto store_w = [&](const Blk& o) {
#pragma unroll
    for (int i = 0; i < NWP; ++i) {
      const int pi = i * 64 + lane;
      if (pi < WPIECES) *reinterpret_cast<u32x4*>(lds + G::W0 + pi * 16) = o.w[i];
    }
  };
  auto xa = [&](int r, int cb) { return G::X0 + xslot(r >> 4) * G::BLK + (r & 15) * XP + cb; };

  // static filter of the lane's channel 16q+n as tap pairs in descending order:
  // (sw[2p+1], sw[2p]) meets the ascending row pair (x[t-2p-1], x[t-2p])
  const int cl = 16 * q + n;
  uint32_t swr[STATIC ? WP2 : 1];
  if constexpr (STATIC) {
    const rsrc_t rs = make_rsrc(sw, (int64_t)W * D * 2);
    uint32_t e[2 * WP2];
#pragma unroll
    for (int k = 0; k < 2 * WP2; ++k) e[k] = k < W ? bload16(rs, (k * D + c0 + cl) * 2) : 0u;
#pragma unroll
    for (int p = 0; p < WP2; ++p) swr[p] = (e[2 * p + 1] & 0xFFFFu) | (e[2 * p] << 16);
  }

  {
    Blk t;
#pragma unroll
    for (int j = 0; j <= NBF; ++j) {
      load_x(m0 - NBF + j, t);
      store_x(m0 - NBF + j, t);
    }
    load_w(m0, t);
    store_w(t);
    if (lane < 4) *reinterpret_cast<uint32_t*>(lds + G::Z0 + 4 * lane) = 0u;
  }
  __syncthreads();

  for (int m = m0; m < m1; ++m) {
    const int t0 = 16 * m;
    Blk nb;
    load_x(m + 1, nb);
    load_w(m + 1, nb);

    // ---- y from the head weights: C = Wf x per head and 16 channels, K = s blocks
    if constexpr (HS < 16) {
      constexpr int HPG = 16 / HS;
      f32x4 c[4];
#pragma unroll
      for (int g = 0; g < 4; ++g) c[g] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int be = 0; be <= NB; ++be) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int L = lane & 15;
          const u32x2 bv0 = lds_read_tr16(lds + xa(t0 - 16 * be + 4 * q + (L >> 2), (g * 16 + 4 * (L & 3)) * 2));
#pragma unroll
          for (int hh = 0; hh < HPG; ++hh) {
            const int h = g * HPG + hh;
            uint32_t e4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int k = 16 * be + n - 4 * q - e;
              const int addr = (k >= 0 && k < W) ? G::W0 + n * WPB + (h * W + k) * 2 : G::Z0;
              e4[e] = *reinterpret_cast<const uint16_t*>(lds + addr);
            }
            const u32x2 av = {e4[0] | (e4[1] << 16), e4[2] | (e4[3] << 16)};
            const u32x2 bv = n / HS == hh ? bv0 : u32x2{0u, 0u};  // column n = channel g*16+n
            c[g] = Mma16<T>::run(av, bv, c[g]);
          }
        }
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) *reinterpret_cast<f32x4*>(lds + G::Y0 + (g * 16 + n) * G::DXP + 16 * q) = c[g];
    } else {
      f32x4 c[NHW][HS / 16];
#pragma unroll
      for (int h = 0; h < NHW; ++h)
#pragma unroll
        for (int j = 0; j < HS / 16; ++j) c[h][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int be = 0; be <= NB; ++be) {
#pragma unroll
        for (int h = 0; h < NHW; ++h) {
          // A[n][4q+e] = w[t0+n, h, t0+n-s] with s = t0-16be+4q+e (0 outside the band)
          uint32_t e4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int k = 16 * be + n - 4 * q - e;
            const int addr = (k >= 0 && k < W) ? G::W0 + n * WPB + (h * W + k) * 2 : G::Z0;
            e4[e] = *reinterpret_cast<const uint16_t*>(lds + addr);
          }
          const u32x2 av = {e4[0] | (e4[1] << 16), e4[2] | (e4[3] << 16)};
#pragma unroll
          for (int j = 0; j < HS / 16; ++j) {
            const int L = lane & 15;
            const u32x2 bv = lds_read_tr16(lds + xa(t0 - 16 * be + 4 * q + (L >> 2), (h * HS + 16 * j + 4 * (L & 3)) * 2));
            c[h][j] = Mma16<T>::run(av, bv, c[h][j]);
          }
        }
      }
#pragma unroll
      for (int h = 0; h < NHW; ++h)
#pragma unroll
        for (int j = 0; j < HS / 16; ++j)
          *reinterpret_cast<f32x4*>(lds + G::Y0 + (h * HS + 16 * j + n) * G::DXP + 16 * q) = c[h][j];
    }
    __syncthreads();

    // ---- vector phase: lane = channel cl of the tile's rows
    {
      const int L = lane & 15;
      const int cb = (16 * q + 4 * (L & 3)) * 2;
      uint32_t xc[2 * NGX];
#pragma unroll
      for (int g = 0; g < NGX; ++g) {
        const u32x2 v = lds_read_tr16(lds + xa(t0 - 4 * NXQ + 4 * g + (L >> 2), cb));
        xc[2 * g] = v[0];
        xc[2 * g + 1] = v[1];
      }
      const f32x4* yd = reinterpret_cast<const f32x4*>(lds + G::Y0 + cl * G::DXP);
      float yv[16];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 v = yd[g];
#pragma unroll
        for (int i = 0; i < 4; ++i) yv[4 * g + i] = v[i];
      }
      if (a.residual) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = r + 4 * NXQ;  // row t0+r in the column
          yv[r] += Mma16<T>::to_f(j & 1 ? xc[j >> 1] >> 16 : xc[j >> 1] & 0xFFFFu);
        }
      }
      if constexpr (STATIC) {
        // y[t0+r] += sum_p (x[t-2p-1], x[t-2p]) . (sw[2p+1], sw[2p])
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
          for (int p = 0; p < WP2; ++p) {
            const int j = r - 2 * p - 1 + 4 * NXQ;  // first row of the pair in the column
            const uint32_t xp = (j & 1) ? odd_pair(xc[j >> 1], xc[(j >> 1) + 1]) : xc[j >> 1];
            yv[r] = Dot2<T>::run(xp, swr[p], yv[r]);
          }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const T v = (T)yv[r];
        uint16_t bits;
        __builtin_memcpy(&bits, &v, 2);
        __builtin_amdgcn_raw_buffer_store_b16(bits, ry, (t0 + r - rb) * rowb + (c0 + cl) * 2, 0, kNt);
      }
    }
    __syncthreads();
    store_x(m + 1, nb);
    store_w(nb);
    __syncthreads();
  }
}

}  // namespace dc

namespace dc {

// Host side (headwise_mma_*.hip instantiate the kernels per dtype and static
// filter; headwise.hip plans and dispatches).
// Widths the kernels take at head size hs: a wavefront's weight-row segment,
// (64 / hs) * W 16-bit elements, in whole 16-byte pieces.
constexpr bool hw_mma_width_ok(int hs, int W) {
  return W >= kHwMmaMinW && W <= kHwMmaMaxW && (hs == 8 || hs == 16 || hs == 32 || hs == 64) && ((64 / hs) * W) % 8 == 0;
}

template <typename T, bool STATIC>
hipError_t hw_bwd_mma_launch(const HwProblem& p, const HwMmaArgs& a, int hs);
template <typename T, bool STATIC>
hipError_t hw_fwd_mma_launch(const HwProblem& p, const HwMmaArgs& a, int hs);

}  // namespace dc
