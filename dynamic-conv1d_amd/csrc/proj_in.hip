// The upstream proj_in GEMM of the lowrank module on gfx950 matrix cores:
//
//   forward   z[m, c]      = sum_k pre_z[m, k] * W_in[c, k]        (c < N = G*R)
//   backward  dpre_z[m, k] = sum_c dz[m, c] * W_in[c, k]
//             dW_in[c, k]  = sum_m dz[m, c] * pre_z[m, k]
//
// README.md:67 and 75 (z = self.proj_in(pre_z), an nn.Linear(d_model, R,
// bias=False) per q / k / v module; the grouped module runs the G modules'
// projections as one GEMM with N = G*R outputs).  All three products are
// skinny (N <= 128 against M = B*T and K = d_model in the thousands) and far
// below the matrix-core ridge: each is bound by streaming pre_z (forward,
// dW_in) or writing dpre_z, so the kernels are laid out for HBM, as the
// lowrank kernels are.  Column c of z belongs to group c / R, rank c % R: the
// G groups' z (and dz) are separate [M, R] tensors, as the lowrank operator
// takes them.
//
// Forward (proj_fwd): a wavefront owns 16 rows and every output column; a
// workgroup of 4 wavefronts (64 rows) stages W_in in K-chunks of 128 through
// LDS, shared by its 4 wavefronts, while each wavefront streams its rows of
// pre_z straight into MFMA operands (v_mfma_f32_16x16x32: lane 16q + n holds
// row n, K elements 8q .. 8q+7 of each 32-wide step).
//
// Backward (proj_bwd): one pass over pre_z.  A workgroup owns 256 channels
// (4 wavefronts of 64) of one run of 16-row tiles; lane 16q + n holds rows
// 4q .. 4q+3, channels 4n .. 4n+3 of its wavefront's 64.  Per tile the
// workgroup stages the 16 rows of dz in LDS twice, row-major (the A operand
// of dpre_z = dz W_in, K = 32 ranks) and rank-major (dz^T, the A operand of
// dW_in += dz^T pre_z, K = 16 rows).  The W_in operands of the wavefront's 64
// channels sit in registers for the whole run.  dW_in is written as one fp32
// partial per run and summed by reduce_partials (fixed order: deterministic).
#include "lowrank_mfma.h"

namespace dc {

struct ProjArgs {
  const uint16_t* pre;              // [M, K]
  const uint16_t* w;                // [N, K]
  uint16_t* z[kMaxGroups];          // forward: G tensors [M, R]
  const uint16_t* dz[kMaxGroups];   // backward: G tensors [M, R]
  uint16_t* dpre;                   // backward: [M, K]
  float* part;                      // backward: dW_in partials [nrun][N][K]
  int M, K, N, R;
  int nblk;                         // grid size
  int ncg;                          // backward: 256-channel groups
  int seg;                          // backward: tiles per run
};

namespace {

constexpr int kProjOob = 0x7FFFFFF0;  // a byte offset past every resource's range (host-checked)

// Group g's pointer out of a table of kMaxGroups, by selects (g may differ by lane).
template <typename P>
__device__ __forceinline__ P pick4(const P (&t)[kMaxGroups], int g) {
  return g == 0 ? t[0] : g == 1 ? t[1] : g == 2 ? t[2] : t[3];
}

}  // namespace

// ---------------------------------------------------------------- forward
// KS K-splits per workgroup: 4 * KS wavefronts, wavefront w owns row tile w % 4
// of the workgroup's 64 rows and K half w / 4 of every staged chunk (KS * 128
// K elements); the halves' sums meet in LDS at the end.
template <typename T, int NB, int KS>
__global__ __launch_bounds__(256 * KS) void proj_fwd(ProjArgs a) {
  constexpr int KC = 128;                // K elements per wavefront per LDS stage
  constexpr int KW = KS * KC;            // K elements per LDS stage
  constexpr int WROW = KW * 2 + 16;      // bytes per staged W_in row: the 16-byte pad keeps the
                                         // 16 rows a quarter-wave reads at once in different banks
  constexpr int NP = NB * 16;            // staged W_in rows (zero past N)
  constexpr int NT = 256 * KS;           // threads
  constexpr int PIECES = NP * KW / 8 / NT;  // 16-byte pieces per thread per stage
  __shared__ __attribute__((aligned(16))) uint8_t wl[2][NP * WROW];

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int q = lane >> 4, n = lane & 15;
  const int rt = wave & 3, kh = wave >> 2;  // row tile, K half
  const int blk = xcd_remap(blockIdx.x, a.nblk);
  const int M = a.M, K = a.K, N = a.N;
  const int m0 = (blk * 4 + rt) * 16;
  const int rows = max(min(M - m0, 16), 0);
  // rows m0 .. m0+15 of pre_z: rows past M and K past the end read 0
  const rsrc_t rp = make_rsrc_wave<kProjOob>(a.pre + (int64_t)max(min(m0, M), 0) * K, (int64_t)rows * K * 2);
  const rsrc_t rw = make_rsrc_wave<kProjOob>(a.w, (int64_t)N * K * 2);
  const int prow = n * K * 2;  // the lane's row in rp

  f32x4 acc[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  // pre_z chunks stream from HBM: AD chunks in flight per wavefront (the K loop
  // is unrolled by AD, so ring slots are compile-time); W_in chunks come from L2
  // one chunk ahead and pass through LDS (two buffers, one barrier per chunk).
  // configs[4] (M 16384, K 4096, N 93): 4 wavefronts of 16 rows, AD 4: 44.7 us;
  // 8 wavefronts on two K halves, AD 4: 43.2 us; AD 2: 40.9 us (AD 6: 45.4 us).
  constexpr int AD = 2;
  u32x4 wv[PIECES];
  u32x4 av[AD][4];
  auto load_w = [&](int kc) {
#pragma unroll
    for (int i = 0; i < PIECES; ++i) {
      const int p = i * NT + (int)threadIdx.x;
      const int r = p / (KW / 8), c = p % (KW / 8);
      const int k = kc + c * 8;  // K % 8 == 0: a piece lies wholly inside K or outside it
      wv[i] = bload128(rw, r < N && k < K ? (r * K + k) * 2 : kProjOob);
    }
  };
  auto store_w = [&](int b) {
#pragma unroll
    for (int i = 0; i < PIECES; ++i) {
      const int p = i * NT + (int)threadIdx.x;
      const int r = p / (KW / 8), c = p % (KW / 8);
      *reinterpret_cast<u32x4*>(&wl[b][r * WROW + c * 16]) = wv[i];
    }
  };
  auto load_a = [&](int kc, u32x4(&av1)[4]) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int k = kc + kh * KC + 32 * c + 8 * q;
      av1[c] = bload128(rp, k < K ? prow + k * 2 : kProjOob);  // chunks past K read 0
    }
  };

  const int nchunk = (K + KW - 1) / KW;
  load_w(0);
#pragma unroll
  for (int i = 0; i < AD - 1; ++i) load_a(i * KW, av[i]);
  store_w(0);
  __syncthreads();
  for (int ch = 0; ch < nchunk; ch += AD) {
#pragma unroll
    for (int u = 0; u < AD; ++u) {
      const int cur = ch + u;
      if (cur >= nchunk) break;  // uniform across the workgroup
      const bool more = cur + 1 < nchunk;
      // next chunk's W_in and the chunk AD-1 ahead of pre_z go out before this chunk's products
      if (more) load_w((cur + 1) * KW);
      load_a((cur + AD - 1) * KW, av[(u + AD - 1) % AD]);
      __builtin_amdgcn_sched_barrier(0);
      const uint8_t* wb = wl[u & 1] + kh * KC * 2;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          const u32x4 b = *reinterpret_cast<const u32x4*>(wb + (nb * 16 + n) * WROW + (32 * c + 8 * q) * 2);
          acc[nb] = Mma32<T>::run(av[u][c], b, acc[nb]);
        }
      }
      if (more) {
        store_w((u + 1) & 1);  // the other buffer was last read before the previous barrier
        __syncthreads();
      }
    }
  }

  if constexpr (KS == 2) {
    // the second K half hands its sums to the first through LDS (the W_in buffers, now free)
    f32x4* xch = reinterpret_cast<f32x4*>(&wl[0][0]);
    static_assert(4 * NB * 64 * 16 <= 2 * NP * WROW, "exchange fits the staging buffers");
    __syncthreads();
    if (kh == 1) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) xch[(rt * NB + nb) * 64 + lane] = acc[nb];
    }
    __syncthreads();
    if (kh == 1) return;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb] += xch[(rt * NB + nb) * 64 + lane];
  }

  // z[m0 + 4q + i][col]: column col = nb*16 + n is rank col % R of group col / R
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int col = nb * 16 + n;
    if (col >= N) continue;
    const int g = col / a.R, r = col - g * a.R;
    uint16_t* zg = pick4(a.z, g);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + 4 * q + i;
      if (m < M) zg[(int64_t)m * a.R + r] = (uint16_t)f2bits<T>(acc[nb][i]);
    }
  }
}

// --------------------------------------------------------------- backward
template <typename T, int NB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(NB <= 6 ? 2 : 1, 8))) void proj_bwd(ProjArgs a) {
  constexpr int NP = NB * 16;          // ranks padded to whole 16-rank chunks (zero past N)
  constexpr int N32 = (NP + 31) / 32;  // 32-rank steps of the dpre_z product
  constexpr int NP32 = N32 * 32;       // ranks of the row-major dz tile (zero past N)
  constexpr int DROW = NP32 * 2 + 16;  // bytes per row of the row-major dz tile (16-byte pad)
  constexpr int TROW = 16 * 2 + 8;     // bytes per rank of the rank-major tile (8-byte pad)
  __shared__ __attribute__((aligned(16))) uint8_t dzr[2][16 * DROW];  // [row][rank]
  __shared__ __attribute__((aligned(16))) uint8_t dzt[2][NP * TROW];  // [rank][row]

  const int lane = threadIdx.x & 63, wave = wave_id();
  const int q = lane >> 4, n = lane & 15;
  const int blk = xcd_remap(blockIdx.x, a.nblk);
  const int cg = blk % a.ncg, run = blk / a.ncg;
  const int M = a.M, K = a.K, N = a.N, R = a.R;
  const int d0 = cg * 256 + wave * 64;   // the wavefront's first channel
  const int col = d0 + 4 * n;            // the lane's first channel (K % 8 == 0: 4 channels wholly in or out)
  const bool chv = col < K;
  const int ntile = (M + 15) >> 4;
  const int tile0 = run * a.seg, tile1 = min(tile0 + a.seg, ntile);
  const int r0 = tile0 * 16;
  const int nrow = max(min(M - r0, (tile1 - tile0) * 16), 0);
  const rsrc_t rp = make_rsrc_wave<kProjOob>(a.pre + (int64_t)min(r0, M) * K, (int64_t)nrow * K * 2);
  const rsrc_t rd = make_rsrc_wave<kProjOob>(a.dpre + (int64_t)min(r0, M) * K, (int64_t)nrow * K * 2);
  // the lane's row-4q channels in pre_z / dpre_z; lanes past K (chv false)
  // take kProjOob alone, never kProjOob plus a row offset (that sum would
  // overflow int32 and wrap back into the range)
  const int lane_off = (4 * q * K + col) * 2;

  // W_in operands of the dpre_z product (B of v_mfma_f32_16x16x32, K = ranks):
  // step s, channel j: ranks 32s + 8q .. +7 of channel col + j, packed.
  u32x4 wop[N32][4];
  {
    const rsrc_t rw = make_rsrc_wave<kProjOob>(a.w, (int64_t)N * K * 2);
#pragma unroll
    for (int s = 0; s < N32; ++s) {
      u32x2 rows8[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = 32 * s + 8 * q + e;
        rows8[e] = bload64(rw, chv && c < N ? (c * K + col) * 2 : kProjOob);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int h = 0; h < 4; ++h)
          wop[s][j][h] = elem16x2(rows8[2 * h], j) | (elem16x2(rows8[2 * h + 1], j) << 16);
    }
  }

  f32x4 dw[NB][4];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) dw[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // dz tile staging: NP32 x 16 elements, ~NP32 / 16 per thread; rank c is group
  // c / R, rank c % R (G separate tensors), zero past N and past M.
  constexpr int SPT = (NP32 * 16 + 255) / 256;
  uint32_t sv[SPT];
  auto load_dz = [&](int tile) {
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      const int e = i * 256 + (int)threadIdx.x;
      const int row = e / NP32, c = e - row * NP32;
      const int m = tile * 16 + row;
      // an unconditional load from a valid address (group 0's first element when
      // the element lies outside the tile), so no load sits under a branch
      const bool ok = e < NP32 * 16 && c < N && m < M && tile < tile1;
      const int g = ok ? c / R : 0;
      const uint16_t* src = ok ? pick4(a.dz, g) + ((int64_t)m * R + (c - g * R)) : a.dz[0];
      const uint32_t v = *src;
      sv[i] = ok ? v : 0u;
    }
  };
  auto store_dz = [&](int b) {
#pragma unroll
    for (int i = 0; i < SPT; ++i) {
      const int e = i * 256 + (int)threadIdx.x;
      if (e >= NP32 * 16) break;
      const int row = e / NP32, c = e - row * NP32;
      *reinterpret_cast<uint16_t*>(&dzr[b][row * DROW + c * 2]) = (uint16_t)sv[i];
      if (c < NP) *reinterpret_cast<uint16_t*>(&dzt[b][c * TROW + row * 2]) = (uint16_t)sv[i];
    }
  };
  // pre_z rows 4q .. 4q+3 of a tile, the lane's 4 channels (rows past the run read 0)
  auto load_pre = [&](int tile, u32x2(&pr)[4]) {
    const bool live = chv && tile < tile1;
    const int toff = (tile - tile0) * 16 * K * 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) pr[i] = bload64<kNt>(rp, live ? lane_off + toff + i * K * 2 : kProjOob);
  };

  u32x2 pa[4], pb[4];
  load_dz(tile0);
  store_dz(0);
  load_pre(tile0, pa);
  __syncthreads();
  auto compute = [&](int tile, int b, const u32x2(&pr)[4]) {
    // dpre_z = dz W_in: A = dz row n, ranks 32s + 8q .. +7
    f32x4 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < N32; ++s) {
      const u32x4 ar = *reinterpret_cast<const u32x4*>(&dzr[b][n * DROW + (32 * s + 8 * q) * 2]);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = Mma32<T>::run(ar, wop[s][j], acc[j]);
    }
    // lane (q, n) now holds rows 4q .. 4q+3 of channels col .. col+3
    const int toff = (tile - tile0) * 16 * K * 2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = tile * 16 + 4 * q + i;
      const u32x2 o = {pack2<T>(acc[0][i], acc[1][i]), pack2<T>(acc[2][i], acc[3][i])};
      bstore64<true>(o, rd, chv && tile < tile1 && m < M ? lane_off + toff + i * K * 2 : kProjOob);
    }
    // dW_in += dz^T pre_z: A = dz^T (ranks 16c + n, rows 4q .. 4q+3), B = pre_z rows 4q .. 4q+3 of channel col + j
    u32x2 bop[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bop[j][0] = elem16x2(pr[0], j) | (elem16x2(pr[1], j) << 16);
      bop[j][1] = elem16x2(pr[2], j) | (elem16x2(pr[3], j) << 16);
    }
#pragma unroll
    for (int c = 0; c < NB; ++c) {
      const u32x2 at = *reinterpret_cast<const u32x2*>(&dzt[b][(16 * c + n) * TROW + 8 * q]);
#pragma unroll
      for (int j = 0; j < 4; ++j) dw[c][j] = Mma16<T>::run(at, bop[j], dw[c][j]);
    }
  };

  const int nt = tile1 - tile0;
  for (int it = 0; it < nt; it += 2) {
    // tile it from (buffer 0, pa); tile it + 1 from (buffer 1, pb)
    load_dz(tile0 + it + 1);
    load_pre(tile0 + it + 1, pb);
    __builtin_amdgcn_sched_barrier(0);
    compute(tile0 + it, 0, pa);
    store_dz(1);  // buffer 1 was last read before the previous barrier
    __syncthreads();
    if (it + 1 >= nt) break;  // uniform across the workgroup
    load_dz(tile0 + it + 2);
    load_pre(tile0 + it + 2, pa);
    __builtin_amdgcn_sched_barrier(0);
    compute(tile0 + it + 1, 1, pb);
    store_dz(0);
    __syncthreads();
  }

  // dW_in partial of this run: rank 16c + 4q + i, channels col .. col+3
  const rsrc_t rpart = make_rsrc_wave<kProjOob>(a.part + (int64_t)run * N * K, (int64_t)N * K * 4);
#pragma unroll
  for (int c = 0; c < NB; ++c)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rk = 16 * c + 4 * q + i;
      const u32x4 v = {__float_as_uint(dw[c][0][i]), __float_as_uint(dw[c][1][i]), __float_as_uint(dw[c][2][i]),
                       __float_as_uint(dw[c][3][i])};
      bstore128<false>(v, rpart, chv && rk < N ? (rk * K + col) * 4 : kProjOob);
    }
}

// ------------------------------------------------------------------ host
namespace {

constexpr int kProjBwdTargetBlocks = 512;

int nb_of(int64_t N) { return (int)((N + 15) / 16); }

struct ProjBwdPlan {
  int ncg, nrun, seg;
};

ProjBwdPlan bwd_plan(const ProjProblem& p) {
  ProjBwdPlan pl;
  const int64_t ntile = (p.M + 15) / 16;
  pl.ncg = (int)((p.K + 255) / 256);
  int64_t nrun = (kProjBwdTargetBlocks + pl.ncg - 1) / pl.ncg;
  if (nrun > ntile) nrun = ntile;
  if (nrun < 1) nrun = 1;
  const int64_t seg = (ntile + nrun - 1) / nrun;
  pl.seg = (int)seg;
  pl.nrun = (int)((ntile + seg - 1) / seg);
  return pl;
}

ProjArgs base_args(const ProjProblem& p) {
  ProjArgs a{};
  a.pre = (const uint16_t*)p.pre_z;
  a.w = (const uint16_t*)p.w_in;
  a.M = (int)p.M;
  a.K = (int)p.K;
  a.N = (int)(p.G * p.R);
  a.R = (int)p.R;
  for (int g = 0; g < kMaxGroups; ++g) {
    const int s = g < p.G ? g : 0;
    a.z[g] = (uint16_t*)p.z[s];
    a.dz[g] = (const uint16_t*)p.dz[s];
  }
  return a;
}

constexpr int kProjFwdKs = 2;  // K halves per forward workgroup (8 wavefronts)

template <typename T>
hipError_t launch_fwd(const ProjProblem& p) {
  ProjArgs a = base_args(p);
  a.nblk = (int)((p.M + 63) / 64);
  switch (nb_of(a.N)) {
#define DC_PF(NBV) \
  case NBV: proj_fwd<T, NBV, kProjFwdKs><<<a.nblk, 256 * kProjFwdKs, 0, p.stream>>>(a); break;
    DC_PF(1) DC_PF(2) DC_PF(3) DC_PF(4) DC_PF(5) DC_PF(6) DC_PF(7) DC_PF(8)
#undef DC_PF
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename T>
hipError_t launch_bwd(const ProjProblem& p) {
  ProjArgs a = base_args(p);
  const ProjBwdPlan pl = bwd_plan(p);
  a.dpre = (uint16_t*)p.dpre_z;
  a.part = p.ws;
  a.ncg = pl.ncg;
  a.seg = pl.seg;
  a.nblk = pl.ncg * pl.nrun;
  switch (nb_of(a.N)) {
#define DC_PB(NBV) \
  case NBV: proj_bwd<T, NBV><<<a.nblk, 256, 0, p.stream>>>(a); break;
    DC_PB(1) DC_PB(2) DC_PB(3) DC_PB(4) DC_PB(5) DC_PB(6) DC_PB(7) DC_PB(8)
#undef DC_PB
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t NK = (int64_t)a.N * p.K;
  return reduce_partials(p.ws, NK, pl.nrun, NK, p.dw_in, p.dtype, p.stream);
}

}  // namespace

bool proj_shape_ok(const ProjProblem& p) {
  if (p.dtype != kBF16 && p.dtype != kFP16) return false;
  const int64_t N = p.G * p.R;
  if (N < 1 || N > 128 || p.K % 8 != 0) return false;
  // row indices (tiles of 16, blocks of 64 rows) are int: m0 + 64 stays in range
  if (p.M > INT32_MAX - 64) return false;
  // byte offsets within int32, below the out-of-range offset
  if ((int64_t)N * p.K * 4 >= kProjOob || 16 * p.K * 2 >= kProjOob) return false;
  const ProjBwdPlan pl = bwd_plan(p);
  return (int64_t)pl.seg * 16 * p.K * 2 + 16 * p.K * 2 < kProjOob;
}

int64_t proj_bwd_ws_bytes(const ProjProblem& p) {
  const ProjBwdPlan pl = bwd_plan(p);
  return (int64_t)pl.nrun * p.G * p.R * p.K * 4;
}

hipError_t proj_fwd_launch(const ProjProblem& p) {
  return p.dtype == kBF16 ? launch_fwd<bf16>(p) : launch_fwd<fp16>(p);
}

hipError_t proj_bwd_launch(const ProjProblem& p) {
  return p.dtype == kBF16 ? launch_bwd<bf16>(p) : launch_bwd<fp16>(p);
}

}  // namespace dc
