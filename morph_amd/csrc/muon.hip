// Hybrid Muon step for gfx950: momentum, Nesterov blend, Frobenius
// normalisation, Newton-Schulz quintic on bf16 MFMA, FP32 master update.
// Follows streamtrain/optimizer.py:13-22 (orthogonalize) and 52-61 (the Muon
// loop) for a batch of matrices that share one Newton-Schulz operand shape
// (each stored [rows, cols] or, with its transposed flag, [cols, rows]):
//
//   momentum.lerp_(g, mom_w)                    fma(mom_w, g - m, m)           (58)
//   u = g.lerp(momentum, nesterov_w)            fma(nesterov_w - 1, m - g, m)  (59)
//   X = u (or u^T when rows > cols) / (|u|_F + 1e-7)                      (15-18)
//   5x: A = X X^T; B' = b A + c A A + a I; X = B' X                        (19-21)
//       bf16 operands, fp32 accumulation
//   p = p * decay + (U * scale) * neg_lr        U = X in p's layout           (60-61)
//
// The reference computes orthogonalize in FP32; here X, A and B are bf16 (the
// precision this path specifies for Newton-Schulz) with fp32 accumulation and
// one rounding per product, so parity with the reference is a tolerance, not
// bit equality.  The momentum pass writes X0 = bf16(u) (transposed when
// rows > cols) and the FP64 sum of u^2; the first iteration's products apply
// the normalisation per matrix, A = X0 X0^T / den^2 and X' = B' X0 / den, so u
// never goes to memory.  The elementwise steps round exactly like
// torch (explicit fmaf where its CPU kernels fuse, plain multiplies elsewhere).
// The quintic's linear term rides on B's diagonal: X' = a X + B X = (B + a I) X,
// so the last product of an iteration reads no third operand (a is added in fp32
// to B's diagonal before its bf16 rounding; measured against the FP32
// reference this is as accurate as the separate a X term or more).  A Muon
// step's master update rides on the chain's last product where the operand has
// no padding (newton_schulz_finish, gemm_kn_apply): its epilogue updates p from
// the bf16 values it would have stored, so X is not written back and read again.
//
// Workspace (caller-allocated, morph_muon_workspace_bytes; no initial contents needed):
// per-block partial sums f64; per-matrix 1/den, 1/den^2, den f32;
// X0/X1 [count][Mp][Np] (iterations alternate: X' = B' X reads all of X as its
// [K, N] operand, so it cannot overwrite it), A and B' [count][Mp][Mp], bf16,
// with m = min(rows, cols), n = max, Mp/Np rounded up to the GEMM tile.  prepare
// writes X0 including its zero padding (pad_zero_kernel) and every product
// rewrites its whole padded output, so no call depends on an earlier one.  The
// zero padding is exact for Newton-Schulz: padded rows of X give zero rows and
// columns of A, and of B' apart from its diagonal (a on every diagonal
// element), so a padded row of X' is a times the padded row of X: zero again.
// Rows are stored kRowPad elements longer than Mp / Np (never read): with
// rows a multiple of 4 KiB apart, the 256 rows of a GEMM operand tile fall
// on few L2 channels; the pad spreads them (about 6% on the K = Mp products).
#include <algorithm>

#include "common.h"
#include "gemm.h"

namespace morph {
namespace {

constexpr int kBlock = 256;
constexpr int kMaxMats = 64;
static_assert(kGemmMaxApply >= kMaxMats, "a whole batch's update rides on one fused product");
// Workgroup shapes of the elementwise passes (HBM-bound; measured round-robin on
// the 42-matrix [3072, 6144] batch, bit-identical results throughout):
//   momentum_kernel: 256 lanes, one 128-bit access each (128 lanes: 6% slower);
//   apply_flat_kernel: 64 lanes, one 128-bit access each (128: 2%, 256: 6% slower);
//   momentum_t_kernel: tiles of 64 stored rows x 128 stored columns (512-byte row
//   segments of the FP32 streams, 128-byte segments of X), every load of a tile
//   in flight before the first is used, 2 workgroups per CU (3: 4% slower, 6 or
//   uncapped: 7% slower; 128 x 64 tiles: 14%, 64 x 256: 2%, tiles taken down
//   the columns first: 6% slower);
//   apply_t_kernel: tiles of 64 x 256 (1 KiB row segments of p, 128-byte ones of
//   X), 2 workgroups per CU (64 x 128 tiles: 2.5% slower);
//   the workgroups per CU set by a dynamic LDS reservation beside the static
//   tile (160 KiB of LDS per CU).
constexpr int kFlat = 256;
constexpr int kFlatApply = 64;
constexpr int kElemsPerBlock = kFlat * 4;
constexpr int kTR = 64;    // stored rows per momentum transpose tile
constexpr int kTC = 128;   // stored columns per momentum transpose tile
constexpr int kATR = 64;   // stored rows per apply transpose tile
constexpr int kATC = 256;  // stored columns per apply transpose tile
constexpr size_t kMomentumTReserve = 40 * 1024;  // + 16.5 KiB tile: 2 workgroups per CU
constexpr size_t kApplyTReserve = 24 * 1024;     // + 34 KiB tile: 2 workgroups per CU
constexpr int64_t kRowPad = 64;                 // bf16 elements appended to every X/A/B row

// The matrices one launch covers, by slot (blockIdx.y of the elementwise passes):
// a pass over one orientation lists only that orientation's matrices, so no
// workgroup is launched for another's.
struct MatPtrs {
  const float* grad[kMaxMats];
  const float* mom[kMaxMats];
  float* mom_out[kMaxMats];  // the updated momentum (== mom when updated in place)
  float* param[kMaxMats];
  int32_t transposed[kMaxMats];  // stored [cols, rows] instead of [rows, cols]
  int32_t index[kMaxMats];       // position in the batch: its X and partial sums
};

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

struct Layout {
  int64_t rows, cols, m, n, mp, np, count, numel;
  int64_t blocks;  // flat blocks per matrix (momentum_kernel)
  int64_t tiles;   // transpose tiles per matrix (momentum_t_kernel)
  int64_t atiles;  // transpose tiles per matrix (apply_t_kernel)
  int64_t parts;   // partial sums per matrix: max(blocks, tiles)
  int64_t ldn, ldm;  // row lengths of X ([Mp][ldn]) and of A, B ([Mp][ldm])
  size_t off_part, off_scale, off_x0, off_x1, off_a, off_b, total;
};

Layout make_layout(int64_t rows, int64_t cols, int64_t count) {
  Layout L;
  L.rows = rows;
  L.cols = cols;
  L.count = count;
  L.m = rows < cols ? rows : cols;
  L.n = rows < cols ? cols : rows;
  L.mp = round_up(L.m, MORPH_GEMM_TILE_M);
  L.np = round_up(L.n, MORPH_GEMM_TILE_N);  // also a multiple of the K tile (64)
  L.ldn = L.np + kRowPad;
  L.ldm = L.mp + kRowPad;
  L.numel = rows * cols;
  L.blocks = (L.numel + kElemsPerBlock - 1) / kElemsPerBlock;
  // tiles of a matrix stored with its long side as rows (the ones X transposes)
  L.tiles = ((L.n + kTR - 1) / kTR) * ((L.m + kTC - 1) / kTC);
  L.atiles = ((L.n + kATR - 1) / kATR) * ((L.m + kATC - 1) / kATC);
  L.parts = L.blocks > L.tiles ? L.blocks : L.tiles;
  size_t off = 0;
  auto take = [&](size_t bytes) {
    const size_t at = off;
    off = (off + bytes + 255) / 256 * 256;
    return at;
  };
  L.off_part = take((size_t)count * L.parts * 8);
  L.off_scale = take((size_t)count * 3 * 4);
  L.off_x0 = take((size_t)count * L.mp * L.ldn * 2);
  L.off_x1 = take((size_t)count * L.mp * L.ldn * 2);
  L.off_a = take((size_t)count * L.mp * L.ldm * 2);
  L.off_b = take((size_t)count * L.mp * L.ldm * 2);
  L.total = off;
  return L;
}

template <int kLanes = kBlock>
__device__ __forceinline__ double block_sum(double x, double* lds) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) lds[wave] = x;
  __syncthreads();
  double s = 0.0;
  if (threadIdx.x == 0)
    for (int w = 0; w < kLanes / 64; ++w) s += lds[w];
  return s;  // valid in thread 0
}

// Stored layout of a matrix: [pr, pc] = [rows, cols], or [cols, rows] when
// transposed.  X is [m, n] with m = min: it has the stored layout when
// pr <= pc, else it is the transpose.
__device__ __forceinline__ bool x_is_stored(const MatPtrs& mats, int mat, int64_t rows,
                                            int64_t cols) {
  const bool tr = mats.transposed[mat] != 0;
  return (tr ? cols : rows) <= (tr ? rows : cols);
}

// Momentum + Nesterov blend, with u = the blend written straight into the
// Newton-Schulz operand as X0 = bf16(u) (the Frobenius scale 1 / (|u| + 1e-7)
// is applied by the first iteration's products, so u itself never goes to
// memory), partial sums of u^2 in FP64 (one per block), and, with a flag,
// the non-finite test of the gradients (the gate of optimizer.py:49-51): a
// wave with a non-finite element stores 1; the caller then discards this
// pass's outputs (X0, and a momentum written to a separate buffer) without
// anything being mutated.  kMomentum = false: u = grad (orthogonalize alone).
template <bool kMomentum>
__device__ __forceinline__ void momentum_one(float gi, float& m, float& ui, float mom_w,
                                             float nest_w, bool large_m, bool large_n) {
  ui = gi;
  if constexpr (kMomentum) {
    m = large_m ? __fmaf_rn(mom_w - 1.0f, gi - m, gi) : __fmaf_rn(mom_w, gi - m, m);
    ui = large_n ? __fmaf_rn(nest_w - 1.0f, m - gi, m) : __fmaf_rn(nest_w, m - gi, gi);
  }
}

__device__ __forceinline__ void flag_nonfinite(uint32_t* found_inf, bool bad) {
  if (found_inf != nullptr && __any(bad) && (threadIdx.x & 63) == 0)
    *reinterpret_cast<volatile uint32_t*>(found_inf) = 1u;
}

// Matrices whose X has the stored layout: a flat pass.  A block covers
// kElemsPerBlock consecutive elements; a lane moves 4 consecutive elements
// (one row, pc a multiple of 4) per 128-bit access when the matrix's buffers
// are 16-byte aligned, else one element per access.  Gradient and momentum
// are touched once here, so their accesses are non-temporal.
template <bool kMomentum>
__global__ __launch_bounds__(kFlat) void momentum_kernel(MatPtrs mats, uint16_t* x_all,
                                                          double* part_all, int64_t rows,
                                                          int64_t cols, int64_t mp, int64_t ldn,
                                                          int64_t parts, float mom_w,
                                                          float nest_w, uint32_t* found_inf) {
  __shared__ double lds[kFlat / 64];
  const int slot = blockIdx.y, mat = mats.index[slot];
  const int64_t pc = mats.transposed[slot] ? rows : cols, numel = rows * cols;
  const float* g = mats.grad[slot];
  const float* mom = mats.mom[slot];
  float* mom_out = mats.mom_out[slot];
  uint16_t* xm = x_all + (int64_t)mat * mp * ldn;
  const int64_t base = (int64_t)blockIdx.x * kElemsPerBlock;
  const bool large_m = mom_w >= 0.5f, large_n = nest_w >= 0.5f;
  const uintptr_t addr = reinterpret_cast<uintptr_t>(g) |
                         (kMomentum ? reinterpret_cast<uintptr_t>(mom) |
                                          reinterpret_cast<uintptr_t>(mom_out)
                                    : 0);
  const bool vec = (addr & 15) == 0 && (pc & 3) == 0 && base + kElemsPerBlock <= numel;
  double ss = 0.0;
  bool bad = false;
  if (vec) {
#pragma unroll
    for (int k = 0; k < kElemsPerBlock / (4 * kFlat); ++k) {
      const int64_t i = base + ((int64_t)k * kFlat + threadIdx.x) * 4;
      const f32x4 gv = load_stream<true>(reinterpret_cast<const f32x4*>(g + i));
      const u32x4 gb = __builtin_bit_cast(u32x4, gv);
      bad |= nonfinite_f32_bits(gb.x) | nonfinite_f32_bits(gb.y) | nonfinite_f32_bits(gb.z) |
             nonfinite_f32_bits(gb.w);
      f32x4 mv = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (kMomentum) mv = load_stream<true>(reinterpret_cast<const f32x4*>(mom + i));
      uint32_t h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float m = mv[e], ui;
        momentum_one<kMomentum>(gv[e], m, ui, mom_w, nest_w, large_m, large_n);
        mv[e] = m;
        h[e] = float_to_bf16_bits(ui);
        ss += (double)ui * (double)ui;
      }
      if constexpr (kMomentum) store_stream<true>(reinterpret_cast<f32x4*>(mom_out + i), mv);
      const int64_t r = i / pc, c = i - r * pc;
      *reinterpret_cast<u32x2*>(xm + r * ldn + c) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    }
  } else {
    for (int64_t i = base + threadIdx.x; i < base + kElemsPerBlock && i < numel; i += kFlat) {
      float m = kMomentum ? mom[i] : 0.f, ui;
      bad |= nonfinite_f32_bits(__builtin_bit_cast(uint32_t, g[i]));
      momentum_one<kMomentum>(g[i], m, ui, mom_w, nest_w, large_m, large_n);
      if constexpr (kMomentum) mom_out[i] = m;
      const int64_t r = i / pc, c = i - r * pc;
      xm[r * ldn + c] = (uint16_t)float_to_bf16_bits(ui);
      ss += (double)ui * (double)ui;
    }
  }
  flag_nonfinite(found_inf, bad);
  const double s = block_sum<kFlat>(ss, lds);
  if (threadIdx.x == 0) part_all[(int64_t)mat * parts + blockIdx.x] = s;
}

// Tile geometry of momentum_t_kernel and apply_t_kernel: tile blockIdx.x
// of the stored layout [pr, pc] (TR x TC, row-major over tiles), for the
// matrices whose X is its transpose.  `vec`: a whole tile with dimensions a
// multiple of 4, moved 4 consecutive elements per lane access.
struct TileGeo {
  int64_t pr, pc, r0, c0, tiles_c, tile;
  bool valid, vec;
};

template <int TR, int TC>
__device__ __forceinline__ TileGeo tile_geo(const MatPtrs& mats, int slot, int64_t rows,
                                            int64_t cols) {
  TileGeo t;
  const bool tr = mats.transposed[slot] != 0;
  t.pr = tr ? cols : rows;
  t.pc = tr ? rows : cols;
  t.tiles_c = (t.pc + TC - 1) / TC;
  t.tile = blockIdx.x;
  t.r0 = (t.tile / t.tiles_c) * TR;
  t.c0 = (t.tile % t.tiles_c) * TC;
  t.valid = t.r0 < t.pr;
  t.vec = (t.pc & 3) == 0 && (t.pr & 3) == 0 && t.r0 + TR <= t.pr && t.c0 + TC <= t.pc;
  return t;
}

// Matrices whose X is the transpose of the stored layout: the momentum pass
// per kTR x kTC tile, bf16(u) transposed through LDS so that both the stored
// reads and the X writes are coalesced.  One partial sum per tile, indexed by
// the tile's place in the stored layout (row-major over tiles), so a matrix
// sums in the same order whichever way the batch describes it.
template <bool kMomentum>
__global__ __launch_bounds__(kBlock) void momentum_t_kernel(MatPtrs mats, uint16_t* x_all,
                                                            double* part_all, int64_t rows,
                                                            int64_t cols, int64_t mp, int64_t ldn,
                                                            int64_t parts, float mom_w,
                                                            float nest_w, uint32_t* found_inf) {
  __shared__ __attribute__((aligned(8))) uint16_t tile[kTR][kTC + 4];
  __shared__ double lds[kBlock / 64];
  const int slot = blockIdx.y, mat = mats.index[slot];
  const TileGeo t = tile_geo<kTR, kTC>(mats, slot, rows, cols);
  if (!t.valid) return;  // block-uniform
  const float* g = mats.grad[slot];
  const float* mom = mats.mom[slot];
  float* mom_out = mats.mom_out[slot];
  uint16_t* xm = x_all + (int64_t)mat * mp * ldn;
  const bool large_m = mom_w >= 0.5f, large_n = nest_w >= 0.5f;
  const uintptr_t addr = reinterpret_cast<uintptr_t>(g) |
                         (kMomentum ? reinterpret_cast<uintptr_t>(mom) |
                                          reinterpret_cast<uintptr_t>(mom_out)
                                    : 0);
  const bool vec = t.vec && (addr & 15) == 0;
  constexpr int kLPR = kTC / 4, kRPP = kBlock / kLPR;  // stored rows: lanes per row, rows per pass
  constexpr int kPasses = kTR / kRPP;
  const int q = threadIdx.x % kLPR, w = threadIdx.x / kLPR;
  double ss = 0.0;
  bool bad = false;
  if (vec) {
    // every load of the tile is issued before the first is used: a lane keeps
    // 2 x kPasses 128-bit loads in flight, which the few workgroups per CU need
    // to cover HBM latency
    f32x4 gv[kPasses], mv[kPasses];
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass)
      gv[pass] = load_stream<true>(reinterpret_cast<const f32x4*>(
          g + (t.r0 + w + pass * kRPP) * t.pc + t.c0 + 4 * q));
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      mv[pass] = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (kMomentum)
        mv[pass] = load_stream<true>(reinterpret_cast<const f32x4*>(
            mom + (t.r0 + w + pass * kRPP) * t.pc + t.c0 + 4 * q));
    }
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      const int rr = w + pass * kRPP;
      const u32x4 gb = __builtin_bit_cast(u32x4, gv[pass]);
      bad |= nonfinite_f32_bits(gb.x) | nonfinite_f32_bits(gb.y) | nonfinite_f32_bits(gb.z) |
             nonfinite_f32_bits(gb.w);
      uint32_t h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float m = mv[pass][e], ui;
        momentum_one<kMomentum>(gv[pass][e], m, ui, mom_w, nest_w, large_m, large_n);
        mv[pass][e] = m;
        h[e] = float_to_bf16_bits(ui);
        ss += (double)ui * (double)ui;
      }
      if constexpr (kMomentum)
        store_stream<true>(reinterpret_cast<f32x4*>(mom_out + (t.r0 + rr) * t.pc + t.c0 + 4 * q),
                           mv[pass]);
      *reinterpret_cast<u32x2*>(&tile[rr][4 * q]) =
          u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    }
  } else {
#pragma unroll
    for (int pass = 0; pass < kPasses; ++pass) {
      const int rr = w + pass * kRPP;
      const int64_t r = t.r0 + rr, c = t.c0 + 4 * q;
      uint32_t h[4] = {0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (r < t.pr && c + e < t.pc) {
          const int64_t i = r * t.pc + c + e;
          float m = kMomentum ? mom[i] : 0.f, ui;
          bad |= nonfinite_f32_bits(__builtin_bit_cast(uint32_t, g[i]));
          momentum_one<kMomentum>(g[i], m, ui, mom_w, nest_w, large_m, large_n);
          if constexpr (kMomentum) mom_out[i] = m;
          h[e] = float_to_bf16_bits(ui);
          ss += (double)ui * (double)ui;
        }
      }
      *reinterpret_cast<u32x2*>(&tile[rr][4 * q]) =
          u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    }
  }
  flag_nonfinite(found_inf, bad);
  __syncthreads();
  constexpr int kXL = kTR / 4, kXRP = kBlock / kXL;  // X rows: lanes per row, rows per pass
  const int q2 = threadIdx.x % kXL, w2 = threadIdx.x / kXL;
#pragma unroll
  for (int pass = 0; pass < kTC / kXRP; ++pass) {
    const int cc = w2 + pass * kXRP;
    const int64_t c = t.c0 + cc, r = t.r0 + 4 * q2;  // X row c, columns r .. r + 3
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = tile[4 * q2 + e][cc];
    if (t.vec) {
      *reinterpret_cast<u32x2*>(xm + c * ldn + r) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (c < t.pc && r + e < t.pr) xm[c * ldn + r + e] = (uint16_t)h[e];
    }
  }
  const double s = block_sum(ss, lds);
  if (threadIdx.x == 0) part_all[(int64_t)mat * parts + t.tile] = s;
}

// den = fp32(sqrt(sum)) + fp32(1e-7): x / (x.norm() + 1e-7) of optimizer.py:18.
// scale[mat] = 1 / den and scale[count + mat] = 1 / den^2 scale the first
// Newton-Schulz products of X0 = bf16(u); scale[2 count + mat] = den.
__global__ __launch_bounds__(kBlock) void norm_kernel(MatPtrs mats, const double* part_all,
                                                      float* scale, int64_t rows, int64_t cols,
                                                      int64_t blocks, int64_t tiles,
                                                      int64_t parts, int count) {
  __shared__ double lds[kBlock / 64];
  const int mat = blockIdx.x;
  const int64_t n = x_is_stored(mats, mat, rows, cols) ? blocks : tiles;
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < n; i += kBlock) s += part_all[(int64_t)mat * parts + i];
  const double t = block_sum(s, lds);
  if (threadIdx.x == 0) {
    const float den = (float)sqrt(t) + 1e-7f;
    scale[mat] = 1.0f / den;
    scale[count + mat] = (float)(1.0 / ((double)den * (double)den));
    scale[2 * count + mat] = den;
  }
}

// Zero padding of X0: columns n .. np - 1 of rows 0 .. m - 1 and all np columns
// of rows m .. mp - 1, per matrix (blockIdx.y).  Every product rewrites its
// whole padded output from its inputs, so X0's padding is the only one a call
// inherits; the chain writes X0 in its second iteration, and a non-finite
// input leaves NaN there (0 * NaN), so every prepare restores the zeros.
__global__ __launch_bounds__(kBlock) void pad_zero_kernel(uint16_t* x_all, int64_t m, int64_t n,
                                                          int64_t mp, int64_t np, int64_t ldn) {
  uint16_t* xm = x_all + (int64_t)blockIdx.y * mp * ldn;
  const int64_t tail = np - n, per_row = tail > 0 ? tail : 0;
  const int64_t total = m * per_row + (mp - m) * np;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kBlock) {
    if (i < m * per_row) {
      const int64_t r = i / per_row;
      xm[r * ldn + n + (i - r * per_row)] = 0;
    } else {
      const int64_t j = i - m * per_row, r = m + j / np;
      xm[r * ldn + (j - (r - m) * np)] = 0;
    }
  }
}

// Without Newton-Schulz iterations X itself is the result: X = bf16(X0 / den)
// over the whole padded buffer (zero padding stays zero).
__global__ __launch_bounds__(kBlock) void rescale_kernel(uint16_t* x_all, const float* den,
                                                         int64_t per_matrix) {
  const int mat = blockIdx.y;
  const float d = den[mat];
  uint16_t* xm = x_all + (int64_t)mat * per_matrix;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < per_matrix;
       i += (int64_t)gridDim.x * kBlock)
    xm[i] = (uint16_t)float_to_bf16_bits(bf16_bits_to_float(xm[i]) / d);
}

// p = p * decay + (U * scale) * neg_lr with U = X in p's layout; scale is
// scale_t for a transposed matrix.  kExtract: p = U instead (orthogonalize
// alone returns the fp32 value of U).
template <bool kExtract>
__device__ __forceinline__ float apply_one(float p, uint32_t u16, float scale, float decay,
                                           float neg_lr) {
  if constexpr (kExtract) {
    return bf16_bits_to_float(u16);
  } else {
    return muon_update_element(p, u16, scale, decay, neg_lr);
  }
}

// Matrices whose X has the stored layout: a flat pass, kFlatApply * 4 consecutive
// elements of p per block (rows of X read at their padded stride).
template <bool kExtract>
__global__ __launch_bounds__(kFlatApply) void apply_flat_kernel(MatPtrs mats,
                                                                const uint16_t* x_all,
                                                                int64_t rows, int64_t cols,
                                                                int64_t mp, int64_t ldn,
                                                                float scale_n, float scale_t,
                                                                float decay, float neg_lr) {
  const int slot = blockIdx.y, mat = mats.index[slot];
  const int64_t pc = mats.transposed[slot] ? rows : cols, numel = rows * cols;
  float* p = mats.param[slot];
  const float scale = mats.transposed[slot] ? scale_t : scale_n;
  const uint16_t* xm = x_all + (int64_t)mat * mp * ldn;
  const int64_t base = (int64_t)blockIdx.x * kFlatApply * 4;
  const bool vec = (reinterpret_cast<uintptr_t>(p) & 15) == 0 && (pc & 3) == 0 &&
                   base + kFlatApply * 4 <= numel;
  if (vec) {
    const int64_t i = base + (int64_t)threadIdx.x * 4;
    const int64_t r = i / pc, c = i - r * pc;
    const u32x2 v = *reinterpret_cast<const u32x2*>(xm + r * ldn + c);
    const uint32_t h[4] = {v.x & 0xFFFFu, v.x >> 16, v.y & 0xFFFFu, v.y >> 16};
    f32x4 pv = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (!kExtract) pv = load_stream<true>(reinterpret_cast<const f32x4*>(p + i));
#pragma unroll
    for (int e = 0; e < 4; ++e) pv[e] = apply_one<kExtract>(pv[e], h[e], scale, decay, neg_lr);
    store_stream<true>(reinterpret_cast<f32x4*>(p + i), pv);
  } else {
    for (int64_t i = base + threadIdx.x; i < base + kFlatApply * 4 && i < numel;
         i += kFlatApply) {
      const int64_t r = i / pc, c = i - r * pc;
      p[i] = apply_one<kExtract>(kExtract ? 0.f : p[i], xm[r * ldn + c], scale, decay, neg_lr);
    }
  }
}

// Matrices whose X is the transpose of the stored layout: per kATR x kATC tile of p,
// the X tile is staged through LDS so that the X reads and the p accesses are both
// coalesced rows.
template <bool kExtract>
__global__ __launch_bounds__(kBlock) void apply_t_kernel(MatPtrs mats, const uint16_t* x_all,
                                                         int64_t rows, int64_t cols, int64_t mp,
                                                         int64_t ldn, float scale_n, float scale_t,
                                                         float decay, float neg_lr) {
  __shared__ __attribute__((aligned(8))) uint16_t tile[kATC][kATR + 4];
  const int slot = blockIdx.y, mat = mats.index[slot];
  const TileGeo t = tile_geo<kATR, kATC>(mats, slot, rows, cols);
  if (!t.valid) return;  // block-uniform
  float* p = mats.param[slot];
  const float scale = mats.transposed[slot] ? scale_t : scale_n;
  const uint16_t* xm = x_all + (int64_t)mat * mp * ldn;
  const bool vec = t.vec && (reinterpret_cast<uintptr_t>(p) & 15) == 0;
  constexpr int kLPR = kATC / 4, kRPP = kBlock / kLPR;  // stored rows: lanes per row, rows per pass
  const int q = threadIdx.x % kLPR, w = threadIdx.x / kLPR;
  // the p rows go out first: they do not wait for the X tile
  f32x4 pv[kATR / kRPP];
  if (vec && !kExtract) {
#pragma unroll
    for (int pass = 0; pass < kATR / kRPP; ++pass)
      pv[pass] = load_stream<true>(
          reinterpret_cast<const f32x4*>(p + (t.r0 + w + pass * kRPP) * t.pc + t.c0 + 4 * q));
  }
  // tile[c - c0][r - r0] = X[c][r]: X rows c0 .. c0 + kATC - 1, columns r0 .. r0 + kATR - 1
  constexpr int kXL = kATR / 4, kXRP = kBlock / kXL, kXPasses = kATC / kXRP;
  const int q2 = threadIdx.x % kXL, w2 = threadIdx.x / kXL;
  if (t.vec) {
    // all X loads in flight together, behind the p loads
    u32x2 xv[kXPasses];
#pragma unroll
    for (int pass = 0; pass < kXPasses; ++pass)
      xv[pass] = *reinterpret_cast<const u32x2*>(xm + (t.c0 + w2 + pass * kXRP) * ldn + t.r0 +
                                                 4 * q2);
#pragma unroll
    for (int pass = 0; pass < kXPasses; ++pass)
      *reinterpret_cast<u32x2*>(&tile[w2 + pass * kXRP][4 * q2]) = xv[pass];
  } else {
#pragma unroll
    for (int pass = 0; pass < kXPasses; ++pass) {
      const int cc = w2 + pass * kXRP;
      const int64_t c = t.c0 + cc, r = t.r0 + 4 * q2;
      uint32_t h[4] = {0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (c < t.pc && r + e < t.pr) h[e] = xm[c * ldn + r + e];
      *reinterpret_cast<u32x2*>(&tile[cc][4 * q2]) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
    }
  }
  __syncthreads();
#pragma unroll
  for (int pass = 0; pass < kATR / kRPP; ++pass) {
    const int rr = w + pass * kRPP;
    const int64_t r = t.r0 + rr, c = t.c0 + 4 * q;
    uint32_t h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = tile[4 * q + e][rr];
    float* pr_ = p + r * t.pc + c;
    if (vec) {
      f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (!kExtract) v = pv[pass];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = apply_one<kExtract>(v[e], h[e], scale, decay, neg_lr);
      store_stream<true>(reinterpret_cast<f32x4*>(pr_), v);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (r < t.pr && c + e < t.pc)
          pr_[e] = apply_one<kExtract>(kExtract ? 0.f : pr_[e], h[e], scale, decay, neg_lr);
    }
  }
}

}  // namespace
}  // namespace morph

using namespace morph;


extern "C" size_t morph_muon_workspace_bytes(int64_t rows, int64_t cols, int count) {
  if (rows <= 0 || cols <= 0 || count <= 0) return 0;
  return make_layout(rows, cols, count).total;
}

namespace {

struct Bufs {
  Layout L;
  double* part;
  float* scale;  // [3][count]: 1 / den, 1 / den^2, den
  uint16_t* X[2];
  uint16_t* A;
  uint16_t* B;
};

// Validates the call and carves the workspace.  need_mats: mats must be given.
int setup(const morph_muon_matrix* mats, int count, int64_t rows, int64_t cols,
          const morph_muon_hp* hp, void* workspace, size_t workspace_bytes, bool need_mats,
          bool need_momentum, Bufs* out) {
  if (hp == nullptr || count < 0 || rows <= 0 || cols <= 0 || hp->ns_steps < 0)
    return MORPH_EINVAL;
  if (count > kMaxMats) return MORPH_ERANGE;
  if (need_mats) {
    if (count > 0 && mats == nullptr) return MORPH_EINVAL;
    for (int i = 0; i < count; ++i)
      if (mats[i].grad == nullptr || mats[i].param == nullptr ||
          (need_momentum && mats[i].momentum == nullptr) ||
          (mats[i].transposed != 0 && mats[i].transposed != 1) || mats[i].reserved != 0)
        return MORPH_EINVAL;
  }
  const Layout L = make_layout(rows, cols, count > 0 ? count : 1);
  if (workspace == nullptr || workspace_bytes < L.total) return MORPH_EWORKSPACE;
  if (reinterpret_cast<uintptr_t>(workspace) % 256) return MORPH_EINVAL;
  // grid x of the tile passes and of apply_flat_kernel (the most blocks of the flat passes)
  if (L.tiles > INT32_MAX || L.atiles > INT32_MAX ||
      (L.numel + kFlatApply * 4 - 1) / (kFlatApply * 4) > INT32_MAX)
    return MORPH_ERANGE;
  char* ws = static_cast<char*>(workspace);
  out->L = L;
  out->part = reinterpret_cast<double*>(ws + L.off_part);
  out->scale = reinterpret_cast<float*>(ws + L.off_scale);
  out->X[0] = reinterpret_cast<uint16_t*>(ws + L.off_x0);
  out->X[1] = reinterpret_cast<uint16_t*>(ws + L.off_x1);
  out->A = reinterpret_cast<uint16_t*>(ws + L.off_a);
  out->B = reinterpret_cast<uint16_t*>(ws + L.off_b);
  return MORPH_OK;
}

// The transpose tiles of `count` matrices (momentum_t_kernel, apply_t_kernel).
dim3 tile_grid(int64_t tiles, int count) { return dim3((unsigned)tiles, (unsigned)count); }

// X0 has the stored layout of a matrix when its stored rows are the shorter side.
bool stored_is_x(const morph_muon_matrix& m, int64_t rows, int64_t cols) {
  const bool tr = m.transposed != 0;
  return (tr ? cols : rows) <= (tr ? rows : cols);
}

enum class Orient { kAll, kStored, kTransposed };

// The batch's matrices of one orientation (kAll: every one) among positions
// first .. last - 1, in batch order; *n = how many.
MatPtrs pointers(const morph_muon_matrix* mats, int count, int64_t rows, int64_t cols,
                 Orient which, int* n, int first = 0, int last = -1) {
  MatPtrs m;
  int k = 0;
  if (last < 0) last = count;
  for (int i = first; i < last; ++i) {
    if (which != Orient::kAll && stored_is_x(mats[i], rows, cols) != (which == Orient::kStored))
      continue;
    m.grad[k] = mats[i].grad;
    m.mom[k] = mats[i].momentum;
    m.mom_out[k] = mats[i].momentum_out != nullptr ? mats[i].momentum_out : mats[i].momentum;
    m.param[k] = mats[i].param;
    m.transposed[k] = mats[i].transposed;
    m.index[k] = i;
    ++k;
  }
  *n = k;
  return m;
}

int prepare(const morph_muon_matrix* mats, int count, int64_t rows, int64_t cols,
            const morph_muon_hp* hp, void* workspace, size_t workspace_bytes, bool orth_only,
            uint32_t* found_inf, void* stream) {
  Bufs W;
  int rc = setup(mats, count, rows, cols, hp, workspace, workspace_bytes, true, !orth_only, &W);
  if (rc || count == 0) return rc;
  const Layout& L = W.L;
  hipStream_t s = as_stream(stream);
  int n_all, n_flat, n_tiled;
  const MatPtrs mp_ = pointers(mats, count, rows, cols, Orient::kAll, &n_all);
  const MatPtrs flat = pointers(mats, count, rows, cols, Orient::kStored, &n_flat);
  const MatPtrs tiled = pointers(mats, count, rows, cols, Orient::kTransposed, &n_tiled);
  const float mw = hp->momentum_weight, nw = hp->nesterov_weight;
  if (L.mp != L.m || L.np != L.n) {
    const int64_t pad = L.m * (L.np - L.n) + (L.mp - L.m) * L.np;
    const int64_t bx = std::min<int64_t>((pad + kBlock - 1) / kBlock, 1024);
    hipLaunchKernelGGL(pad_zero_kernel, dim3((unsigned)bx, count), dim3(kBlock), 0, s, W.X[0],
                       L.m, L.n, L.mp, L.np, L.ldn);
    if ((rc = launch_status())) return rc;
  }
  if (n_flat) {
    const dim3 ew((unsigned)L.blocks, n_flat);
    if (orth_only)
      hipLaunchKernelGGL(momentum_kernel<false>, ew, dim3(kFlat), 0, s, flat, W.X[0], W.part,
                         rows, cols, L.mp, L.ldn, L.parts, mw, nw, found_inf);
    else
      hipLaunchKernelGGL(momentum_kernel<true>, ew, dim3(kFlat), 0, s, flat, W.X[0], W.part,
                         rows, cols, L.mp, L.ldn, L.parts, mw, nw, found_inf);
    if ((rc = launch_status())) return rc;
  }
  if (n_tiled) {
    const dim3 tg = tile_grid(L.tiles, n_tiled);
    if (orth_only)
      hipLaunchKernelGGL(momentum_t_kernel<false>, tg, dim3(kBlock), kMomentumTReserve, s, tiled,
                         W.X[0], W.part, rows, cols, L.mp, L.ldn, L.parts, mw, nw, found_inf);
    else
      hipLaunchKernelGGL(momentum_t_kernel<true>, tg, dim3(kBlock), kMomentumTReserve, s, tiled,
                         W.X[0], W.part, rows, cols, L.mp, L.ldn, L.parts, mw, nw, found_inf);
    if ((rc = launch_status())) return rc;
  }
  hipLaunchKernelGGL(norm_kernel, dim3(count), dim3(kBlock), 0, s, mp_, W.part, W.scale, rows,
                     cols, L.blocks, L.tiles, L.parts, count);
  if ((rc = launch_status())) return rc;
  if (hp->ns_steps == 0) {
    const int64_t per = L.mp * L.ldn;
    const int64_t bx = std::min<int64_t>((per + kBlock - 1) / kBlock, 4096);
    hipLaunchKernelGGL(rescale_kernel, dim3((unsigned)bx, count), dim3(kBlock), 0, s, W.X[0],
                       W.scale + 2 * count, per);
    rc = launch_status();
  }
  return rc;
}

// Whether the last product can carry the parameter update (gemm_kn_apply): the
// operands have no padding and every parameter is 16-byte aligned.
bool can_fuse_update(const morph_muon_matrix* mats, int count, const Layout& L) {
  if (L.mp != L.m || L.np != L.n) return false;
  for (int i = 0; i < count; ++i)
    if (reinterpret_cast<uintptr_t>(mats[i].param) % 16) return false;
  return true;
}

// fuse: the batch's matrices, whose parameter update the last product carries in
// place of writing X (can_fuse_update must hold); nullptr: X is written.
int newton_schulz(int count, int64_t rows, int64_t cols, const morph_muon_hp* hp,
                  void* workspace, size_t workspace_bytes, void* stream,
                  const morph_muon_matrix* fuse = nullptr) {
  Bufs W;
  int rc = setup(nullptr, count, rows, cols, hp, workspace, workspace_bytes, false, false, &W);
  if (rc || count == 0) return rc;
  const Layout& L = W.L;
  const int64_t sx = L.mp * L.ldn, ss = L.mp * L.ldm;
  const int64_t n = L.ldn, m = L.ldm;  // leading dimensions
  int cur = 0;
  for (int it = 0; it < hp->ns_steps; ++it) {
    uint16_t* X = W.X[cur];
    // X0 = bf16(u) is not normalised yet: the first iteration's products take
    // the per-matrix factors, A = (X0 X0^T) / den^2 and X' = (B' X0) / den
    const float* inv_den = it == 0 ? W.scale : nullptr;
    const float* inv_den2 = it == 0 ? W.scale + count : nullptr;
    // A = X X^T (symmetric: upper triangle of tiles, mirrored)
    rc = gemm_nt_bf16_scaled(X, X, nullptr, W.A, nullptr, L.mp, L.mp, L.np, count, n, n, 0, m, 0,
                             sx, sx, 0, ss, 0, 1.0f, 0.0f, inv_den2, 0.0f, MORPH_GEMM_SYMMETRIC,
                             stream);
    if (rc) return rc;
    // B' = c (A A^T) + b A + a I (symmetric; a added on the diagonal before rounding)
    rc = gemm_nt_bf16_scaled(W.A, W.A, W.A, W.B, nullptr, L.mp, L.mp, L.mp, count, m, m, m, m, 0,
                             ss, ss, ss, ss, 0, hp->c, hp->b, nullptr, hp->a, MORPH_GEMM_SYMMETRIC,
                             stream);
    if (rc) return rc;
    if (fuse != nullptr && it == hp->ns_steps - 1) {
      // the last X' = B' X updates the parameters instead of being stored: the
      // finish pass's arithmetic (muon_update_element) on the same bf16 values
      GemmApply ap;
      for (int i = 0; i < count; ++i) {
        ap.p[i] = fuse[i].param;
        ap.transposed[i] = stored_is_x(fuse[i], rows, cols) ? 0 : 1;
        ap.scale[i] = fuse[i].transposed ? hp->update_scale_transposed : hp->update_scale;
      }
      ap.m = L.m;
      ap.n = L.n;
      ap.decay = hp->decay;
      ap.neg_lr = hp->neg_lr;
      rc = gemm_kn_apply(W.B, X, L.mp, L.np, L.mp, count, m, n, ss, sx, inv_den, ap, stream);
      if (rc) return rc;
      break;
    }
    // X' = B' X: X as the [K, N] operand (transposing LDS reads), into the other buffer
    rc = gemm_nt_bf16_scaled(W.B, X, nullptr, W.X[cur ^ 1], nullptr, L.mp, L.np, L.mp, count, m,
                             n, 0, n, 0, ss, sx, 0, sx, 0, 1.0f, 0.0f, inv_den, 0.0f,
                             MORPH_GEMM_Q_KN, stream);
    if (rc) return rc;
    cur ^= 1;
  }
  return MORPH_OK;
}

int finish(const morph_muon_matrix* mats, int count, int64_t rows, int64_t cols,
           const morph_muon_hp* hp, void* workspace, size_t workspace_bytes, bool orth_only,
           void* stream, int first = 0, int n = -1) {
  if (n < 0) n = count;
  if (first < 0 || first > count || n > count - first) return MORPH_EINVAL;
  Bufs W;
  int rc = setup(mats, count, rows, cols, hp, workspace, workspace_bytes, true, false, &W);
  if (rc || n == 0) return rc;
  const Layout& L = W.L;
  const uint16_t* x = W.X[hp->ns_steps & 1];  // the buffer the last iteration wrote
  hipStream_t s = as_stream(stream);
  int n_flat, n_tiled;
  const MatPtrs flat = pointers(mats, count, rows, cols, Orient::kStored, &n_flat, first,
                                first + n);
  const MatPtrs tiled = pointers(mats, count, rows, cols, Orient::kTransposed, &n_tiled, first,
                                 first + n);
  const float sn = hp->update_scale, st = hp->update_scale_transposed;
  if (n_flat) {
    const dim3 ew((unsigned)((L.numel + kFlatApply * 4 - 1) / (kFlatApply * 4)), n_flat);
    if (orth_only)
      hipLaunchKernelGGL(apply_flat_kernel<true>, ew, dim3(kFlatApply), 0, s, flat, x, rows,
                         cols, L.mp, L.ldn, sn, st, hp->decay, hp->neg_lr);
    else
      hipLaunchKernelGGL(apply_flat_kernel<false>, ew, dim3(kFlatApply), 0, s, flat, x, rows,
                         cols, L.mp, L.ldn, sn, st, hp->decay, hp->neg_lr);
    if ((rc = launch_status())) return rc;
  }
  if (n_tiled) {
    const dim3 tg = tile_grid(L.atiles, n_tiled);
    if (orth_only)
      hipLaunchKernelGGL(apply_t_kernel<true>, tg, dim3(kBlock), kApplyTReserve, s, tiled, x,
                         rows, cols, L.mp, L.ldn, sn, st, hp->decay, hp->neg_lr);
    else
      hipLaunchKernelGGL(apply_t_kernel<false>, tg, dim3(kBlock), kApplyTReserve, s, tiled, x,
                         rows, cols, L.mp, L.ldn, sn, st, hp->decay, hp->neg_lr);
  }
  return launch_status();
}

// newton_schulz, then the parameter update of finish: carried by the last product
// when the shape allows (can_fuse_update), else the finish pass after the chain.
int newton_schulz_finish(const morph_muon_matrix* mats, int count, int64_t rows, int64_t cols,
                         const morph_muon_hp* hp, void* workspace, size_t workspace_bytes,
                         void* stream) {
  Bufs W;
  int rc = setup(mats, count, rows, cols, hp, workspace, workspace_bytes, true, false, &W);
  if (rc || count == 0) return rc;
  if (hp->ns_steps >= 1 && can_fuse_update(mats, count, W.L))
    return newton_schulz(count, rows, cols, hp, workspace, workspace_bytes, stream, mats);
  rc = newton_schulz(count, rows, cols, hp, workspace, workspace_bytes, stream);
  if (!rc) rc = finish(mats, count, rows, cols, hp, workspace, workspace_bytes, false, stream);
  return rc;
}

}  // namespace

extern "C" int morph_muon_prepare(const morph_muon_matrix* mats, int count, int64_t rows,
                                  int64_t cols, const morph_muon_hp* hp, int orthogonalize_only,
                                  void* workspace, size_t workspace_bytes, uint32_t* d_found_inf,
                                  void* stream) {
  return prepare(mats, count, rows, cols, hp, workspace, workspace_bytes, orthogonalize_only != 0,
                 d_found_inf, stream);
}

extern "C" int morph_muon_newton_schulz(int count, int64_t rows, int64_t cols,
                                        const morph_muon_hp* hp, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  return newton_schulz(count, rows, cols, hp, workspace, workspace_bytes, stream);
}

extern "C" int morph_muon_finish(const morph_muon_matrix* mats, int count, int64_t rows,
                                 int64_t cols, const morph_muon_hp* hp, int orthogonalize_only,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  return finish(mats, count, rows, cols, hp, workspace, workspace_bytes, orthogonalize_only != 0,
                stream);
}

extern "C" int morph_muon_finish_range(const morph_muon_matrix* mats, int count, int64_t rows,
                                       int64_t cols, const morph_muon_hp* hp,
                                       int orthogonalize_only, int first, int n, void* workspace,
                                       size_t workspace_bytes, void* stream) {
  if (first < 0 || n < 0) return MORPH_EINVAL;  // n = -1 ("the rest") is internal only
  return finish(mats, count, rows, cols, hp, workspace, workspace_bytes, orthogonalize_only != 0,
                stream, first, n);
}

extern "C" int morph_muon_newton_schulz_finish(const morph_muon_matrix* mats, int count,
                                               int64_t rows, int64_t cols,
                                               const morph_muon_hp* hp, void* workspace,
                                               size_t workspace_bytes, void* stream) {
  return newton_schulz_finish(mats, count, rows, cols, hp, workspace, workspace_bytes, stream);
}

extern "C" int morph_muon_step(const morph_muon_matrix* mats, int count, int64_t rows,
                               int64_t cols, const morph_muon_hp* hp, void* workspace,
                               size_t workspace_bytes, void* stream) {
  int rc = prepare(mats, count, rows, cols, hp, workspace, workspace_bytes, false, nullptr, stream);
  if (!rc) rc = newton_schulz_finish(mats, count, rows, cols, hp, workspace, workspace_bytes, stream);
  return rc;
}

extern "C" int morph_muon_orthogonalize(const morph_muon_matrix* mats, int count, int64_t rows,
                                        int64_t cols, const morph_muon_hp* hp, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  int rc = prepare(mats, count, rows, cols, hp, workspace, workspace_bytes, true, nullptr, stream);
  if (!rc) rc = newton_schulz(count, rows, cols, hp, workspace, workspace_bytes, stream);
  if (!rc) rc = finish(mats, count, rows, cols, hp, workspace, workspace_bytes, true, stream);
  return rc;
}
