// Batched bf16 GEMM on gfx950 MFMA, the building block of the Muon
// Newton-Schulz iteration (streamtrain/optimizer.py:19-21):
//
//   C[b] = alpha * P[b] . Q[b]^T + beta * D[b]      (bf16 in, fp32 accumulate, bf16 out)
//   Ct[b] = C[b]^T                                   (optional second output)
//
// P is [M, K] row-major with K contiguous, so every P fragment is 16
// contiguous bytes of one row.  Q is [N, K] likewise ("NT"), or [K, N] with N
// contiguous (MORPH_GEMM_Q_KN): then its fragments come from LDS through
// gfx950's transposing reads (ds_read_b64_tr_b16) and the product is P . Q.
// One NS iteration is three products: A = X X^T and B' = c A A^T + b A + a I
// (A is symmetric; a is added to the diagonal in fp32 before the rounding) in
// the NT form, and X' = B' X with X as the [K, N] operand.
//
// Tiling.  A workgroup (256 lanes, 4 wave64) owns a 256 x 256 tile of C; wave w
// owns the 128 x 128 quarter (w / 2, w % 2) as 4 x 4 tiles of
// v_mfma_f32_32x32x16_bf16 (256 fp32 accumulators per lane).  Per 16-deep
// sub-step a wave reads 8 fragments (8 KiB) from LDS for 16 MFMAs.
//
// Operand pipeline.  K advances 64 per stage.  The LDS holds a ring of five
// 32 KiB slots, each the P or the Q sub-tile (256 x 64 bf16) of one stage, and
// two register sets of fragments hold one 16-deep sub-step each.  Operands go
// global -> LDS directly (buffer_load_dwordx4 ... lds: lane l's 16 bytes land
// at the instruction's LDS base + 16 l), so no registers are spent on staging.
// A row of a stage is one 128-byte line and its eight chunks are fetched by
// eight adjacent lanes, so every L2 request is a full line (32-deep stages
// fetch half lines and double the request count for the same bytes).  The
// load path accepts about 64 bytes per clock per CU, so loads are spread a
// quarter stage per sub-step under the MFMAs; five slots give the loads of a
// stage two steps of cover.  Each sub-step's 16 MFMAs run under the fragment
// reads of the next; one LDS-only barrier per stage.
// Because the DMA writes LDS linearly, rows cannot be padded; instead the
// eight 16-byte chunks of each 128-byte row are stored XOR-swizzled (slot =
// chunk ^ ((row ^ (row >> 3)) & 7)), chosen on the load side by which global
// chunk each lane fetches, so the 128-bit fragment reads of 8 or 16
// consecutive rows hit distinct banks.
//
// Workgroup order.  The dispatcher hands workgroup i to XCD i % 8; each XCD
// has its own L2.  Tiles are therefore numbered so that the workgroups one
// XCD runs at a time form a compact block (groups of kGroupM tile rows walked
// column by column), and each XCD gets a contiguous range of that numbering:
// the concurrently running tiles of an XCD share operand panels in its L2.
//
// Symmetric mode (A = X X^T and B' = c A A^T + b A + a I are symmetric): only tiles
// with tile_row <= tile_col run, and each off-diagonal tile is also written
// transposed into the mirror position, halving the work of those products.
//
// Epilogue.  Each lane combines alpha * acc + beta * D in fp32 and rounds once
// to bf16 (packed converter, round to nearest even).  D and C pass through an
// LDS copy of the tile for coalesced 16-byte rows.  In the MFMA output layout
// four consecutive registers of a lane are four consecutive rows of one
// column, i.e. 8 contiguous bytes of a row of the transposed tile: Ct and the
// mirror tile of a symmetric product are written into the same LDS with one
// 64-bit write per four values, then leave as coalesced rows too.  Loads are
// issued in batches ahead of their use so the epilogue pays memory latency a
// few times, not per element.
//
// The [K, N] kernel (X' = B' X) and the diagonal-add kernel (B' = c A A + b A +
// a I) pass the Q fragment as the MFMA's first operand: their accumulators are
// then row chunks of C (register r of lane l holds C[l % 32][8 (r / 4) +
// 4 (l / 32) + r % 4]; both fragment shapes are "a row of 8 consecutive k"), so
// C and D move through the LDS tile with 64-bit accesses instead of 2-byte ones
// and the mirror tile leaves through transposing LDS reads (epilogue_rows).
// Sustained over the whole chain: 0.7% faster for X', then 0.4% more for B'
// (whose kernel also spills no registers this way: 0 against 14).  The same
// change in the A = X X^T kernel measured even (36.10 against 36.12 ms).
//
// Each epilogue variant (D or not, alpha multiply or not, diagonal add or not)
// is a kernel of its own, chosen on the host: a kernel holding every variant
// spilled 32-50 VGPRs to scratch in its epilogue, and the Newton-Schulz chain
// ran 1.2% faster with one variant per kernel (0-14 spilled VGPRs).
//
// MFMA 32x32x16 lane layout (checked on the device): lane l holds
// A[l % 32][8 (l / 32) + i] and B[8 (l / 32) + i][l % 32] for i < 8; output
// register r of lane l is C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
//
// The last product of a Muon step's chain can carry the FP32 master update
// instead of storing X' (gemm_apply_kernel, gemm_kn_apply): the epilogue stages
// bf16(X') through the LDS tile exactly as for the store, then updates the
// parameter tile (p rows = tile rows, or = tile columns through transposing LDS
// reads for a parameter stored transposed) with the finish pass's arithmetic.
//
// Dimensions must be multiples of the tile (M, N of 256, K of 64): callers pad
// with zeros, which is exact for Newton-Schulz (zero rows stay zero).
#include "common.h"
#include "gemm.h"

namespace morph {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int BM = MORPH_GEMM_TILE_M;
constexpr int BN = MORPH_GEMM_TILE_N;
constexpr int BK = 64;               // K per pipeline stage: one 128-byte line per row
constexpr int kSlots = 5;            // LDS ring of operand sub-tiles (P or Q of one stage)
constexpr int LDE = BN + 8;          // padded LDS row of the output tile (bf16)
constexpr int kThreads = 256;
constexpr int kSubTile = BM * BK;                    // bf16 per operand sub-tile (256 x 64, 32 KiB)
constexpr int kSmemElems = (kSlots * kSubTile > BM * LDE) ? kSlots * kSubTile : BM * LDE;
static_assert(kSmemElems * 2 <= 160 * 1024, "LDS of one workgroup");
constexpr int kGroupM = 4;
static_assert(BM == BN && BM == 256 && MORPH_GEMM_TILE_K % BK == 0, "256 x 256 tiles, K % 64");

typedef __attribute__((address_space(3))) void lds_void;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 (a in the low half), one v_cvt_pk_bf16_f32:
// round to nearest even, the same bits as float_to_bf16_bits for every
// non-NaN input (NaN payloads may differ; both stay NaN).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

struct GemmArgs {
  const uint16_t* P;
  const uint16_t* Q;
  const uint16_t* D;
  uint16_t* C;
  uint16_t* Ct;
  int64_t K;
  int64_t ldp, ldq, ldd, ldc, ldct;
  int64_t sp, sq, sd, sc, sct;
  float alpha, beta;
  const float* bscale;       // optional per-matrix factor of alpha and beta (device)
  float diag;                // added to the diagonal elements of a symmetric product
  int32_t tiles_m, tiles_n;
  int32_t tiles_per_matrix;  // tiles_m * tiles_n, or the upper triangle when symmetric
  int32_t flags;             // MORPH_GEMM_SYMMETRIC
  int64_t total_tiles;       // batch * tiles_per_matrix
};

// Tile (row, col) of the t-th tile of one matrix.
__device__ __forceinline__ void tile_of(const GemmArgs& g, int t, int& tr, int& tc) {
  if (g.flags & MORPH_GEMM_SYMMETRIC) {  // upper triangle, row by row
    int r = 0;
    while (t >= g.tiles_n - r) {
      t -= g.tiles_n - r;
      ++r;
    }
    tr = r;
    tc = r + t;
    return;
  }
  const int per_group = kGroupM * g.tiles_n;
  const int group = t / per_group;
  const int within = t - group * per_group;
  const int first = group * kGroupM;
  const int rows = min(kGroupM, g.tiles_m - first);
  tc = within / rows;
  tr = first + within % rows;
}

enum DMode { kNoD, kDRowMajor };

// dst rows (256 x 256 bf16, leading dimension ld) from the LDS tile E, in
// coalesced 16-byte chunks; reads are batched 8 per lane ahead of the stores.
__device__ __forceinline__ void store_tile(const uint16_t* E, uint16_t* dst, uint32_t ld) {
  constexpr int kChunks = BM * (BN / 8) / kThreads;  // 32 per lane
  constexpr int kBatch = 8;
  const int tid = threadIdx.x;
#pragma unroll
  for (int b = 0; b < kChunks; b += kBatch) {
    u32x4 v[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int c = tid + (b + i) * kThreads;
      v[i] = *reinterpret_cast<const u32x4*>(E + (c / (BN / 8)) * LDE + (c % (BN / 8)) * 8);
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int c = tid + (b + i) * kThreads;
      *reinterpret_cast<u32x4*>(dst + ((uint32_t)(c / (BN / 8)) * ld + (c % (BN / 8)) * 8)) = v[i];
    }
  }
}

// Epilogue of one tile.  acc[i][j][r] of lane (fh, fr) of wave (wr, wc) is tile
// element (wr + 32 i + 8 (r / 4) + 4 fh + r % 4, wc + 32 j + fr).  The D mode
// and the alpha multiply are template parameters so that each variant is
// straight-line code.
template <int kDMode, bool kScaled, bool kDiag>
__device__ __forceinline__ void epilogue(const GemmArgs& g, float alpha, float beta,
                                         f32x16 (&acc)[4][4], uint16_t* smem, const uint16_t* D,
                                         uint16_t* C, uint16_t* T, int64_t ldt) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = (wave >> 1) * 128, wc = (wave & 1) * 128;
  const int fr = lane & 31, fh = lane >> 5;
  uint16_t* E = smem;  // [BM][LDE] bf16 copy of the output tile
  const uint32_t ldd = (uint32_t)g.ldd;

  if (kDMode == kDRowMajor) {
    // Row-major D into the LDS tile, all 32 loads of a lane in flight at once.
    constexpr int kDChunks = BM * (BN / 8) / kThreads;
    u32x4 dv[kDChunks];
#pragma unroll
    for (int i = 0; i < kDChunks; ++i) {
      const int c = tid + i * kThreads;
      dv[i] = *reinterpret_cast<const u32x4*>(D + (uint32_t)(c / (BN / 8)) * ldd + (c % (BN / 8)) * 8);
    }
#pragma unroll
    for (int i = 0; i < kDChunks; ++i) {
      const int c = tid + i * kThreads;
      *reinterpret_cast<u32x4*>(E + (c / (BN / 8)) * LDE + (c % (BN / 8)) * 8) = dv[i];
    }
    __syncthreads();
  }
  // Per element: (alpha *) acc, fma with beta * D, one RNE rounding to bf16 by
  // the packed converter (two rows per instruction).  The FP32 result goes
  // back into acc (accumulation registers, free by now) so the transposed pass
  // can round it again to the same bits without holding 128 packed words.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = wc + j * 32 + fr;
      const int rbase = wr + i * 32 + fh * 4;
      float dval[16];
      if (kDMode == kDRowMajor) {
        // all 16 reads of the block before its arithmetic and writes: one LDS round
        // trip (the barrier keeps the scheduler from splitting them into short batches)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          dval[r] = bf16_bits_to_float(E[(rbase + (r >> 2) * 8 + (r & 3)) * LDE + col]);
        __builtin_amdgcn_sched_barrier(0);
      }
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        x[r] = kScaled ? alpha * acc[i][j][r] : acc[i][j][r];
        if (kDMode != kNoD) x[r] = __fmaf_rn(beta, dval[r], x[r]);
      }
      if constexpr (kDiag) {
        // a diagonal tile: its diagonal runs through the blocks i == j of waves 0 and 3
        if (i == j && wr == wc) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (rbase + (r >> 2) * 8 + (r & 3) == col) x[r] = x[r] + g.diag;
        }
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        // w: rows row and row + 1 of column col
        const uint32_t w = pack_bf16x2(x[2 * k], x[2 * k + 1]);
        const int row = rbase + (k >> 1) * 8 + (k & 1) * 2;
        E[row * LDE + col] = (uint16_t)w;
        E[(row + 1) * LDE + col] = (uint16_t)(w >> 16);
      }
      if (kDMode != kNoD || kScaled || kDiag) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = x[r];
      }
    }
  }
  __syncthreads();
  store_tile(E, C, (uint32_t)g.ldc);  // C rows from the LDS tile
  if (T) {
    // Transposed copy (Ct, or the mirror tile): ET[c][r] = tile[r][c] in the
    // same LDS.  Four consecutive rows of one column are 8 contiguous bytes of
    // an ET row, so every two packed pairs go out with one 64-bit LDS write;
    // then ET's rows leave as coalesced 16-byte stores like C's.
    __syncthreads();  // every lane has read its C rows out of E
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          u32x2 v;
          v.x = pack_bf16x2(acc[i][j][4 * q], acc[i][j][4 * q + 1]);
          v.y = pack_bf16x2(acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
          *reinterpret_cast<u32x2*>(E + (wc + j * 32 + fr) * LDE + wr + i * 32 + fh * 4 + q * 8) = v;
        }
    __syncthreads();
    store_tile(E, T, (uint32_t)ldt);
  }
}

// T rows from the row-major LDS tile E through transposing reads: the 16 lanes of
// a group read a 4 x 16 block (source lane j: row rb + j / 4, columns c0 +
// 4 (j % 4) .. + 3) and lane j receives the four rows of column c0 + j, four
// consecutive elements of T row c0 + j; two reads give 16 bytes of a T row.
__device__ __forceinline__ void store_tile_t(const uint16_t* E, uint16_t* dst, uint32_t ld) {
  typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = lane >> 4, j = lane & 15;
  auto tr = [](const uint16_t* at) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
        (lds_bf16x4*)(__attribute__((address_space(3))) uint16_t*)at));
  };
  constexpr int kBatch = 8;
#pragma unroll
  for (int b = 0; b < 32; b += kBatch) {
    u32x2 lo[kBatch], hi[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int item = wave * 32 + b + k;  // 16 blocks of 16 T rows x 8 groups of 32 C rows
      const int c0 = (item >> 3) * 16, rb = (item & 7) * 32 + grp * 8;
      const uint16_t* at = E + (rb + (j >> 2)) * LDE + c0 + 4 * (j & 3);
      lo[k] = tr(at);
      hi[k] = tr(at + 4 * LDE);
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int item = wave * 32 + b + k;
      const int c0 = (item >> 3) * 16, rb = (item & 7) * 32 + grp * 8;
      *reinterpret_cast<u32x4*>(dst + (uint32_t)(c0 + j) * ld + rb) =
          u32x4{lo[k].x, lo[k].y, hi[k].x, hi[k].y};
    }
  }
}

// Epilogue of the [K, N] kernel, whose MFMAs take the Q fragment first: acc[i][j][r]
// of lane (fh, fr) of wave (wr, wc) is tile element (wr + 32 i + fr, wc + 32 j +
// 8 (r / 4) + 4 fh + r % 4), four consecutive columns of a row per group of four
// registers, so D and C move through the row-major LDS tile with one 64-bit access
// per four values (T, the transposed copy, with transposing reads).
template <int kDMode, bool kScaled, bool kDiag = false>
__device__ __forceinline__ void stage_rows(const GemmArgs& g, float alpha, float beta,
                                           f32x16 (&acc)[4][4], uint16_t* smem,
                                           const uint16_t* D, bool diag_tile = false) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wr = (wave >> 1) * 128, wc = (wave & 1) * 128;
  const int fr = lane & 31, fh = lane >> 5;
  uint16_t* E = smem;
  const uint32_t ldd = (uint32_t)g.ldd;
  if (kDMode == kDRowMajor) {
    constexpr int kDChunks = BM * (BN / 8) / kThreads;
    u32x4 dv[kDChunks];
#pragma unroll
    for (int i = 0; i < kDChunks; ++i) {
      const int c = tid + i * kThreads;
      dv[i] = *reinterpret_cast<const u32x4*>(D + (uint32_t)(c / (BN / 8)) * ldd + (c % (BN / 8)) * 8);
    }
#pragma unroll
    for (int i = 0; i < kDChunks; ++i) {
      const int c = tid + i * kThreads;
      *reinterpret_cast<u32x4*>(E + (c / (BN / 8)) * LDE + (c % (BN / 8)) * 8) = dv[i];
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    u32x2 draw[4][4];
    if (kDMode == kDRowMajor) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          draw[j][q] = *reinterpret_cast<const u32x2*>(E + (wr + i * 32 + fr) * LDE + wc + j * 32 +
                                                       fh * 4 + 8 * q);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint16_t* at = E + (wr + i * 32 + fr) * LDE + wc + j * 32 + fh * 4;
      float x[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        x[r] = kScaled ? alpha * acc[i][j][r] : acc[i][j][r];
        if (kDMode != kNoD) {
          const u32x2 v = draw[j][r >> 2];
          const uint32_t w = (r & 2) ? v.y : v.x;
          x[r] = __fmaf_rn(beta, bf16_bits_to_float((r & 1) ? (w >> 16) : (w & 0xFFFFu)), x[r]);
        }
      }
      if constexpr (kDiag) {
        // element (wr + 32 i + fr, wc + 32 j + 8 (r / 4) + 4 fh + r % 4) is diagonal
        if (diag_tile && i == j && wr == wc) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            if (fr == 8 * (r >> 2) + 4 * fh + (r & 3)) x[r] = x[r] + g.diag;
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<u32x2*>(at + 8 * q) =
            u32x2{pack_bf16x2(x[4 * q], x[4 * q + 1]), pack_bf16x2(x[4 * q + 2], x[4 * q + 3])};
    }
  }
}

template <int kDMode, bool kScaled, bool kDiag = false>
__device__ __forceinline__ void epilogue_rows(const GemmArgs& g, float alpha, float beta,
                                              f32x16 (&acc)[4][4], uint16_t* smem,
                                              const uint16_t* D, uint16_t* C, uint16_t* T,
                                              int64_t ldt, bool diag_tile = false) {
  stage_rows<kDMode, kScaled, kDiag>(g, alpha, beta, acc, smem, D, diag_tile);
  __syncthreads();
  store_tile(smem, C, (uint32_t)g.ldc);
  if (T) store_tile_t(smem, T, (uint32_t)ldt);
}

// The Muon update of four consecutive parameters from four bf16 results u (two
// per word, the lower element in the low half).
__device__ __forceinline__ void update4(const u32x2 u, f32x4& v, float scale, float decay,
                                        float neg_lr) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t w = u[e >> 1];
    v[e] = muon_update_element(v[e], (e & 1) ? (w >> 16) : (w & 0xFFFFu), scale, decay, neg_lr);
  }
}

// The Muon update in place of the store of C (gemm_apply_kernel).  Quad i
// (0..63) of a lane is 4 consecutive parameters of one p row and the 4 bf16
// results that update them; every access instruction covers whole contiguous
// pieces of rows (a non-temporal access to every other 16 bytes of a line
// fetches and writes lines twice).  kCols = false: p holds the tile (p rows =
// tile rows); a wave's instruction covers one whole 1 KiB row.  kCols = true: p
// holds the transposed tile, p[c][r] = tile[r][c]; a transposing LDS read gives
// lane j of a 16-lane group the 4 consecutive elements of p row c0 + j at
// columns t .. t + 3, and the four groups take adjacent t, so an instruction
// covers 64 contiguous bytes of each of 16 p rows (the quad's other half the
// next 64).
template <bool kCols>
__device__ __forceinline__ uint32_t apply_offset(int i, uint32_t ld) {
  const int tid = threadIdx.x;
  if constexpr (!kCols) {
    const int q = tid + i * kThreads;
    return (uint32_t)(q >> 6) * ld + (q & 63) * 4;
  } else {
    const int lane = tid & 63, item = (tid >> 6) * 32 + (i >> 1);
    const int c0 = (item >> 3) * 16, t = (item & 7) * 32 + 16 * (i & 1) + 4 * (lane >> 4);
    return (uint32_t)(c0 + (lane & 15)) * ld + t;
  }
}

template <bool kCols>
__device__ __forceinline__ u32x2 apply_source(const uint16_t* E, int i) {
  const int tid = threadIdx.x;
  if constexpr (!kCols) {
    const int q = tid + i * kThreads;
    return *reinterpret_cast<const u32x2*>(E + (q >> 6) * LDE + (q & 63) * 4);
  } else {
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
    // lane j, slot e <- element j % 4 of source lane 4 e + j / 4 (ds_read_b64_tr_b16):
    // source lane s reads tile row t + s / 4, columns c0 + 4 (s % 4) .. + 3, so lane j
    // receives tile rows t .. t + 3 of column c0 + j
    const int lane = tid & 63, j = lane & 15, item = (tid >> 6) * 32 + (i >> 1);
    const int c0 = (item >> 3) * 16, t = (item & 7) * 32 + 16 * (i & 1) + 4 * (lane >> 4);
    const uint16_t* e = E + (t + (j >> 2)) * LDE + c0 + 4 * (j & 3);
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
        (lds_bf16x4*)(__attribute__((address_space(3))) uint16_t*)e));
  }
}

// The whole epilogue of one tile: the accumulators go through the LDS tile as
// bf16 (the values the store of X' would write), then the parameters are
// updated in four batches of 16 quads, every load of a batch in flight before
// its first update.  Measured against the separate finish pass on the config-5
// batch (Muon step, round-robin on one box): 39.14 -> 38.77 ms per step with
// 32-byte chunks per lane; a rolling look-ahead (a load issued with every
// update) gave 38.84, and issuing the first loads before the staging spilled
// registers.
template <bool kScaled, bool kCols>
__device__ __forceinline__ void epilogue_apply(const GemmArgs& g, float alpha, f32x16 (&acc)[4][4],
                                               uint16_t* smem, float* p, uint32_t ld, float scale,
                                               float decay, float neg_lr) {
  constexpr int kQuads = 64, kBatch = 16;
  stage_rows<kNoD, kScaled>(g, alpha, 0.0f, acc, smem, nullptr);
  __syncthreads();
#pragma unroll
  for (int b0 = 0; b0 < kQuads; b0 += kBatch) {
    f32x4 v[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i)
      v[i] = load_stream<true>(reinterpret_cast<const f32x4*>(p + apply_offset<kCols>(b0 + i, ld)));
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      update4(apply_source<kCols>(smem, b0 + i), v[i], scale, decay, neg_lr);
      store_stream<true>(reinterpret_cast<f32x4*>(p + apply_offset<kCols>(b0 + i, ld)), v[i]);
    }
  }
}

// kQKN: Q is stored [K, N] (row-major, N contiguous) instead of [N, K]; its
// fragments come from the LDS through transposing reads.  kApply (with kQKN):
// the Muon update of GemmApply in place of the store of C.
template <bool kQKN, int kDMode, bool kScaled, bool kDiag, bool kApply>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, const GemmApply* ap) {
  static_assert(!kApply || (kQKN && kDMode == kNoD && !kDiag), "the update rides on X' = B' X");
  __shared__ __attribute__((aligned(16))) uint16_t smem[kSmemElems];

  // XCD-aware numbering: the grid is a multiple of 8; XCD x = id % 8 runs the
  // contiguous logical range [x * per_xcd, (x + 1) * per_xcd).
  const int64_t per_xcd = (int64_t)gridDim.x / 8;
  const int64_t logical = (int64_t)(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
  if (logical >= g.total_tiles) return;
  const int64_t b = logical / g.tiles_per_matrix;
  int tr, tc;
  tile_of(g, (int)(logical - b * g.tiles_per_matrix), tr, tc);
  const int64_t row0 = (int64_t)tr * BM, col0 = (int64_t)tc * BN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar registers
  // The tile's operand bases are wave-uniform; readfirstlane states it, so the
  // buffer descriptors built from them live in scalar registers.
  auto uniform = [](const uint16_t* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const uint16_t*>(lo | (hi << 32));
  };
  const uint16_t* P = uniform(g.P + b * g.sp + row0 * g.ldp);
  const uint16_t* Q = uniform(g.Q + b * g.sq + (kQKN ? col0 : col0 * g.ldq));

  // DMA assignment: a wave loads rows [64 w, 64 w + 64) of an operand
  // sub-tile, 8 rows per instruction; lane l -> row base + l / 8, LDS slot
  // l % 8, which holds the global 16-byte chunk slot ^ swz(row).  The eight
  // lanes of a row fetch the eight chunks of one 128-byte line (one full-line
  // request).  A lane's byte offset from the operand's stage base is the same
  // for every stage, so it is computed once; each load is then a uniform base
  // (scalar registers) plus a 32-bit per-lane offset, the cheapest form to
  // issue (the host keeps 256 rows of a leading dimension under 4 GiB).
  const int lrow = lane >> 3, lslot = lane & 7;
  auto swz = [](int r) { return (r ^ (r >> 3)) & 7; };
  const int64_t KT = g.K / BK;  // >= 1
  uint32_t offp[8], offq[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = wave * 64 + j * 8 + lrow;
    const uint32_t c = (uint32_t)(lslot ^ swz(r));
    offp[j] = (uint32_t)r * (uint32_t)g.ldp * 2u + c * 16u;
    if constexpr (kQKN) {
      // [K, N] operand: an instruction loads two 512-byte k-rows of the stage;
      // lane l -> k-row 16 w + 2 j + l / 32, slot l % 32 holding global chunk
      // slot ^ (4 (row % 4)).  Eight adjacent lanes still cover one 128-byte line.
      const int rk = wave * 16 + j * 2 + (lane >> 5);
      const uint32_t ck = (uint32_t)((lane & 31) ^ (4 * (rk & 3)));
      offq[j] = (uint32_t)rk * (uint32_t)g.ldq * 2u + ck * 16u;
    } else {
      offq[j] = (uint32_t)r * (uint32_t)g.ldq * 2u + c * 16u;
    }
  }
  // Load j (0..7) of operand Q (or P) of stage `stage` into ring slot `slot`;
  // stages past the end load the last one again (never read; it keeps every
  // step's load count, and so the vmcnt bookkeeping, the same).
  //
  // With a [K, N] Q the load is written as inline assembly, not the
  // compiler's builtin: the compiler then tracks no LDS-DMA writes and cannot
  // add vmcnt(0) waits in front of the transposing LDS reads, which it does
  // for every one of them (it cannot prove them disjoint from a pending DMA),
  // serializing the pipeline.  Completion is managed explicitly anyway: the
  // vmcnt waits before the per-stage barriers, and the vmcnt(0) of the
  // barrier before the epilogue.  The [N, K] form keeps the builtin, which
  // the compiler schedules a little tighter (about 120 cycles per stage).
  auto issue_load = [&](bool q, int slot, int64_t stage, int j) {
    const int64_t k0 = (stage < KT ? stage : KT - 1) * BK;
    const uint16_t* base = q ? (kQKN ? Q + k0 * g.ldq : Q + k0) : P + k0;
    const uint16_t* dst = smem + slot * kSubTile +
                          ((q && kQKN) ? (wave * 16 + j * 2) * BN : (wave * 64 + j * 8) * BK);
    const uint32_t off = q ? offq[j] : offp[j];
    if constexpr (kQKN) {
      // raw buffer descriptor: 48-bit base, stride 0, no range limit beyond
      // the 32-bit offsets, 32-bit data format
      const uint64_t addr = reinterpret_cast<uint64_t>(base);
      const u32x4 rsrc = u32x4{(uint32_t)addr, (uint32_t)(addr >> 32) & 0xFFFFu, 0xFFFFFFFFu,
                               0x00020000u};
      const uint32_t m0 = (uint32_t)reinterpret_cast<uintptr_t>(
          (__attribute__((address_space(3))) const uint16_t*)dst);
      // M0 (the instruction's LDS base) is an input the compiler sets; the
      // s_nop is the wait state between an M0 write and an LDS DMA
      asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                   :
                   : "v"(off), "s"(rsrc), "{m0}"(m0)
                   : "memory");
    } else {
      const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint16_t*>(base), (short)0, (int)0xFFFFFFFF, 0x00020000);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)dst, 16, off, 0, 0, 0);
    }
  };

  const int wr = (wave >> 1) * 128, wc = (wave & 1) * 128;
  const int fr = lane & 31, fh = lane >> 5;  // fragment row in a 32-row tile, k half
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

  // Fragment of row R, 16-byte chunk c (c = 2 kk + k half, kk < 4): swizzled slot.
  auto frag = [&](const uint16_t* sub, int R, int c) {
    return *reinterpret_cast<const bf16x8*>(sub + R * BK + ((c ^ swz(R)) * 8));
  };

  // Workgroup barrier for LDS only: the memory clobber keeps the compiler from
  // moving LDS accesses across it and no vmcnt wait is attached, so younger
  // loads stay in flight (__syncthreads would drain them).
  auto lds_barrier = []() { asm volatile("s_barrier" ::: "memory"); };
  // Fragments of one 16-deep sub-step: 4 P row-blocks and 4 Q row-blocks.
  struct Frags {
    bf16x8 a[4], q[4];
  };
  auto mfma = [&](int n, const Frags& f) {
    const int i = n >> 2, j = n & 3;
    if constexpr (kQKN || kDiag)  // row-chunk accumulators (epilogue_rows)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.q[j], f.a[i], acc[i][j], 0, 0, 0);
    else
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[i], f.q[j], acc[i][j], 0, 0, 0);
  };
  // [K, N] operand: half h (k 4h .. 4h + 3 of this lane's 8) of the Q
  // fragment of columns n0 .. n0 + 31 at depth kk.  In each 16-lane group
  // ds_read_b64_tr_b16 hands destination lane j, slot e, element j % 4 of
  // source lane 4 e + j / 4 (checked on the device); so source lane s reads
  // row kbase + s / 4, columns n0' + 4 (s % 4) .. + 3, and lane j receives
  // rows kbase .. kbase + 3 of column n0' + j: the MFMA B layout.  The chunk
  // swizzle puts the 4 rows x 4 chunks a half-wave reads on 16 distinct banks.
  auto frag_kn = [&](const uint16_t* sub, int n0, int kk, int h) {
    const int j = lane & 15;
    const int row = kk * 16 + 8 * (lane >> 5) + 4 * h + (j >> 2);
    const int col = n0 + 16 * ((lane >> 4) & 1) + 4 * (j & 3);
    const uint16_t* at = sub + row * BN + ((((col >> 3) ^ (4 * (row & 3))) << 3) | (col & 7));
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
    // the result is used only as a whole: extracting elements of this
    // builtin's vector has been miscompiled
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(
        (lds_bf16x4*)(__attribute__((address_space(3))) uint16_t*)at));
  };
  // Fragment reads of one sub-step: 8 (P and Q rows), or 12 with a [K, N]
  // Q (4 P rows and two halves per Q fragment), read n of them.
  constexpr int kReads = kQKN ? 12 : 8;
  auto read = [&](int n, Frags& f, int pslot, int qslot, int kk) {
    if constexpr (kQKN) {
      const int i = n / 3, part = n % 3;
      if (part == 0) {
        f.a[i] = frag(smem + pslot * kSubTile, wr + i * 32 + fr, kk * 2 + fh);
      } else {
        const u32x2 half = frag_kn(smem + qslot * kSubTile, wc + i * 32, kk, part - 1);
        u32x4 q = __builtin_bit_cast(u32x4, f.q[i]);
        if (part == 1) q.x = half.x, q.y = half.y;
        else q.z = half.x, q.w = half.y;
        f.q[i] = __builtin_bit_cast(bf16x8, q);
      }
    } else {
      const int i = n >> 1;
      if (n & 1)
        f.q[i] = frag(smem + qslot * kSubTile, wc + i * 32 + fr, kk * 2 + fh);
      else
        f.a[i] = frag(smem + pslot * kSubTile, wr + i * 32 + fr, kk * 2 + fh);
    }
  };

  // Pipeline.  The LDS is a ring of five 32 KiB slots holding operand
  // sub-tiles in the order P0 Q0 P1 Q1 P2 ... (item x = 2 stage + operand in
  // slot x % 5), and two register sets of fragments (F0, F1) hold one 16-deep
  // sub-step each.  Step t computes stage t in four sub-steps; each
  // sub-step's 16 MFMAs run while the next sub-step's 8 fragments are read.
  // Before the last sub-step one barrier (after this wave's vmcnt) frees the
  // two slots of stage t -- every wave has its last fragments in registers --
  // and publishes stage t + 1; the last sub-step then reads the first
  // fragments of stage t + 1.  Loads: the load path accepts about 64 bytes per
  // clock per CU, so a stage (64 KiB) issued in one sub-step stalls the
  // issuing waves; here every sub-step issues 4 of a wave's loads (a quarter
  // stage): Q of stage t + 2 into the freed P slot of stage t in the last
  // sub-step of step t and the first of step t + 1 (due at the barrier of step
  // t + 1), P of stage t + 3 into the freed Q slot in the second and third
  // sub-steps of step t + 1 (due a step later).  The scheduling barriers pin
  // the interleave: without them the compiler is free to hoist the LDS waits
  // above the MFMAs.
  Frags f0, f1;
  // One sub-step: 16 MFMAs on `cur`, the 8 fragments of `nxt` read from the
  // slots (rp, rq) at depth kk, and loads j0 .. j0 + 3 of (lq ? Q : P) of
  // stage lstage into slot ls_.
  auto substep = [&](const Frags& cur, Frags& nxt, int rp, int rq, int kk, bool lq, int ls_,
                     int64_t lstage, int j0) {
#pragma unroll
    for (int n = 0; n < 16; ++n) {
      mfma(n, cur);
      __builtin_amdgcn_sched_barrier(0);
      if (n < kReads) read(n, nxt, rp, rq, kk);
      if (n >= 2 && n < 10 && (n & 1) == 0) issue_load(lq, ls_, lstage, j0 + ((n - 2) >> 1));
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): next fragments in registers
  };
  // ps/qs: slots of stage t's P and Q; the slots of stage t + 1 and of P of
  // stage t + 2 follow in ring order.
  auto step = [&](int64_t t, int ps, auto next_tag) {
    constexpr bool kNext = decltype(next_tag)::value;
    const int qs = ps + 1 == kSlots ? 0 : ps + 1;
    const int ps1 = qs + 1 == kSlots ? 0 : qs + 1;
    const int qs1 = ps1 + 1 == kSlots ? 0 : ps1 + 1;
    const int ps2 = qs1 + 1 == kSlots ? 0 : qs1 + 1;
    substep(f0, f1, ps, qs, 1, true, qs1, t + 1, 4);   // Q of t + 1, loads 4..7
    substep(f1, f0, ps, qs, 2, false, ps2, t + 2, 0);  // P of t + 2, loads 0..3
    substep(f0, f1, ps, qs, 3, false, ps2, t + 2, 4);  // P of t + 2, loads 4..7
    mfma(0, f1);
    mfma(1, f1);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kNext) {
      __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8): all but P of t + 2 landed for this wave
      lds_barrier();
    }
#pragma unroll
    for (int n = 2; n < 16; ++n) {
      mfma(n, f1);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (kNext) {
        if (n - 2 < kReads) read(n - 2, f0, ps1, qs1, 0);
        // Q of t + 2 into the freed P slot of t, loads 0..3
        if (n >= 6 && n < 14 && (n & 1) == 0) issue_load(true, ps, t + 2, (n - 6) >> 1);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (kNext) __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  };

  // Prologue: P0 Q0 P1 in full and the first half of Q1 (slots 0..3), then
  // stage 0 is waited for and its first fragments read.
#pragma unroll
  for (int j = 0; j < 8; ++j) issue_load(false, 0, 0, j);
#pragma unroll
  for (int j = 0; j < 8; ++j) issue_load(true, 1, 0, j);
#pragma unroll
  for (int j = 0; j < 8; ++j) issue_load(false, 2, 1, j);
#pragma unroll
  for (int j = 0; j < 4; ++j) issue_load(true, 3, 1, j);
  __builtin_amdgcn_s_waitcnt(0x0F7C);  // vmcnt(12): P0 and Q0 landed for this wave
  lds_barrier();
#pragma unroll
  for (int n = 0; n < kReads; ++n) read(n, f0, 0, 1, 0);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)

  int ps = 0;
  for (int64_t t = 0; t + 1 < KT; ++t) {
    step(t, ps, std::true_type{});
    ps = ps + 2 >= kSlots ? ps + 2 - kSlots : ps + 2;
  }
  step(KT - 1, ps, std::false_type{});
  __syncthreads();  // all fragment reads and trailing loads done before the epilogue reuses the LDS

  // ---- epilogue ------------------------------------------------------------
  if constexpr (kApply) {
    float alpha = g.alpha;
    if (g.bscale != nullptr) alpha *= g.bscale[b];
    if (ap->transposed[b] == 0)  // p [m, n]: the tile's rows are p rows
      epilogue_apply<kScaled, false>(g, alpha, acc, smem, ap->p[b] + row0 * ap->n + col0,
                                     (uint32_t)ap->n, ap->scale[b], ap->decay, ap->neg_lr);
    else  // p [n, m]: the tile's columns are p rows
      epilogue_apply<kScaled, true>(g, alpha, acc, smem, ap->p[b] + col0 * ap->m + row0,
                                    (uint32_t)ap->m, ap->scale[b], ap->decay, ap->neg_lr);
    return;
  }
  const uint16_t* D = nullptr;
  if (g.D) D = g.D + b * g.sd + row0 * g.ldd + col0;
  uint16_t* T = nullptr;  // transposed destination: Ct, or the mirror tile
  int64_t ldt = 0;
  if (g.flags & MORPH_GEMM_SYMMETRIC) {
    if (tr != tc) {
      T = g.C + b * g.sc + col0 * g.ldc + row0;
      ldt = g.ldc;
    }
  } else if (g.Ct) {
    T = g.Ct + b * g.sct + col0 * g.ldct + row0;
    ldt = g.ldct;
  }
  uint16_t* C = g.C + b * g.sc + row0 * g.ldc + col0;
  float alpha = g.alpha, beta = g.beta;
  if (g.bscale != nullptr) {
    const float s = g.bscale[b];
    alpha *= s;
    beta *= s;
  }
  // The epilogue variant is the kernel's (chosen on the host: D or not, alpha
  // multiply or not -- alpha == 1 without per-matrix factors skips it, exact then --
  // diagonal add or not); only a diagonal tile of a symmetric product takes the add.
  if constexpr (kQKN)
    epilogue_rows<kDMode, kScaled>(g, alpha, beta, acc, smem, D, C, T, ldt);
  else if constexpr (kDiag)
    epilogue_rows<kDMode, kScaled, true>(g, alpha, beta, acc, smem, D, C, T, ldt, tr == tc);
  else if (kDiag && tr == tc)
    epilogue<kDMode, kScaled, true>(g, alpha, beta, acc, smem, D, C, T, ldt);
  else
    epilogue<kDMode, kScaled, false>(g, alpha, beta, acc, smem, D, C, T, ldt);
}

template <bool kQKN, int kDMode, bool kScaled, bool kDiag>
__global__ __launch_bounds__(kThreads, 1) void gemm_kernel(const GemmArgs g) {
  gemm_tile<kQKN, kDMode, kScaled, kDiag, false>(g, nullptr);
}

template <bool kScaled>
__global__ __launch_bounds__(kThreads, 1) void gemm_apply_kernel(const GemmArgs g,
                                                                 const GemmApply ap) {
  gemm_tile<true, kNoD, kScaled, false, true>(g, &ap);
}

}  // namespace
}  // namespace morph

int morph::gemm_nt_bf16_scaled(const uint16_t* P, const uint16_t* Q, const uint16_t* D,
                               uint16_t* C, uint16_t* Ct, int64_t M, int64_t N, int64_t K,
                               int64_t batch, int64_t ldp, int64_t ldq, int64_t ldd,
                               int64_t ldc, int64_t ldct, int64_t stride_p, int64_t stride_q,
                               int64_t stride_d, int64_t stride_c, int64_t stride_ct,
                               float alpha, float beta, const float* bscale, float diag,
                               int flags, void* stream) {
  if (P == nullptr || Q == nullptr || C == nullptr || M < 0 || N < 0 || K <= 0 || batch < 0)
    return MORPH_EINVAL;
  auto misaligned = [](const void* p, uintptr_t a) {
    return p != nullptr && (reinterpret_cast<uintptr_t>(p) % a) != 0;
  };
  if (misaligned(P, 16) || misaligned(Q, 16) || misaligned(C, 16) || misaligned(D, 16) ||
      misaligned(Ct, 16))
    return MORPH_EINVAL;
  if (M % BM || N % BN || K % MORPH_GEMM_TILE_K) return MORPH_ERANGE;
  if (flags & ~(MORPH_GEMM_SYMMETRIC | MORPH_GEMM_Q_KN)) return MORPH_EINVAL;
  const bool symmetric = (flags & MORPH_GEMM_SYMMETRIC) != 0;
  const bool qkn = (flags & MORPH_GEMM_Q_KN) != 0;
  if (ldp < K || ldq < (qkn ? N : K) || ldc < N || (D && ldd < N) || (Ct && ldct < M))
    return MORPH_EINVAL;
  // 16-byte loads and stores of rows: every leading dimension and batch stride a multiple of 8
  if ((ldp | ldq | ldc | stride_p | stride_q | stride_c) % 8 ||
      (D && (ldd | stride_d) % 8) || (Ct && (ldct | stride_ct) % 8))
    return MORPH_EINVAL;
  if (symmetric && (M != N || Ct != nullptr || qkn)) return MORPH_EINVAL;
  if (diag != 0.0f && !symmetric) return MORPH_EINVAL;
  // operand-load and epilogue offsets inside a tile are 32-bit: 255 rows of
  // the widest leading dimension
  constexpr int64_t kMaxLd = int64_t(1) << 23;
  if (ldp > kMaxLd || ldq > kMaxLd || ldc > kMaxLd || (D && ldd > kMaxLd) ||
      (Ct && ldct > kMaxLd))
    return MORPH_ERANGE;
  if (M == 0 || N == 0 || batch == 0) return MORPH_OK;
  // Outputs are written while other tiles still read P and Q: the address
  // ranges of C and Ct may not meet those of P and Q (D may alias C).
  auto span = [&](const uint16_t* base, int64_t stride, int64_t rows, int64_t ld,
                  int64_t cols) {
    const uintptr_t lo = reinterpret_cast<uintptr_t>(base);
    return std::pair<uintptr_t, uintptr_t>(
        lo, lo + 2 * (uintptr_t)((batch - 1) * stride + (rows - 1) * ld + cols));
  };
  auto meet = [](std::pair<uintptr_t, uintptr_t> a, std::pair<uintptr_t, uintptr_t> b) {
    return a.first < b.second && b.first < a.second;
  };
  const auto sp = span(P, stride_p, M, ldp, K);
  const auto sq = qkn ? span(Q, stride_q, K, ldq, N) : span(Q, stride_q, N, ldq, K);
  const auto sc = span(C, stride_c, M, ldc, N);
  if (meet(sc, sp) || meet(sc, sq)) return MORPH_EINVAL;
  if (Ct) {
    const auto st = span(Ct, stride_ct, N, ldct, M);
    if (meet(st, sp) || meet(st, sq) || meet(st, sc)) return MORPH_EINVAL;
  }
  const int64_t tm = M / BM, tn = N / BN;
  const int64_t per = symmetric ? tm * (tm + 1) / 2 : tm * tn;
  const int64_t total = batch * per;
  const int64_t grid = (total + 7) / 8 * 8;
  if (per > (int64_t(1) << 31) - 1 || grid > (int64_t(1) << 31) - 1) return MORPH_ERANGE;
  GemmArgs g{P, Q, D, C, Ct, K, ldp, ldq, ldd, ldc, ldct,
             stride_p, stride_q, stride_d, stride_c, stride_ct, alpha, beta, bscale, diag,
             (int32_t)tm, (int32_t)tn, (int32_t)per, flags, total};
  // one kernel per epilogue variant keeps each kernel's register demand to its own path
  const bool scaled = bscale != nullptr || alpha != 1.0f;
  const bool has_d = D != nullptr, has_diag = diag != 0.0f;
  const dim3 gd((unsigned)grid), bd(kThreads);
  hipStream_t s = as_stream(stream);
#define MORPH_GEMM_LAUNCH(Q, DM, SC, DG) hipLaunchKernelGGL((gemm_kernel<Q, DM, SC, DG>), gd, bd, 0, s, g)
  if (qkn) {
    if (has_d) {
      if (scaled) MORPH_GEMM_LAUNCH(true, kDRowMajor, true, false);
      else MORPH_GEMM_LAUNCH(true, kDRowMajor, false, false);
    } else {
      if (scaled) MORPH_GEMM_LAUNCH(true, kNoD, true, false);
      else MORPH_GEMM_LAUNCH(true, kNoD, false, false);
    }
  } else if (has_diag) {
    if (has_d) MORPH_GEMM_LAUNCH(false, kDRowMajor, true, true);
    else MORPH_GEMM_LAUNCH(false, kNoD, true, true);
  } else if (has_d) {
    if (scaled) MORPH_GEMM_LAUNCH(false, kDRowMajor, true, false);
    else MORPH_GEMM_LAUNCH(false, kDRowMajor, false, false);
  } else {
    if (scaled) MORPH_GEMM_LAUNCH(false, kNoD, true, false);
    else MORPH_GEMM_LAUNCH(false, kNoD, false, false);
  }
#undef MORPH_GEMM_LAUNCH
  return launch_status();
}

int morph::gemm_kn_apply(const uint16_t* P, const uint16_t* Q, int64_t M, int64_t N, int64_t K,
                         int64_t batch, int64_t ldp, int64_t ldq, int64_t stride_p,
                         int64_t stride_q, const float* bscale, const GemmApply& ap,
                         void* stream) {
  if (P == nullptr || Q == nullptr || M <= 0 || N <= 0 || K <= 0 || batch <= 0 ||
      batch > kGemmMaxApply)
    return MORPH_EINVAL;
  if (M % BM || N % BN || K % MORPH_GEMM_TILE_K) return MORPH_ERANGE;
  if (ap.m != M || ap.n != N || ldp < K || ldq < N || (ldp | ldq | stride_p | stride_q) % 8)
    return MORPH_EINVAL;
  if ((reinterpret_cast<uintptr_t>(P) | reinterpret_cast<uintptr_t>(Q)) % 16) return MORPH_EINVAL;
  for (int64_t b = 0; b < batch; ++b)
    if (ap.p[b] == nullptr || reinterpret_cast<uintptr_t>(ap.p[b]) % 16 ||
        (ap.transposed[b] != 0 && ap.transposed[b] != 1))
      return MORPH_EINVAL;
  // 32-bit offsets inside a tile: 255 rows of the widest row length
  constexpr int64_t kMaxLd = int64_t(1) << 23;
  if (ldp > kMaxLd || ldq > kMaxLd || M > kMaxLd || N > kMaxLd) return MORPH_ERANGE;
  const int64_t tm = M / BM, tn = N / BN, per = tm * tn, total = batch * per;
  const int64_t grid = (total + 7) / 8 * 8;
  if (grid > (int64_t(1) << 31) - 1) return MORPH_ERANGE;
  GemmArgs g{P, Q, nullptr, nullptr, nullptr, K, ldp, ldq, 0, 0, 0,
             stride_p, stride_q, 0, 0, 0, 1.0f, 0.0f, bscale, 0.0f,
             (int32_t)tm, (int32_t)tn, (int32_t)per, MORPH_GEMM_Q_KN, total};
  hipStream_t s = as_stream(stream);
  if (bscale != nullptr)
    hipLaunchKernelGGL(gemm_apply_kernel<true>, dim3((unsigned)grid), dim3(kThreads), 0, s, g, ap);
  else
    hipLaunchKernelGGL(gemm_apply_kernel<false>, dim3((unsigned)grid), dim3(kThreads), 0, s, g, ap);
  return launch_status();
}

using namespace morph;

extern "C" int morph_gemm_nt_bf16(const uint16_t* P, const uint16_t* Q, const uint16_t* D,
                                  uint16_t* C, uint16_t* Ct, int64_t M, int64_t N, int64_t K,
                                  int64_t batch, int64_t ldp, int64_t ldq, int64_t ldd,
                                  int64_t ldc, int64_t ldct, int64_t stride_p, int64_t stride_q,
                                  int64_t stride_d, int64_t stride_c, int64_t stride_ct,
                                  float alpha, float beta, int flags, void* stream) {
  return gemm_nt_bf16_scaled(P, Q, D, C, Ct, M, N, K, batch, ldp, ldq, ldd, ldc, ldct, stride_p,
                             stride_q, stride_d, stride_c, stride_ct, alpha, beta, nullptr, 0.0f, flags,
                             stream);
}
