// Batched matmul C[b] = A[b] . B[b] (+ C_old[b]) on strided views.
//
// fp32 runs on the gfx950 matrix cores (v_mfma_f32_32x32x2_f32).  The
// reference (src/cpp/ops/matmul.cu) has a SIMT 128x128x16 kernel that only
// accepts contiguous operands and sends every transposed operand -- hence
// both backward products of MatmulOp (ops_binary.py:264-267) -- to a naive
// one-thread-per-output kernel.  Here each operand is read in place in
// whichever orientation it has:
//
//   layout K  : the reduction index k is the unit-stride one (A row-major,
//               or B = W^T of a row-major W).  Stored in LDS as [mn][k].
//   layout MN : the m (or n) index is unit-stride (A = X^T of a row-major
//               X, or B row-major).  Stored in LDS as [k][mn].
//   layout GEN: anything else (e.g. `[:, ::2]` views): scalar loads, stored
//               as [mn][k].
//
// Workgroup tile 128x128, k-tile 32, 256 threads = 4 waves in a 2x2 grid,
// each wave owns a 64x64 block = 2x2 MFMA 32x32 blocks (64 accumulator
// registers per lane).  Global loads for k-tile t+1 are issued before the
// MFMAs of tile t; LDS is double buffered so one barrier per k-tile
// suffices.  Workgroups are numbered so that consecutive tiles of a group of
// 8 tile-rows land on the same XCD (gfx950 dispatches workgroups round-robin
// over its 8 XCDs, each with its own L2).
//
// MFMA k assignment: in MFMA step kk (0..15) of a k-tile, the lanes of wave
// half h (lane / 32) supply k = h*16 + kk, for A and B alike, so each lane's
// 16 fragments of a k-tile are contiguous in a [mn][k] LDS row.  The sum over
// k is unchanged; only the fp32 accumulation order differs from the
// reference's sequential loop (|diff| <= 1e-4 * (|A|.|B|) is the parity
// bound).  Accumulate mode adds C_old after the full dot product: one
// rounding, like the reference's `x._grad += grad`.
//
// When both operands are in a vector layout and K is a multiple of 32, the
// operands skip the register round trip: mm_f32_mfma_dl_kernel stages them
// with gfx950's direct global-to-LDS loads (same tiles, same MFMA schedule).
// Large products (M, N multiples of 256, K of 64, a 256x256 tile per CU)
// use mm_f32_mfma_wide_kernel: 256x256 tiles, 8 waves of 128x64.
//
// Other dtypes (fp64, int32, int64) use a tiled SIMT kernel that accumulates
// in k order exactly like the reference's CPU loop (matmul.cu:33-45).
#include <algorithm>

#include "nt_internal.h"

namespace nt {

typedef float floatx16 __attribute__((ext_vector_type(16)));

// Largest split of K for a single product with fewer wide tiles than CUs.
#ifndef NT_MM_SPLITK_MAX
#define NT_MM_SPLITK_MAX 8
#endif
// The split-K sum kernel is instantiated for 2, 4 and 8 slices only.
static_assert(NT_MM_SPLITK_MAX == 1 || NT_MM_SPLITK_MAX == 2 ||
                  NT_MM_SPLITK_MAX == 4 || NT_MM_SPLITK_MAX == 8,
              "NT_MM_SPLITK_MAX must be 1, 2, 4 or 8");

constexpr int MM_BM = 128, MM_BN = 128, MM_BK = 32, MM_THREADS = 256;
constexpr int MM_KPAD = MM_BK + 4;  // [mn][k] row length (floats)
constexpr int MM_MNPAD = MM_BM + 4; // [k][mn] row length (floats)
constexpr int MM_REGION = (MM_BM * MM_KPAD > MM_BK * MM_MNPAD)
                              ? MM_BM * MM_KPAD
                              : MM_BK * MM_MNPAD; // floats per operand stage
constexpr int MM_MAX_BATCH = NT_MAX_DIMS - 2;

enum { LAY_K = 0, LAY_MN = 1, LAY_GEN = 2 };

struct MMArgs {
  const float *A;
  const float *B;
  float *C;
  int64_t M, N, K;
  int64_t sAm, sAk, sBk, sBn, sCm, sCn;
  int nb;
  int64_t bshape[MM_MAX_BATCH];
  int64_t bsA[MM_MAX_BATCH], bsB[MM_MAX_BATCH], bsC[MM_MAX_BATCH];
  int64_t tiles_m, tiles_n;
  int accumulate;
  // Wide kernel, split over K: blockIdx.y = s takes k in [s kslice,
  // (s + 1) kslice) and writes its raw sum to part + s M N ([M][N]
  // contiguous); mm_splitk_sum_kernel adds the slices.  part == nullptr: no
  // split (kslice == K), results go to C.
  int64_t kslice;
  float *part;
  // Optional bias added to every output row in the epilogue, C = fl(acc) +
  // bias[n] (one fp32 rounding after the product's own, as a separate add
  // would give); nullptr: none.  Never combined with accumulate.
  const float *bias;
  int64_t sBias;
};

// Operand tile loader: global -> registers -> LDS.  ROWS x MM_BK tile of
// the operand in (mn, k) coordinates, where mn is m for A and n for B.
// s_mn / s_k are the element strides of the mn and k indices.
template <int LAY> struct TileLoad {
  float4 r[4];
  __device__ __forceinline__ void load(const float *p, int64_t mn0, int64_t k0,
                                       int64_t MN, int64_t K, int64_t s_mn,
                                       int64_t s_k, int t) {
    if constexpr (LAY == LAY_K) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t mn = mn0 + (t >> 3) + 32 * i;
        const int64_t k = k0 + (t & 7) * 4;
        if (mn < MN && k < K)
          r[i] = *reinterpret_cast<const float4 *>(p + mn * s_mn + k);
        else
          r[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    } else if constexpr (LAY == LAY_MN) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t k = k0 + (t >> 5) + 8 * i;
        const int64_t mn = mn0 + (t & 31) * 4;
        if (mn < MN && k < K)
          r[i] = *reinterpret_cast<const float4 *>(p + mn + k * s_k);
        else
          r[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int flat = t + MM_THREADS * (4 * i + q); // 0..4095
          const int64_t mn = mn0 + (flat >> 5);
          const int64_t k = k0 + (flat & 31);
          v[q] = (mn < MN && k < K) ? p[mn * s_mn + k * s_k] : 0.f;
        }
        r[i] = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  }
  __device__ __forceinline__ void store(float *lds, int t) const {
    if constexpr (LAY == LAY_K) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int mn = (t >> 3) + 32 * i, k = (t & 7) * 4;
        *reinterpret_cast<float4 *>(lds + mn * MM_KPAD + k) = r[i];
      }
    } else if constexpr (LAY == LAY_MN) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int k = (t >> 5) + 8 * i, mn = (t & 31) * 4;
        *reinterpret_cast<float4 *>(lds + k * MM_MNPAD + mn) = r[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v[4] = {r[i].x, r[i].y, r[i].z, r[i].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int flat = t + MM_THREADS * (4 * i + q);
          lds[(flat >> 5) * MM_KPAD + (flat & 31)] = v[q];
        }
      }
    }
  }
};

// Fragment read: element (mn, k) of the staged tile.
template <int LAY>
__device__ __forceinline__ float frag(const float *lds, int mn, int k) {
  if constexpr (LAY == LAY_MN)
    return lds[k * MM_MNPAD + mn];
  else
    return lds[mn * MM_KPAD + k];
}

// Workgroup -> (batch, tile) with an XCD-contiguous numbering, then groups
// of 8 tile-rows walked column by column; A, B, C advanced to the batch.
struct TileCoord {
  int64_t m0, n0;
  const float *A, *B;
  float *C;
};

template <int BM = MM_BM, int BN = MM_BN>
__device__ __forceinline__ TileCoord mm_tile_coord(const MMArgs &g) {
  const int64_t per_batch = g.tiles_m * g.tiles_n;
  int64_t bid = blockIdx.x;
  const int64_t nblk = gridDim.x;
  if (nblk % 8 == 0)
    bid = (bid % 8) * (nblk / 8) + bid / 8;
  const int64_t batch = bid / per_batch;
  const int64_t tile = bid - batch * per_batch;
  constexpr int64_t GROUP = 8;
  const int64_t group = tile / (GROUP * g.tiles_n);
  const int64_t first_m = group * GROUP;
  const int64_t gsize = (g.tiles_m - first_m) < GROUP ? (g.tiles_m - first_m)
                                                       : GROUP;
  const int64_t in_group = tile - group * GROUP * g.tiles_n;
  TileCoord tc;
  tc.m0 = (first_m + in_group % gsize) * BM;
  tc.n0 = (in_group / gsize) * BN;
  tc.A = g.A;
  tc.B = g.B;
  tc.C = g.C;
  int64_t rem = batch;
  for (int d = g.nb - 1; d >= 0; --d) {
    const int64_t q = rem / g.bshape[d];
    const int64_t c = rem - q * g.bshape[d];
    rem = q;
    tc.A += c * g.bsA[d];
    tc.B += c * g.bsB[d];
    tc.C += c * g.bsC[d];
  }
  return tc;
}

// Lane holds column li of each 32x32 block, rows 8*(r/4) + 4*h + (r%4).
__device__ __forceinline__ void mm_epilogue(const MMArgs &g, const TileCoord &tc,
                                            const floatx16 (&acc)[2][2], int wm,
                                            int wn, int h, int li) {
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = tc.n0 + wn * 64 + j * 32 + li;
      if (col >= g.N)
        continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row =
            tc.m0 + wm * 64 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
        if (row < g.M) {
          float *dst = tc.C + row * g.sCm + col * g.sCn;
          const float v = acc[i][j][r];
          *dst = g.accumulate ? (*dst + v) : (g.bias ? v + g.bias[col * g.sBias] : v);
        }
      }
    }
}

template <int LA, int LB>
__global__ __launch_bounds__(MM_THREADS, 2) void mm_f32_mfma_kernel(MMArgs g) {
  __shared__ __align__(16) float lds[2][2][MM_REGION]; // [stage][A/B]
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int h = lane >> 5, li = lane & 31;

  const TileCoord tc = mm_tile_coord(g);
  const int64_t m0 = tc.m0, n0 = tc.n0;
  const float *A = tc.A;
  const float *B = tc.B;

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc[i][j][r] = 0.f;

  TileLoad<LA> la;
  TileLoad<LB> lb;
  const int64_t ktiles = (g.K + MM_BK - 1) / MM_BK;
  la.load(A, m0, 0, g.M, g.K, g.sAm, g.sAk, t);
  lb.load(B, n0, 0, g.N, g.K, g.sBn, g.sBk, t);
  la.store(lds[0][0], t);
  lb.store(lds[0][1], t);
  __syncthreads();

  for (int64_t kt = 0; kt < ktiles; ++kt) {
    const int cur = int(kt & 1);
    if (kt + 1 < ktiles) {
      la.load(A, m0, (kt + 1) * MM_BK, g.M, g.K, g.sAm, g.sAk, t);
      lb.load(B, n0, (kt + 1) * MM_BK, g.N, g.K, g.sBn, g.sBk, t);
    }
    const float *As = lds[cur][0];
    const float *Bs = lds[cur][1];
#pragma unroll
    for (int kk = 0; kk < 16; ++kk) {
      const int k = h * 16 + kk;
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        a[i] = frag<LA>(As, wm * 64 + i * 32 + li, k);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        b[j] = frag<LB>(Bs, wn * 64 + j * 32 + li, k);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j],
                                                           acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < ktiles) {
      la.store(lds[cur ^ 1][0], t);
      lb.store(lds[cur ^ 1][1], t);
    }
    __syncthreads();
  }

  mm_epilogue(g, tc, acc, wm, wn, h, li);
}

// ------------------------------------------ direct-to-LDS staging (gfx950)

// gfx950 can move 16 bytes per lane from global memory straight into LDS
// (global_load_lds_dwordx4): lane L of a wave lands at LDS base + 16 L, with
// the base wave-uniform.  The kernel below stages both operands that way --
// no VGPR round trip, no LDS store instructions -- when both are in a vector
// layout and K is a multiple of the 32-deep k-tile.  Each wave instruction
// fills 1 KB of a stage:
//   layout K : the stage is [128 mn][32 k] without padding, 16-byte chunks
//              swizzled within a row (dl_swz) so that fragment reads are
//              bank-conflict free.  One instruction covers 8 rows.
//   layout MN: the stage is [32 k][128 mn]; one instruction covers 2 k rows.
// Rows (columns) past M (N) re-read the last valid one: their results are
// never stored.
constexpr int DL_STAGE = 128 * 32; // floats per operand stage

// Chunk swizzle of a [mn][k] stage row.  A fragment read is a 16-byte read
// per lane of one chunk from 16 consecutive rows (lanes li of a half-wave);
// gfx950's LDS serves 16 lanes x 16 bytes over its 64 banks at once, so the
// 16 (row parity, chunk) pairs must differ: chunk c of row r is stored at
// c ^ (r % 8) ^ ((r / 8) % 2).  (With c ^ (r % 8) alone, rows r and r + 8
// collide: rocprof counted one LDS bank conflict per read.)
__device__ __forceinline__ int dl_swz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

template <int LAY> struct DirectTile {
  const float *src[4]; // this work-item's source for instruction j, k-tile 0
  int64_t kstep;       // elements between two k-tiles
  __device__ __forceinline__ void init(const float *p, int64_t mn0, int64_t MN,
                                       int64_t s_mn, int64_t s_k, int wave,
                                       int lane) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (LAY == LAY_K) {
        const int r = (wave * 4 + j) * 8 + lane / 8;
        const int c = (lane % 8) ^ dl_swz(r);
        const int64_t row = mn0 + r < MN ? mn0 + r : MN - 1;
        src[j] = p + row * s_mn + 4 * c;
      } else {
        const int kr = (wave * 4 + j) * 2 + lane / 32;
        const int64_t mn = mn0 + 4 * (lane % 32) <= MN - 4
                               ? mn0 + 4 * (lane % 32)
                               : MN - 4;
        src[j] = p + kr * s_k + mn;
      }
    }
    kstep = LAY == LAY_K ? 32 : 32 * s_k;
  }
  __device__ __forceinline__ void issue(float *stage, int64_t kt,
                                        int wave) const {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void *)(src[j] + kt * kstep),
          (__attribute__((address_space(3))) void *)(stage +
                                                     (wave * 4 + j) * 256),
          16, 0, 0);
  }
};

// f[i][kk] = element (mn + 32 i, h * 16 + kk) of a direct-loaded stage.
template <int LAY>
__device__ __forceinline__ void dl_frags(const float *stage, int mn, int li,
                                         int h, float (&f)[2][16]) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = mn + 32 * i + li;
    if constexpr (LAY == LAY_K) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int pc = (4 * h + q) ^ dl_swz(row);
        const float4 w =
            *reinterpret_cast<const float4 *>(stage + row * 32 + pc * 4);
        f[i][4 * q + 0] = w.x;
        f[i][4 * q + 1] = w.y;
        f[i][4 * q + 2] = w.z;
        f[i][4 * q + 3] = w.w;
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < 16; ++kk)
        f[i][kk] = stage[(h * 16 + kk) * 128 + row];
    }
  }
}

template <int LA, int LB>
__device__ __forceinline__ void dl_compute(const float *sa, const float *sb,
                                           int wm, int wn, int li, int h,
                                           floatx16 (&acc)[2][2]) {
  float fa[2][16], fb[2][16];
  dl_frags<LA>(sa, wm * 64, li, h, fa);
  dl_frags<LB>(sb, wn * 64, li, h, fb);
#pragma unroll
  for (int kk = 0; kk < 16; ++kk)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][kk], fb[j][kk],
                                                         acc[i][j], 0, 0, 0);
}

// Keeps a stage's direct loads where the source issues them, ahead of the
// MFMAs that overlap their latency.  The loads write LDS, not registers, so
// the scheduler sees no consumer and sank one stage's loads to the end of
// the other stage's MFMAs, right before the wait on them (config-5 step
// 1.8% slower that way).
__device__ __forceinline__ void pin_issued_loads() {
  __builtin_amdgcn_sched_barrier(0);
}

__device__ __forceinline__ void dl_wait_and_sync() {
  // the stage's direct loads have landed in LDS, then every wave sees them
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// Same tiling and MFMA schedule as mm_f32_mfma_kernel, operands staged by
// direct loads into two named stage pairs (the k loop is unrolled by two so
// that every LDS access names its stage at compile time).
template <int LA, int LB>
__global__ __launch_bounds__(MM_THREADS, 2) void mm_f32_mfma_dl_kernel(
    MMArgs g) {
  __shared__ __align__(16) float sA0[DL_STAGE], sB0[DL_STAGE];
  __shared__ __align__(16) float sA1[DL_STAGE], sB1[DL_STAGE];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int h = lane >> 5, li = lane & 31;
  const TileCoord tc = mm_tile_coord(g);

  floatx16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc[i][j][r] = 0.f;

  DirectTile<LA> ta;
  DirectTile<LB> tb;
  ta.init(tc.A, tc.m0, g.M, g.sAm, g.sAk, wave, lane);
  tb.init(tc.B, tc.n0, g.N, g.sBn, g.sBk, wave, lane);
  const int64_t ktiles = g.K / 32;
  ta.issue(sA0, 0, wave);
  tb.issue(sB0, 0, wave);
  dl_wait_and_sync();
  for (int64_t kt = 0; kt < ktiles; kt += 2) {
    if (kt + 1 < ktiles) {
      ta.issue(sA1, kt + 1, wave);
      tb.issue(sB1, kt + 1, wave);
    }
    pin_issued_loads();
    dl_compute<LA, LB>(sA0, sB0, wm, wn, li, h, acc);
    dl_wait_and_sync();
    if (kt + 1 >= ktiles)
      break;
    if (kt + 2 < ktiles) {
      ta.issue(sA0, kt + 2, wave);
      tb.issue(sB0, kt + 2, wave);
    }
    pin_issued_loads();
    dl_compute<LA, LB>(sA1, sB1, wm, wn, li, h, acc);
    dl_wait_and_sync();
  }
  mm_epilogue(g, tc, acc, wm, wn, h, li);
}

// ---------------------------------------- wide tile (direct-to-LDS, gfx950)

// Workgroup tile 256x256, k-tile 32, 8 waves in a 2x4 grid (two per SIMD),
// each wave owns a 128x64 block = 4x2 MFMA 32x32 blocks (128 accumulator
// registers per lane).  Between two barriers a SIMD runs 256 MFMAs against
// 128 in the 128x128 kernel, each A fragment read from LDS feeds two MFMAs
// and each B fragment four, and every operand element crosses from L2 once
// per 256 (not 128) outputs.  Two direct-loaded stages per operand take
// 128 KB of LDS: one workgroup per CU.  Used for M and N multiples of 256
// and K a multiple of 64 when the 256x256 tiles give every CU one.
constexpr int WD_BM = 256, WD_BN = 256, WD_THREADS = 512;
constexpr int WD_STAGE = WD_BM * MM_BK; // floats per operand stage (32 KB)

// As DirectTile, for 256 rows of full tiles (no row is clamped): each of the
// 4 instructions of a wave fills 1 KB of a stage:
//   layout K : [256 mn][32 k], chunks swizzled (dl_swz); 8 rows each.
//              Instruction j covers rows 32 wave + 8 j + lane / 8, whose
//              swizzle is (lane / 8) ^ (j & 1): two per-lane bases, the
//              rest uniform offsets.
//   layout MN: [32 k][256 mn]; one k row each: one per-lane base.
template <int LAY> struct WideDirectTile {
  const float *base[2];
  int64_t jstep; // elements between instruction j and j + 2 (K) / j + 1 (MN)
  int64_t kstep; // elements between two k-tiles
  __device__ __forceinline__ void init(const float *p, int64_t mn0,
                                       int64_t s_mn, int64_t s_k, int wave,
                                       int lane) {
    if constexpr (LAY == LAY_K) {
      const int64_t row = mn0 + wave * 32 + lane / 8;
#pragma unroll
      for (int par = 0; par < 2; ++par)
        base[par] = p + (row + 8 * par) * s_mn +
                    4 * ((lane % 8) ^ (lane / 8) ^ par);
      jstep = 16 * s_mn;
      kstep = 32;
    } else {
      base[0] = base[1] = p + int64_t(wave * 4) * s_k + mn0 + 4 * lane;
      jstep = s_k;
      kstep = 32 * s_k;
    }
  }
  __device__ __forceinline__ void issue(float *stage, int64_t kt,
                                        int wave) const {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float *src =
          LAY == LAY_K ? base[j & 1] + (j / 2) * jstep + kt * kstep
                       : base[0] + j * jstep + kt * kstep;
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void *)src,
          (__attribute__((address_space(3))) void *)(stage +
                                                     (wave * 4 + j) * 256),
          16, 0, 0);
    }
  }
};

// f[i][kk] = element (mn + 32 i, h * 16 + 8 * half + kk) of a wide stage.
template <int LAY, int NB>
__device__ __forceinline__ void wd_frags(const float *stage, int mn, int li,
                                         int h, int half, float (&f)[NB][8]) {
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int row = mn + 32 * i + li;
    if constexpr (LAY == LAY_K) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int pc = (4 * h + 2 * half + q) ^ dl_swz(row);
        const float4 w =
            *reinterpret_cast<const float4 *>(stage + row * 32 + pc * 4);
        f[i][4 * q + 0] = w.x;
        f[i][4 * q + 1] = w.y;
        f[i][4 * q + 2] = w.z;
        f[i][4 * q + 3] = w.w;
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < 8; ++kk)
        f[i][kk] = stage[(h * 16 + 8 * half + kk) * WD_BM + row];
    }
  }
}

// The k-tile in two halves of 8 MFMA steps: 48 fragment registers live.
template <int LA, int LB>
__device__ __forceinline__ void wd_compute(const float *sa, const float *sb,
                                           int wm, int wn, int li, int h,
                                           floatx16 (&acc)[4][2]) {
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    float fa[4][8], fb[2][8];
    wd_frags<LA, 4>(sa, wm * 128, li, h, half, fa);
    wd_frags<LB, 2>(sb, wn * 64, li, h, half, fb);
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(
              fa[i][kk], fb[j][kk], acc[i][j], 0, 0, 0);
  }
}

template <int LA, int LB>
__global__ __launch_bounds__(WD_THREADS, 1) void mm_f32_mfma_wide_kernel(
    MMArgs g) {
  __shared__ __align__(16) float sA0[WD_STAGE], sB0[WD_STAGE];
  __shared__ __align__(16) float sA1[WD_STAGE], sB1[WD_STAGE];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave >> 2, wn = wave & 3;
  const int h = lane >> 5, li = lane & 31;
  const TileCoord tc = mm_tile_coord<WD_BM, WD_BN>(g);

  floatx16 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        acc[i][j][r] = 0.f;

  WideDirectTile<LA> ta;
  WideDirectTile<LB> tb;
  const int64_t k0 = int64_t(blockIdx.y) * g.kslice;
  ta.init(tc.A + k0 * g.sAk, tc.m0, g.sAm, g.sAk, wave, lane);
  tb.init(tc.B + k0 * g.sBk, tc.n0, g.sBn, g.sBk, wave, lane);
  // The slice is a multiple of 64: k-tiles come in pairs, one per stage,
  // and the loop has a single exit (an exit between the two stages made the
  // compiler copy and spill the accumulators).
  const int64_t ktiles = g.kslice / 32;
  ta.issue(sA0, 0, wave);
  tb.issue(sB0, 0, wave);
  dl_wait_and_sync();
  for (int64_t kt = 0; kt < ktiles; kt += 2) {
    ta.issue(sA1, kt + 1, wave);
    tb.issue(sB1, kt + 1, wave);
    pin_issued_loads();
    wd_compute<LA, LB>(sA0, sB0, wm, wn, li, h, acc);
    dl_wait_and_sync();
    if (kt + 2 < ktiles) {
      ta.issue(sA0, kt + 2, wave);
      tb.issue(sB0, kt + 2, wave);
    }
    pin_issued_loads();
    wd_compute<LA, LB>(sA1, sB1, wm, wn, li, h, acc);
    dl_wait_and_sync();
  }

  // lane holds column li of each 32x32 block, rows 8*(r/4) + 4*h + (r%4)
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int64_t col = tc.n0 + wn * 64 + j * 32 + li;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row =
            tc.m0 + wm * 128 + i * 32 + (r >> 2) * 8 + h * 4 + (r & 3);
        const float v = acc[i][j][r];
        if (g.part) {
          g.part[(int64_t(blockIdx.y) * g.M + row) * g.N + col] = v;
        } else {
          float *dst = tc.C + row * g.sCm + col * g.sCn;
          *dst = g.accumulate ? (*dst + v) : (g.bias ? v + g.bias[col * g.sBias] : v);
        }
      }
    }
}

// C[m][n] (+)= part[0][m][n] + part[1][m][n] + ... in slice order (a fixed
// order: the result does not depend on scheduling).  Four columns per
// work-item; N is a multiple of 4.
template <int S, bool VEC_C>
__global__ __launch_bounds__(256) void mm_splitk_sum_kernel(
    const float *__restrict__ part, int64_t M, int64_t N, float *C,
    int64_t sCm, int64_t sCn, int accumulate, const float *__restrict__ bias,
    int64_t sBias, FastDivU32 fdn4, uint32_t total) {
  // one work-item per 4 columns of one row, in a one-shot grid; the S slice
  // loads are independent (S is a template argument) and go out together
  const uint32_t q = blockIdx.x * 256u + threadIdx.x;
  if (q >= total)
    return;
  const uint32_t n4 = uint32_t(N / 4);
  const uint32_t m32 = fdn4.div(q);
  const int64_t m = m32, n = int64_t(q - m32 * n4) * 4;
  typedef float f4 __attribute__((ext_vector_type(4)));
  f4 w[S];
#pragma unroll
  for (int s = 0; s < S; ++s)
    w[s] = __builtin_nontemporal_load(
        reinterpret_cast<const f4 *>(part + (int64_t(s) * M + m) * N + n));
  float4 v = make_float4(w[0].x, w[0].y, w[0].z, w[0].w);
#pragma unroll
  for (int s = 1; s < S; ++s) {
    v.x = v.x + w[s].x;
    v.y = v.y + w[s].y;
    v.z = v.z + w[s].z;
    v.w = v.w + w[s].w;
  }
  if (bias) { // the product's value, then the bias add (its own rounding)
    v.x = v.x + bias[(n + 0) * sBias];
    v.y = v.y + bias[(n + 1) * sBias];
    v.z = v.z + bias[(n + 2) * sBias];
    v.w = v.w + bias[(n + 3) * sBias];
  }
  if constexpr (VEC_C) {
    float4 *dst = reinterpret_cast<float4 *>(C + m * sCm + n);
    if (accumulate) {
      const float4 old = *dst;
      v.x = old.x + v.x;
      v.y = old.y + v.y;
      v.z = old.z + v.z;
      v.w = old.w + v.w;
    }
    *dst = v;
  } else {
    const float o[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float *dst = C + m * sCm + (n + e) * sCn;
      *dst = accumulate ? (*dst + o[e]) : o[e];
    }
  }
}

// ------------------------------------------------ SIMT (non-fp32) kernel

template <class T> struct MMArgsT {
  const T *A;
  const T *B;
  T *C;
  int64_t M, N, K;
  int64_t sAm, sAk, sBk, sBn, sCm, sCn;
  int nb;
  int64_t bshape[MM_MAX_BATCH];
  int64_t bsA[MM_MAX_BATCH], bsB[MM_MAX_BATCH], bsC[MM_MAX_BATCH];
  int accumulate;
};

template <class T>
__global__ __launch_bounds__(256) void mm_simt_kernel(MMArgsT<T> g) {
  constexpr int TS = 16;
  __shared__ T As[TS][TS + 1];
  __shared__ T Bs[TS][TS + 1];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t row = int64_t(blockIdx.y) * TS + ty;
  const int64_t col = int64_t(blockIdx.x) * TS + tx;
  const T *A = g.A;
  const T *B = g.B;
  T *C = g.C;
  int64_t rem = blockIdx.z;
  for (int d = g.nb - 1; d >= 0; --d) {
    const int64_t q = rem / g.bshape[d];
    const int64_t c = rem - q * g.bshape[d];
    rem = q;
    A += c * g.bsA[d];
    B += c * g.bsB[d];
    C += c * g.bsC[d];
  }
  T acc = T(0);
  for (int64_t k0 = 0; k0 < g.K; k0 += TS) {
    const int64_t ka = k0 + tx, kb = k0 + ty;
    As[ty][tx] = (row < g.M && ka < g.K) ? A[row * g.sAm + ka * g.sAk] : T(0);
    Bs[ty][tx] = (kb < g.K && col < g.N) ? B[kb * g.sBk + col * g.sBn] : T(0);
    __syncthreads();
    const int kmax = (g.K - k0) < TS ? int(g.K - k0) : TS;
    for (int k = 0; k < kmax; ++k)
      acc = acc + As[ty][k] * Bs[k][tx];
    __syncthreads();
  }
  if (row < g.M && col < g.N) {
    T *dst = C + row * g.sCm + col * g.sCn;
    *dst = g.accumulate ? T(*dst + acc) : acc;
  }
}

namespace {

template <int LA, int LB> void launch_mfma(const MMArgs &a, int64_t blocks) {
  if constexpr (LA != LAY_GEN && LB != LAY_GEN) {
    if (a.K % 32 == 0) {
      // 256x256 tiles when they (or, for one product, they times a split of
      // K into 2, 4 or 8 slices of at least 1024) give every CU one
      const int64_t nbatch = blocks / (a.tiles_m * a.tiles_n);
      MMArgs w = a;
      w.tiles_m = (a.M + WD_BM - 1) / WD_BM;
      w.tiles_n = (a.N + WD_BN - 1) / WD_BN;
      const int64_t wblocks = w.tiles_m * w.tiles_n * nbatch;
      const int64_t cus = device_cu_count();
      if (a.M % WD_BM == 0 && a.N % WD_BN == 0 && a.K % 64 == 0) {
        int S = 1;
        while (wblocks * S < cus && nbatch == 1 && S < NT_MM_SPLITK_MAX &&
               a.K % (64 * 2 * S) == 0 && a.K / (2 * S) >= 1024)
          S *= 2;
        if (wblocks * S >= cus) {
          w.kslice = a.K / S;
          if (S == 1) {
            mm_f32_mfma_wide_kernel<LA, LB>
                <<<dim3(unsigned(wblocks)), WD_THREADS, 0, stream()>>>(w);
            return;
          }
          DeviceScratch part(size_t(S) * size_t(a.M) * size_t(a.N) *
                             sizeof(float));
          w.part = part.get<float>();
          mm_f32_mfma_wide_kernel<LA, LB>
              <<<dim3(unsigned(wblocks), unsigned(S)), WD_THREADS, 0,
                 stream()>>>(w);
          NT_LAUNCH_CHECK();
          const int64_t items = a.M * (a.N / 4);
          if (items >= (int64_t(1) << 32))
            fail(NT_ERR_RUNTIME, "matmul: split-K output too large");
          const unsigned grid = unsigned((items + 255) / 256);
          const bool vec_c =
              a.sCn == 1 && a.sCm % 4 == 0 &&
              reinterpret_cast<uintptr_t>(a.C) % 16 == 0;
          const FastDivU32 fdn4{uint32_t(a.N / 4)};
#define NT_SPLITK_SUM(SS)                                                      \
  do {                                                                         \
    if (vec_c)                                                                 \
      mm_splitk_sum_kernel<SS, true><<<grid, 256, 0, stream()>>>(              \
          w.part, a.M, a.N, a.C, a.sCm, a.sCn, a.accumulate, a.bias, a.sBias,  \
          fdn4, uint32_t(items));                                              \
    else                                                                       \
      mm_splitk_sum_kernel<SS, false><<<grid, 256, 0, stream()>>>(             \
          w.part, a.M, a.N, a.C, a.sCm, a.sCn, a.accumulate, a.bias, a.sBias,  \
          fdn4, uint32_t(items));                                              \
  } while (0)
          if (S == 2)
            NT_SPLITK_SUM(2);
          else if (S == 4)
            NT_SPLITK_SUM(4);
          else if (S == 8)
            NT_SPLITK_SUM(8);
          else
            fail(NT_ERR_RUNTIME, "matmul: no split-K sum for this slice count");
#undef NT_SPLITK_SUM
          return;
        }
      }
      mm_f32_mfma_dl_kernel<LA, LB>
          <<<dim3(unsigned(blocks)), MM_THREADS, 0, stream()>>>(a);
      return;
    }
  }
  mm_f32_mfma_kernel<LA, LB>
      <<<dim3(unsigned(blocks)), MM_THREADS, 0, stream()>>>(a);
}

template <int LA> void launch_mfma_b(int lb, const MMArgs &a, int64_t blocks) {
  switch (lb) {
  case LAY_K:
    return launch_mfma<LA, LAY_K>(a, blocks);
  case LAY_MN:
    return launch_mfma<LA, LAY_MN>(a, blocks);
  default:
    return launch_mfma<LA, LAY_GEN>(a, blocks);
  }
}

bool aligned16(const void *p) {
  return reinterpret_cast<uintptr_t>(p) % 16 == 0;
}

} // namespace
} // namespace nt

using namespace nt;

namespace {

// C (+)= A . B, or C = A . B + bias (bias: one value per column of C,
// fp32 only, never with accumulate).
void matmul_run(const nt_view *a, const nt_view *b, const nt_view *c,
                int32_t accumulate, const nt_view *bias) {
  {
    check_view(a, "matmul");
    check_view(b, "matmul");
    check_view(c, "matmul");
    if (a->dtype != b->dtype || a->dtype != c->dtype)
      fail(NT_ERR_RUNTIME, "matmul: dtype mismatch");
    if (a->ndim != b->ndim || a->ndim != c->ndim)
      fail(NT_ERR_VALUE, "matmul: x1 and x2 have different ndim.");
    if (a->ndim < 2)
      fail(NT_ERR_VALUE, "matmul: kernel should be called with >=2d tensors.");
    const int nd = a->ndim, nb = nd - 2;
    for (int d = 0; d < nb; ++d)
      if (a->shape[d] != b->shape[d] || a->shape[d] != c->shape[d])
        fail(NT_ERR_VALUE, "Invalid broacast shapes.");
    const int64_t M = a->shape[nd - 2], K = a->shape[nd - 1];
    const int64_t N = b->shape[nd - 1];
    if (b->shape[nd - 2] != K)
      fail(NT_ERR_VALUE, "Invalid matmul shape.");
    if (c->shape[nd - 2] != M || c->shape[nd - 1] != N)
      fail(NT_ERR_RUNTIME, "matmul: output shape mismatch");
    if (a->dtype == NT_BOOL)
      fail(NT_ERR_VALUE, "Invalid dtype.");
    int64_t nbatch = 1;
    for (int d = 0; d < nb; ++d)
      nbatch *= a->shape[d];
    if (bias) {
      check_view(bias, "matmul_bias");
      if (a->dtype != NT_FLOAT32 || bias->dtype != NT_FLOAT32)
        fail(NT_ERR_VALUE, "matmul_bias: float32 operands only");
      if (accumulate)
        fail(NT_ERR_RUNTIME, "matmul_bias: no accumulate form");
      if (bias->ndim != 1 || bias->shape[0] != N)
        fail(NT_ERR_RUNTIME, "matmul_bias: bias must be 1-D with one value per column");
    }
    if (M == 0 || N == 0 || nbatch == 0)
      return;
    if (K == 0 && bias) {
      // C = fl(0 + bias), the bias broadcast over the rows (and batches), as
      // the empty product followed by the add gives (a -0.0 bias gives +0.0)
      DeviceScratch zero_buf(sizeof(float));
      if (nt_fill(zero_buf.get(), NT_FLOAT32, 1, 0.0) != NT_OK)
        fail(NT_ERR_RUNTIME, nt_last_error());
      nt_view zv = *c, bv = *c;
      zv.data = zero_buf.get();
      zv.offset = 0;
      bv.data = bias->data;
      bv.offset = bias->offset;
      for (int d = 0; d < nd; ++d)
        zv.strides[d] = bv.strides[d] = 0;
      bv.strides[nd - 1] = bias->strides[0];
      const int rc = nt_binary(NT_ADD, &zv, &bv, c);
      if (rc != NT_OK)
        fail(rc, nt_last_error());
      return;
    }
    if (K == 0) {
      if (!accumulate) {
        dispatch_arith(c->dtype, [&]<class T>() {
          // C = 0 through the copy kernel from a broadcast zero.
          DeviceScratch zero_buf(sizeof(T));
          T *zero = zero_buf.get<T>();
          if (nt_fill(zero, c->dtype, 1, 0.0) != NT_OK)
            fail(NT_ERR_RUNTIME, nt_last_error());
          nt_view zv = *c;
          zv.data = zero;
          zv.offset = 0;
          for (int d = 0; d < zv.ndim; ++d)
            zv.strides[d] = 0;
          const int rc = nt_copy(&zv, c);
          if (rc != NT_OK)
            fail(rc, nt_last_error());
        });
      }
      return;
    }
    // Size-1 dims carry no stride information; normalise them to 0.
    auto st = [](const nt_view *v, int d) {
      return v->shape[d] == 1 ? int64_t(0) : v->strides[d];
    };
    const int64_t sAm = st(a, nd - 2), sAk = st(a, nd - 1);
    const int64_t sBk = st(b, nd - 2), sBn = st(b, nd - 1);
    const int64_t sCm = c->strides[nd - 2], sCn = c->strides[nd - 1];

    if (a->dtype == NT_FLOAT32) {
      MMArgs g{};
      g.A = typed_ptr<const float>(a);
      g.B = typed_ptr<const float>(b);
      g.C = typed_ptr<float>(c);
      g.M = M;
      g.N = N;
      g.K = K;
      g.sAm = sAm;
      g.sAk = sAk;
      g.sBk = sBk;
      g.sBn = sBn;
      g.sCm = sCm;
      g.sCn = sCn;
      g.nb = nb;
      bool batch_al = true;
      for (int d = 0; d < nb; ++d) {
        g.bshape[d] = a->shape[d];
        g.bsA[d] = st(a, d);
        g.bsB[d] = st(b, d);
        g.bsC[d] = st(c, d);
        if (g.bsA[d] % 4 != 0 || g.bsB[d] % 4 != 0)
          batch_al = false;
      }
      g.accumulate = accumulate ? 1 : 0;
      g.kslice = K;
      g.part = nullptr;
      g.bias = bias ? typed_ptr<const float>(bias) : nullptr;
      g.sBias = bias ? bias->strides[0] : 0;
      // Vector (16-byte) tile loads need the unit-stride extent and the other
      // stride to be multiples of 4 and a 16-byte aligned base.
      int la = LAY_GEN, lb = LAY_GEN;
      if (batch_al && aligned16(g.A)) {
        if (sAk == 1 && sAm % 4 == 0 && K % 4 == 0)
          la = LAY_K;
        else if (sAm == 1 && sAk % 4 == 0 && M % 4 == 0)
          la = LAY_MN;
      }
      if (batch_al && aligned16(g.B)) {
        if (sBn == 1 && sBk % 4 == 0 && N % 4 == 0)
          lb = LAY_MN;
        else if (sBk == 1 && sBn % 4 == 0 && K % 4 == 0)
          lb = LAY_K;
      }
      g.tiles_m = (M + MM_BM - 1) / MM_BM;
      g.tiles_n = (N + MM_BN - 1) / MM_BN;
      const int64_t blocks = g.tiles_m * g.tiles_n * nbatch;
      if (blocks >= (int64_t(1) << 31))
        fail(NT_ERR_RUNTIME, "matmul: problem too large");
      switch (la) {
      case LAY_K:
        launch_mfma_b<LAY_K>(lb, g, blocks);
        break;
      case LAY_MN:
        launch_mfma_b<LAY_MN>(lb, g, blocks);
        break;
      default:
        launch_mfma_b<LAY_GEN>(lb, g, blocks);
      }
      NT_LAUNCH_CHECK();
      return;
    }

    dispatch_arith(a->dtype, [&]<class T>() {
      MMArgsT<T> g{};
      g.A = typed_ptr<const T>(a);
      g.B = typed_ptr<const T>(b);
      g.C = typed_ptr<T>(c);
      g.M = M;
      g.N = N;
      g.K = K;
      g.sAm = sAm;
      g.sAk = sAk;
      g.sBk = sBk;
      g.sBn = sBn;
      g.sCm = sCm;
      g.sCn = sCn;
      g.nb = nb;
      for (int d = 0; d < nb; ++d) {
        g.bshape[d] = a->shape[d];
        g.bsA[d] = st(a, d);
        g.bsB[d] = st(b, d);
        g.bsC[d] = st(c, d);
      }
      g.accumulate = accumulate ? 1 : 0;
      if (nbatch > 65535)
        fail(NT_ERR_RUNTIME, "matmul: too many batches for the SIMT path");
      dim3 grid{unsigned((N + 15) / 16), unsigned((M + 15) / 16),
                unsigned(nbatch)};
      mm_simt_kernel<T><<<grid, 256, 0, stream()>>>(g);
      NT_LAUNCH_CHECK();
    });
  }
}

} // namespace

extern "C" {

int nt_matmul(const nt_view *a, const nt_view *b, const nt_view *c,
              int32_t accumulate) {
  return guard([&] { matmul_run(a, b, c, accumulate, nullptr); });
}

int nt_matmul_bias(const nt_view *a, const nt_view *b, const nt_view *bias,
                   const nt_view *c) {
  return guard([&] { matmul_run(a, b, c, 0, bias); });
}

} // extern "C"
