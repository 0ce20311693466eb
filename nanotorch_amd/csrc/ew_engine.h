// Elementwise engine: one launcher that runs a device functor over NI input
// and NO output views of one logical shape, picking among four kernels:
//
//  * flat    -- every operand is contiguous in the same logical order (or a
//               broadcast scalar).  Each thread moves UNROLL vectors of 16 B
//               per operand (dwordx4 loads/stores with the streaming hint).
//  * rows    -- 2-D, contiguous outputs, every input either contiguous, a
//               broadcast row, a broadcast column or a scalar: flat-kernel
//               I/O with the (row, column) of each vector from one
//               multiply-high division.
//  * tile2d  -- after merging dims, the iteration space is 2-D.  One tile
//               per workgroup (64x64; fp32 also 64x128, 128x128 and 32x256,
//               chosen by the streams in each layout); operands whose rows are
//               contiguous are read straight; operands contiguous along the
//               other axis (e.g. `x.T`) are staged through a padded LDS tile
//               so both the global read and the global write stay
//               coalesced.  Outputs laid out that way go back through the
//               same LDS tile.  The tile walks whichever orientation
//               exchanges less.  With 4-aligned sizes and strides every
//               access is a 16-byte vector (ew_tile4_kernel); otherwise
//               element accesses (ew_tile_kernel).
//  * generic -- anything else (up to 8 dims): per-element unravel with
//               multiply-high division when the index fits in 32 bits.
//
// The reference has one thread per element and a 64-bit div/mod per dim per
// element for every non-contiguous view (src/cpp/tensor_view.cuh:42-84,
// src/cpp/ops/unary_ops.cu:19-26, binary_ops.cu:22-41).
//
// Functor contract: `void operator()(const TI (&x)[NI], TO (&y)[NO]) const`,
// __device__, trivially copyable.  Each element's inputs are read before its
// outputs are written by the same work-item (flat/generic) or workgroup
// (tile2d), so an output may be the same view as an input (in-place ops and
// gradient accumulation).
#pragma once

#include <algorithm>
#include <type_traits>

#include <hip/hip_ext.h>

#include "nt_internal.h"

// Vector groups per thread, and threads per workgroup, in the contiguous
// (flat) kernel.
#ifndef NT_FLAT_UNROLL
#define NT_FLAT_UNROLL 1 // measured, whole sweep on one box: 5659 GB/s mean against 5634 (2), 5535 (4)
#endif
#ifndef NT_FLAT_THREADS
#define NT_FLAT_THREADS 512 // measured, one vector group: 256 is 1.4% slower on the sweep, 1024 equal
#endif
constexpr int FLAT_THREADS = NT_FLAT_THREADS;

namespace nt {

constexpr int EW_THREADS = 256;
#ifndef NT_ROWS_THREADS
#define NT_ROWS_THREADS 256
#endif
#ifndef NT_ROWS_RR
#define NT_ROWS_RR 2 // measured (config-3 broadcast backwards): 0.68-0.76 -> 0.77-0.84 of peak against 1; 4 and 512 work-items no better
#endif
constexpr int EW_TILE = 64;
constexpr int EW_TILE_PAD = 65;
// LDS tile buffers in the transposing kernel.  Two let consecutive exchange
// rounds skip the barrier between them; one halves the kernel's LDS (16.6 KB
// for fp32), which doubles the workgroups a CU can hold.  Measured on the
// [4096, 4096] sweep, three alternating pairs on one MI355X: one buffer
// 5599-5628 GB/s against 5568-5594 GB/s with two.
#ifndef NT_TILE_LDS_BUFS
#define NT_TILE_LDS_BUFS 1
#endif
constexpr int EW_TILE_BUFS = NT_TILE_LDS_BUFS;
static_assert(EW_TILE_BUFS == 1 || EW_TILE_BUFS == 2, "one or two tile buffers");

template <class T, int N> struct PtrPack {
  T *p[N > 0 ? N : 1];
};

template <class T, int VEC> struct alignas(sizeof(T) * VEC) VecT {
  T v[VEC];
};

template <int N> struct Strides2 {
  int64_t r[N > 0 ? N : 1];
  int64_t c[N > 0 ? N : 1];
};

// Element offsets between consecutive batch elements of each operand (the
// tile kernel over a batch of 2-D planes).
template <int NI, int NO> struct BatchStrides {
  int64_t in[NI > 0 ? NI : 1];
  int64_t out[NO];
};

template <int N> struct StridesN {
  int64_t s[N][NT_MAX_DIMS];
};

struct ShapeN {
  int ndim;
  int64_t shape[NT_MAX_DIMS];
  FastDivU32 fd[NT_MAX_DIMS];
};

// ------------------------------------------------------------ vector I/O

// Loads VEC consecutive elements; with NTL the load carries the nontemporal
// (streaming) hint.  On MI355X a cold stream read that way sustains ~9% more
// HBM bandwidth than a plain load (measured with a copy-style kernel on
// 64 MB arrays that are not resident in the 256 MB Infinity Cache).  The
// kernels that stream loads also stream their stores (vstore): over the
// 48-kernel elementwise sweep on 64 MB operands that is ~4% faster overall,
// although a kernel that re-reads a just-written output then finds it in
// HBM rather than in the Infinity Cache.
template <bool NTL, class T, int VEC>
__device__ __forceinline__ VecT<T, VEC> vload(const T *p) {
  constexpr int BYTES = VEC * int(sizeof(T));
  if constexpr (NTL && BYTES % 16 == 0) {
    // 16-byte nontemporal loads (one or two per vector)
    typedef int nat4 __attribute__((ext_vector_type(4)));
    nat4 v[BYTES / 16];
#pragma unroll
    for (int c = 0; c < BYTES / 16; ++c)
      v[c] = __builtin_nontemporal_load(reinterpret_cast<const nat4 *>(p) + c);
    VecT<T, VEC> r;
    __builtin_memcpy(&r, v, sizeof(r));
    return r;
  } else {
    return *reinterpret_cast<const VecT<T, VEC> *>(p);
  }
}

// Store forms.  ST_STREAM carries the nontemporal hint (global_store ... nt).
// ST_THROUGH is a device-scope store (buffer_store ... sc1): it writes
// through the XCD's L2 instead of leaving the line dirty there.  A kernel
// with one output stream runs faster that way on MI355X: on cold 64 MB
// arrays, back-to-back launches, y = -x 21.9 -> 20.3 us, y = a * b 31.7 ->
// 29.4 us, gx += g * y 43.0 -> 37.8 us, the 64x64 transposed tile of
// y = -x.T 24.9 -> 21.4 us; with two output streams (the binary backwards)
// it measured no faster and up to 4% slower than ST_STREAM.  The compiler
// emits the scope bit only on buffer stores (the buffer-store builtin's
// cache-policy argument), so ST_THROUGH stores go through vstore_through
// with a wave-uniform base; 64-bit atomic stores at device scope carry the
// bit too but measured 50% slower (two 8-byte stores per 16 bytes).
enum : int { ST_PLAIN = 0, ST_STREAM = 1, ST_THROUGH = 2 };

// Which one-output kernels store through, by kernel kind.  Kernels queued
// back to back share the cost of the streaming stores' dirty L2 lines: a
// kernel that leaves them makes the next one slower while they drain, so
// per-kernel times move between neighbours and the totals decide.  Measured
// on one MI355X, alternating builds on the same box, with the sweep queuing
// each layout's forwards before its backwards and independent kernels
// overlapping: every flat and tile kernel streaming its stores, against the
// flat kernels, the transposed tiles and the max/min backward over all axes
// storing through, config-2 sweep 5929-5939 -> 5989-6006 GB/s (+1.1%; the
// dominant kernel 0.683-0.686 -> 0.703-0.708), config-3 and config-5 within
// 1% except one kernel: a flat kernel whose inputs are all broadcast scalars
// (a pure write, the mean backward over all axes) fell from 0.874 to 0.779
// of peak streaming.  So the flat kernel stores through at run time exactly
// when it reads no full operand (ew_flat_kernel's `through`), the max/min
// backward over all axes (TK_SELVEC) always, everything else streams.  (In
// an earlier sweep that queued each backward right after its forward,
// storing through measured 1.2% faster: the backwards then re-read outputs
// the forwards had just written.)  NT_THROUGH_KINDS overrides the
// compile-time set.
enum : int { TK_FLAT = 1, TK_ROWS = 2, TK_TILE = 4, TK_SEL2D = 8, TK_SELVEC = 16 };
#ifndef NT_THROUGH_KINDS
#define NT_THROUGH_KINDS (TK_SELVEC)
#endif
constexpr bool through_pays(int kind) { return (kind & (NT_THROUGH_KINDS)) != 0; }

// The form a kernel of kind KIND with NOUT output streams uses when
// streaming is on.
constexpr int store_form(bool stream, int nout, int kind) {
  return !stream ? ST_PLAIN
                 : ((nout == 1 && through_pays(kind)) ? ST_THROUGH : ST_STREAM);
}

// Plain or streaming store of one vector (ST_THROUGH is vstore_through's).
template <int SF, class T, int VEC>
__device__ __forceinline__ void vstore(T *p, const VecT<T, VEC> &w) {
  constexpr int BYTES = VEC * int(sizeof(T));
  if constexpr (SF == ST_STREAM && BYTES % 16 == 0) {
    typedef int nat4 __attribute__((ext_vector_type(4)));
    nat4 v[BYTES / 16];
    __builtin_memcpy(v, &w, sizeof(v));
#pragma unroll
    for (int c = 0; c < BYTES / 16; ++c)
      __builtin_nontemporal_store(v[c], reinterpret_cast<nat4 *>(p) + c);
  } else {
    *reinterpret_cast<VecT<T, VEC> *>(p) = w;
  }
}

// Buffer resources for vstore_through: a raw buffer (stride 0) of 2^31 - 1
// bytes from the base; the fourth word's data format field (32-bit) must be
// non-zero for untyped buffer accesses on CDNA.
constexpr int BUF_WORD3 = 0x00020000;
constexpr int BUF_BYTES = 0x7fffffff;
constexpr int CPOL_SC1 = 16; // the cache-policy argument's device-scope bit

// True when every byte a workgroup stores lies less than 2^31 bytes past the
// base it passes to vstore_through (its largest element offset is last_off).
template <class T>
__device__ __forceinline__ bool through_fits(int64_t last_off, int vec) {
  return (last_off + vec) * int64_t(sizeof(T)) <= int64_t(BUF_BYTES);
}

// Device-scope store of the VEC elements at base + off.  base must be the
// same for every lane of the wave (it goes into the scalar buffer resource);
// off * sizeof(T) + the vector's bytes must stay below 2^31 (through_fits).
template <class T, int VEC>
__device__ __forceinline__ void vstore_through(T *base, int64_t off,
                                               const VecT<T, VEC> &w) {
  constexpr int BYTES = VEC * int(sizeof(T));
  // The callers' bases depend only on the workgroup (or the wave) and the
  // kernel arguments, but the compiler does not always prove it (a tile's
  // origin from its diagonal order was taken for divergent, which wrapped
  // the store in a loop over distinct bases); reading the first active
  // lane's copy states it.
  const uint64_t ub = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(ub));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(ub >> 32));
  T *const ubase = reinterpret_cast<T *>((uint64_t(hi) << 32) | lo);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(ubase, 0, BUF_BYTES, BUF_WORD3);
  const int boff = int(off * int64_t(sizeof(T)));
  if constexpr (BYTES % 16 == 0) {
    typedef int nat4 __attribute__((ext_vector_type(4)));
    nat4 v[BYTES / 16];
    __builtin_memcpy(v, &w, sizeof(v));
#pragma unroll
    for (int c = 0; c < BYTES / 16; ++c)
      __builtin_amdgcn_raw_buffer_store_b128(v[c], rs, boff + 16 * c, 0,
                                             CPOL_SC1);
  } else if constexpr (BYTES == 8) {
    typedef int nat2 __attribute__((ext_vector_type(2)));
    nat2 v;
    __builtin_memcpy(&v, &w, sizeof(v));
    __builtin_amdgcn_raw_buffer_store_b64(v, rs, boff, 0, CPOL_SC1);
  } else if constexpr (BYTES == 4) {
    int v;
    __builtin_memcpy(&v, &w, sizeof(v));
    __builtin_amdgcn_raw_buffer_store_b32(v, rs, boff, 0, CPOL_SC1);
  } else {
    *reinterpret_cast<VecT<T, VEC> *>(ubase + off) = w;
  }
}

// The store of one output vector in a kernel with NO outputs: through the
// workgroup's uniform base when that form applies and fits, else plain or
// streaming at base + off.
template <bool NTL, int NO, int KIND, class T, int VEC>
__device__ __forceinline__ void vstore_out(T *base, int64_t off, bool fits,
                                           const VecT<T, VEC> &w) {
  constexpr int SF = store_form(NTL, NO, KIND);
  if constexpr (SF == ST_THROUGH) {
    if (fits) {
      vstore_through<T, VEC>(base, off, w);
      return;
    }
    vstore<ST_STREAM, T, VEC>(base + off, w);
  } else {
    vstore<SF, T, VEC>(base + off, w);
  }
}

// Process-wide switch for the nontemporal hint (NT_NONTEMPORAL=0 turns it
// off; data that is still resident in the Infinity Cache reads faster
// without it).
bool ew_nontemporal();

// ------------------------------------------------------------------- flat

template <class TI, class TO, int NI, int NO, int VEC, int UNROLL, bool NTL,
          class F>
__global__ __launch_bounds__(FLAT_THREADS) void ew_flat_kernel(
    PtrPack<const TI, NI> in, uint32_t scalar_mask, PtrPack<TO, NO> out,
    int64_t nvec, int64_t n, bool through, F f) {
  using VI = VecT<TI, VEC>;
  using VO = VecT<TO, VEC>;
  // wg0: the workgroup's first vector (its outputs start there: a uniform
  // base for device-scope stores, offsets below FLAT_THREADS * UNROLL)
  const int64_t wg0 = int64_t(blockIdx.x) * (FLAT_THREADS * UNROLL);
  const int64_t base = wg0 + threadIdx.x;
  VI a[UNROLL][NI > 0 ? NI : 1];
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const int64_t vi = base + int64_t(u) * FLAT_THREADS;
    if (vi < nvec) {
#pragma unroll
      for (int k = 0; k < NI; ++k) {
        if (scalar_mask & (1u << k)) {
          const TI s = in.p[k][0];
#pragma unroll
          for (int j = 0; j < VEC; ++j)
            a[u][k].v[j] = s;
        } else {
          a[u][k] = vload<NTL, TI, VEC>(in.p[k] + vi * VEC);
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const int64_t vi = base + int64_t(u) * FLAT_THREADS;
    if (vi < nvec) {
      VO o[NO];
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        TI x[NI > 0 ? NI : 1];
        TO y[NO];
#pragma unroll
        for (int k = 0; k < NI; ++k)
          x[k] = a[u][k].v[j];
        f(x, y);
#pragma unroll
        for (int m = 0; m < NO; ++m)
          o[m].v[j] = y[m];
      }
#pragma unroll
      for (int m = 0; m < NO; ++m) {
        if constexpr (NTL && NO == 1) {
          if (through) { // a pure write (every input a broadcast scalar)
            vstore_through<TO, VEC>(out.p[m] + wg0 * VEC, (vi - wg0) * VEC, o[m]);
            continue;
          }
        }
        vstore_out<NTL, NO, TK_FLAT, TO, VEC>(out.p[m] + wg0 * VEC, (vi - wg0) * VEC,
                                              true, o[m]);
      }
    }
  }
  // Fewer than VEC trailing elements: block 0 takes them one per thread.
  const int64_t tail0 = nvec * VEC;
  if (blockIdx.x == 0 && int64_t(threadIdx.x) < n - tail0) {
    const int64_t i = tail0 + threadIdx.x;
    TI x[NI > 0 ? NI : 1];
    TO y[NO];
#pragma unroll
    for (int k = 0; k < NI; ++k)
      x[k] = in.p[k][(scalar_mask & (1u << k)) ? 0 : i];
    f(x, y);
#pragma unroll
    for (int m = 0; m < NO; ++m)
      out.p[m][i] = y[m];
  }
}

// ------------------------------------------------------------------- rows

// Row-major [R, C] outputs whose inputs are each a full [R, C] operand, a
// broadcast row (strides 0, 1: a bias), a broadcast column (strides s, 0:
// a reduced axis re-expanded) or a scalar.  Work-items take VEC-wide groups
// along the rows as in the flat kernel; the group's (r, c) comes from one
// multiply-high division by C (C % VEC == 0, so a group never straddles two
// rows).  Broadcast rows are re-read by every row of the grid and stay in
// cache, so they are loaded without the streaming hint.
template <class TI, class TO, int NI, int NO, int VEC, int RR, bool NTL,
          class F>
__global__ __launch_bounds__(NT_ROWS_THREADS) void ew_rows_kernel(
    PtrPack<const TI, NI> in, uint32_t scalar_mask, uint32_t rowb_mask,
    uint32_t colb_mask, Strides2<NI> sin, PtrPack<TO, NO> out, uint32_t nvec,
    FastDivU32 fdc, uint32_t C, F f) {
  // RR rows per work-item at the same columns: a broadcast row is loaded
  // once for all of them.  vi counts VEC-groups of the [R / RR, C] grid.
  using VI = VecT<TI, VEC>;
  using VO = VecT<TO, VEC>;
  const uint32_t vi = blockIdx.x * NT_ROWS_THREADS + threadIdx.x;
  // The workgroup's first and last row groups: its outputs lie in rows
  // [rbase, rlast * RR + RR), a uniform base for device-scope stores.
  const uint32_t v0 = blockIdx.x * NT_ROWS_THREADS;
  const uint32_t vl = (v0 + NT_ROWS_THREADS < nvec ? v0 + NT_ROWS_THREADS : nvec) - 1;
  const int64_t rbase = int64_t(fdc.div(v0 * VEC)) * RR;
  const bool fits = through_fits<TO>(
      (int64_t(fdc.div(vl * VEC)) * RR + RR - rbase) * C - 1, 1);
  if (vi >= nvec)
    return;
  const uint32_t i = vi * VEC;
  const uint32_t rg = fdc.div(i);
  const uint32_t c = i - rg * C;
  VI a[RR][NI > 0 ? NI : 1];
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    const uint32_t bit = 1u << k;
    if (scalar_mask & bit) {
      const TI v = in.p[k][0];
#pragma unroll
      for (int q = 0; q < RR; ++q)
#pragma unroll
        for (int j = 0; j < VEC; ++j)
          a[q][k].v[j] = v;
    } else if (rowb_mask & bit) {
      const VI v = vload<false, TI, VEC>(in.p[k] + c);
#pragma unroll
      for (int q = 0; q < RR; ++q)
        a[q][k] = v;
    } else {
#pragma unroll
      for (int q = 0; q < RR; ++q) {
        const int64_t r = int64_t(rg) * RR + q;
        if (colb_mask & bit) {
          const TI v = in.p[k][r * sin.r[k]];
#pragma unroll
          for (int j = 0; j < VEC; ++j)
            a[q][k].v[j] = v;
        } else {
          a[q][k] = vload<NTL, TI, VEC>(in.p[k] + r * C + c);
        }
      }
    }
  }
#pragma unroll
  for (int q = 0; q < RR; ++q) {
    const int64_t r = int64_t(rg) * RR + q;
    VO o[NO];
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      TI x[NI > 0 ? NI : 1];
      TO y[NO];
#pragma unroll
      for (int k = 0; k < NI; ++k)
        x[k] = a[q][k].v[j];
      f(x, y);
#pragma unroll
      for (int m = 0; m < NO; ++m)
        o[m].v[j] = y[m];
    }
#pragma unroll
    for (int m = 0; m < NO; ++m)
      vstore_out<NTL, NO, TK_ROWS, TO, VEC>(out.p[m] + rbase * C, (r - rbase) * C + c,
                                   fits, o[m]);
  }
}

// --------------------------------------------------------------- tile2d x4

// Tile (tr, tc) of workgroup b in a tiles_r x tiles_c grid (fewer than 2^24
// tiles), in diagonal order: consecutive workgroups take consecutive tile
// columns, each one tile row further on, tr = (b / tiles_c + tc) mod tiles_r.
// The tiles in flight at once then spread over every tile row and column of
// both the operands read along rows and those read along columns, instead
// of sharing 256-byte column offsets within a few tile rows.  Measured on
// the [4096, 4096] sweep, three alternations on one MI355X, against groups
// of 8 tile-rows walked column by column: transposed forwards 5.01 -> 5.16
// TB/s, transposed backwards unchanged, the whole sweep 5.66 -> 5.71 TB/s;
// row-major order was 2% slower than the groups.
__device__ __forceinline__ void diagonal_tile(uint32_t b, int64_t tiles_r,
                                              int64_t tiles_c, int64_t &tr,
                                              int64_t &tc) {
  const uint32_t nc = uint32_t(tiles_c), nr = uint32_t(tiles_r);
  const uint32_t q = b / nc, c = b - q * nc;
  tc = c;
  tr = (q + c) % nr;
}

// TR x TC tile (TR rows by TC columns of the iteration space) with 4-element
// vector accesses (16 B for fp32), TR * TC / 16 work-items.
//  * ROW operands (unit column stride) are read/written straight: TC / 4
//    work-items cover one row segment of TC elements (256 bytes of fp32 at
//    TC = 64).
//  * COL operands (unit row stride, e.g. `x.T`) are read as column segments
//    of TR elements, 4 consecutive rows per work-item, and exchanged through
//    a [col][row] LDS tile whose rows are padded to TR + 1 elements (a
//    wave's accesses spread over the banks).  Outputs of that layout take
//    the reverse path.
//  * Other operands (stride-0 broadcasts, general strides) are read per
//    element in the owner (ROW) layout.
// All global loads of all inputs are issued before the first LDS exchange.
template <class TI, class TO, int NI, int NO, bool NTL, int TR, int TC,
          class F>
__global__ __launch_bounds__(TR * TC / 16) void ew_tile4_kernel(
    PtrPack<const TI, NI> in, Strides2<NI> sin, uint32_t row_in,
    uint32_t col_in, uint32_t bcol_in, PtrPack<TO, NO> out, Strides2<NO> sout,
    uint32_t row_out, uint32_t col_out, int64_t R, int64_t C, int64_t tiles_c,
    FastDivU32 tiles_b, BatchStrides<NI, NO> bs, F f) {
  // NTH work-items, each owning EL = 4 vectors of 4 elements per operand.
  // ROW ownership: vector f = t + NTH * i is row l = f / QC, columns
  // 4 * (f % QC) + 0..3; COL ownership: column f / QR, rows
  // 4 * (f % QR) + 0..3.
  constexpr int NTH = TR * TC / 16, EL = 4, PR = TR + 1;
  constexpr int QC = TC / 4, QR = TR / 4;
  constexpr size_t LB = sizeof(TI) > sizeof(TO) ? sizeof(TI) : sizeof(TO);
  __shared__ __align__(16) unsigned char lds_raw[EW_TILE_BUFS][TC * PR * LB];
  const int t = threadIdx.x;
  // Workgroup b takes tile b % tiles_b of batch element b / tiles_b (one
  // element, tiles_b = every tile, for a 2-D launch).
  const uint32_t bb = tiles_b.div(blockIdx.x);
  const uint32_t bt = blockIdx.x - bb * tiles_b.d;
#pragma unroll
  for (int k = 0; k < NI; ++k)
    in.p[k] += int64_t(bb) * bs.in[k];
#pragma unroll
  for (int m = 0; m < NO; ++m)
    out.p[m] += int64_t(bb) * bs.out[m];
  int64_t tr, tc;
  diagonal_tile(bt, (R + TR - 1) / TR, tiles_c, tr, tc);
  const int64_t r0 = tr * TR, c0 = tc * TC;

  TI v[NI > 0 ? NI : 1][EL][4];
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    const TI *p = in.p[k];
    const int64_t sr = sin.r[k], sc = sin.c[k];
#pragma unroll
    for (int i = 0; i < EL; ++i) {
      const unsigned f_ = unsigned(t + NTH * i);
      const int q = int(f_ % QC), l = int(f_ / QC);
      if (col_in & (1u << k)) {
        const int qq = int(f_ % QR), ll = int(f_ / QR);
        const int64_t r = r0 + 4 * qq, c = c0 + ll; // raw COL layout
        if (r < R && c < C) {
          const VecT<TI, 4> w = vload<NTL, TI, 4>(p + r + c * sc);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            v[k][i][j] = w.v[j];
        }
      } else if (row_in & (1u << k)) {
        const int64_t r = r0 + l, c = c0 + 4 * q;
        if (r < R && c < C) {
          const VecT<TI, 4> w = vload<NTL, TI, 4>(p + r * sr + c);
#pragma unroll
          for (int j = 0; j < 4; ++j)
            v[k][i][j] = w.v[j];
        }
      } else if (bcol_in & (1u << k)) { // constant along a row
        const int64_t r = r0 + l;
        const TI s = (r < R) ? p[r * sr] : TI(0);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[k][i][j] = s;
      } else {
        const int64_t r = r0 + l;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t c = c0 + 4 * q + j;
          v[k][i][j] = (r < R && c < C) ? p[r * sr + c * sc] : TI(0);
        }
      }
    }
  }
  // LDS exchange of COL inputs ([column][row] tile, rows padded to TR + 1):
  // one round (and one barrier) per operand.  With two buffers the rounds
  // alternate between them: a buffer is rewritten two rounds after it was
  // read, and every work-item has passed the barrier of the round in
  // between, so its reads are complete.  With one buffer each round after
  // the first waits at a barrier of its own before it writes.  The number of
  // rounds follows the layout masks, which are kernel arguments, so every
  // such barrier is workgroup-uniform.
  int rnd = 0;
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    if (col_in & (1u << k)) {
      if (EW_TILE_BUFS == 1 && rnd > 0)
        __syncthreads();
      TI *lds = reinterpret_cast<TI *>(lds_raw[rnd % EW_TILE_BUFS]);
#pragma unroll
      for (int i = 0; i < EL; ++i) {
        const unsigned f_ = unsigned(t + NTH * i);
        const int qq = int(f_ % QR), ll = int(f_ / QR);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          lds[ll * PR + 4 * qq + j] = v[k][i][j];
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < EL; ++i) {
        const unsigned f_ = unsigned(t + NTH * i);
        const int q = int(f_ % QC), l = int(f_ / QC);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          v[k][i][j] = lds[(4 * q + j) * PR + l];
      }
      ++rnd;
    }
  }
  TO o[NO][EL][4];
#pragma unroll
  for (int i = 0; i < EL; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      TI x[NI > 0 ? NI : 1];
      TO y[NO];
#pragma unroll
      for (int k = 0; k < NI; ++k)
        x[k] = v[k][i][j];
      f(x, y);
#pragma unroll
      for (int m = 0; m < NO; ++m)
        o[m][i][j] = y[m];
    }
#pragma unroll
  for (int m = 0; m < NO; ++m) {
    TO *p = out.p[m];
    const int64_t sr = sout.r[m], sc = sout.c[m];
    // the tile's first element: a uniform base for device-scope stores
    TO *const tb = p + r0 * sr + c0 * sc;
    const bool fits = sr >= 0 && sc >= 0 &&
                      through_fits<TO>((TR - 1) * sr + (TC - 1) * sc, 1);
    if (col_out & (1u << m)) {
      if (EW_TILE_BUFS == 1 && rnd > 0)
        __syncthreads();
      TO *lds = reinterpret_cast<TO *>(lds_raw[rnd % EW_TILE_BUFS]);
      ++rnd;
#pragma unroll
      for (int i = 0; i < EL; ++i) {
        const unsigned f_ = unsigned(t + NTH * i);
        const int q = int(f_ % QC), l = int(f_ / QC);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          lds[(4 * q + j) * PR + l] = o[m][i][j];
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < EL; ++i) {
        const unsigned f_ = unsigned(t + NTH * i);
        const int qq = int(f_ % QR), ll = int(f_ / QR);
        const int64_t r = r0 + 4 * qq, c = c0 + ll;
        if (r < R && c < C) {
          VecT<TO, 4> w;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            w.v[j] = lds[ll * PR + 4 * qq + j];
          vstore_out<NTL, NO, TK_TILE, TO, 4>(tb, 4 * qq + ll * sc, fits, w);
        }
      }
    } else if (row_out & (1u << m)) {
#pragma unroll
      for (int i = 0; i < EL; ++i) {
        const unsigned f_ = unsigned(t + NTH * i);
        const int q = int(f_ % QC), l = int(f_ / QC);
        const int64_t r = r0 + l, c = c0 + 4 * q;
        if (r < R && c < C) {
          VecT<TO, 4> w;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            w.v[j] = o[m][i][j];
          vstore_out<NTL, NO, TK_TILE, TO, 4>(tb, l * sr + 4 * q, fits, w);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < EL; ++i) {
        const unsigned f_ = unsigned(t + NTH * i);
        const int q = int(f_ % QC), l = int(f_ / QC);
        const int64_t r = r0 + l;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int64_t c = c0 + 4 * q + j;
          if (r < R && c < C)
            p[r * sr + c * sc] = o[m][i][j];
        }
      }
    }
  }
}

// ----------------------------------------------------------------- tile2d

template <class TI, class TO, int NI, int NO, class F>
__global__ __launch_bounds__(EW_THREADS) void ew_tile_kernel(
    PtrPack<const TI, NI> in, Strides2<NI> sin, uint32_t col_in,
    PtrPack<TO, NO> out, Strides2<NO> sout, uint32_t col_out, int64_t R,
    int64_t C, int64_t tiles_c, F f) {
  constexpr int T = EW_TILE, P = EW_TILE_PAD;
  constexpr size_t LB = sizeof(TI) > sizeof(TO) ? sizeof(TI) : sizeof(TO);
  __shared__ __align__(16) unsigned char lds_raw[T * P * LB];
  const int tx = threadIdx.x & (T - 1);
  const int ty = threadIdx.x >> 6; // 0..3
  int64_t tr, tc;
  diagonal_tile(blockIdx.x, (R + T - 1) / T, tiles_c, tr, tc);
  const int64_t r0 = tr * T, c0 = tc * T;
  constexpr int EPT = T * T / EW_THREADS; // 16 elements per thread

  // Work-item (tx, ty) owns tile elements (row ty + 4j, col tx), j < 16.
  TI v[NI > 0 ? NI : 1][EPT];
#pragma unroll
  for (int k = 0; k < NI; ++k) {
    const TI *p = in.p[k];
    const int64_t sr = sin.r[k], sc = sin.c[k];
    if (col_in & (1u << k)) {
      // Rows are contiguous in memory along the tile's row index: lanes
      // walk rows, the tile is stored column-major in LDS, then read back
      // in the owner layout.
      TI *lds = reinterpret_cast<TI *>(lds_raw);
      __syncthreads();
#pragma unroll
      for (int j = 0; j < EPT; ++j) {
        const int cl = ty + 4 * j;
        const int64_t r = r0 + tx, c = c0 + cl;
        if (r < R && c < C)
          lds[cl * P + tx] = p[r * sr + c * sc];
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < EPT; ++j)
        v[k][j] = lds[tx * P + ty + 4 * j];
    } else {
#pragma unroll
      for (int j = 0; j < EPT; ++j) {
        const int64_t r = r0 + ty + 4 * j, c = c0 + tx;
        v[k][j] = (r < R && c < C) ? p[r * sr + c * sc] : TI(0);
      }
    }
  }
  TO o[NO][EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    TI x[NI > 0 ? NI : 1];
    TO y[NO];
#pragma unroll
    for (int k = 0; k < NI; ++k)
      x[k] = v[k][j];
    f(x, y);
#pragma unroll
    for (int m = 0; m < NO; ++m)
      o[m][j] = y[m];
  }
#pragma unroll
  for (int m = 0; m < NO; ++m) {
    TO *p = out.p[m];
    const int64_t sr = sout.r[m], sc = sout.c[m];
    if (col_out & (1u << m)) {
      TO *lds = reinterpret_cast<TO *>(lds_raw);
      __syncthreads();
#pragma unroll
      for (int j = 0; j < EPT; ++j)
        lds[tx * P + ty + 4 * j] = o[m][j];
      __syncthreads();
#pragma unroll
      for (int j = 0; j < EPT; ++j) {
        const int cl = ty + 4 * j;
        const int64_t r = r0 + tx, c = c0 + cl;
        if (r < R && c < C)
          p[r * sr + c * sc] = lds[cl * P + tx];
      }
    } else {
#pragma unroll
      for (int j = 0; j < EPT; ++j) {
        const int64_t r = r0 + ty + 4 * j, c = c0 + tx;
        if (r < R && c < C)
          p[r * sr + c * sc] = o[m][j];
      }
    }
  }
}

// ---------------------------------------------------------------- generic

template <class TI, class TO, int NI, int NO, bool IDX32, class F>
__global__ __launch_bounds__(EW_THREADS) void ew_generic_kernel(
    PtrPack<const TI, NI> in, PtrPack<TO, NO> out, StridesN<NI + NO> st,
    ShapeN sh, int64_t n, F f) {
  const int64_t stride = int64_t(gridDim.x) * EW_THREADS;
  for (int64_t i = int64_t(blockIdx.x) * EW_THREADS + threadIdx.x; i < n;
       i += stride) {
    int64_t off[NI + NO];
#pragma unroll
    for (int k = 0; k < NI + NO; ++k)
      off[k] = 0;
    if constexpr (IDX32) {
      uint32_t rem = uint32_t(i);
#pragma unroll
      for (int d = NT_MAX_DIMS - 1; d >= 0; --d) {
        if (d < sh.ndim) {
          const uint32_t q = sh.fd[d].div(rem);
          const int64_t coord = int64_t(rem - q * uint32_t(sh.shape[d]));
          rem = q;
#pragma unroll
          for (int k = 0; k < NI + NO; ++k)
            off[k] += coord * st.s[k][d];
        }
      }
    } else {
      int64_t rem = i;
#pragma unroll
      for (int d = NT_MAX_DIMS - 1; d >= 0; --d) {
        if (d < sh.ndim) {
          const int64_t q = rem / sh.shape[d];
          const int64_t coord = rem - q * sh.shape[d];
          rem = q;
#pragma unroll
          for (int k = 0; k < NI + NO; ++k)
            off[k] += coord * st.s[k][d];
        }
      }
    }
    TI x[NI > 0 ? NI : 1];
    TO y[NO];
#pragma unroll
    for (int k = 0; k < NI; ++k)
      x[k] = in.p[k][off[k]];
    f(x, y);
#pragma unroll
    for (int m = 0; m < NO; ++m)
      out.p[m][off[NI + m]] = y[m];
  }
}

// ---------------------------------------------------------------- launcher

// Queues kernel<<<grid, block, 0, s>>>(args...), without the stream barrier
// when flags holds hipExtAnyOrderLaunch (ew_launch_flags).
template <class... KA>
void ew_launch(void (*kernel)(KA...), dim3 grid, dim3 block, hipStream_t s,
               uint32_t flags, std::type_identity_t<KA>... args) {
  if (flags == 0) {
    kernel<<<grid, block, 0, s>>>(args...);
    NT_LAUNCH_CHECK();
    return;
  }
  void *ptrs[] = {static_cast<void *>(&args)...};
  NT_HIP_CHECK(hipExtLaunchKernel(reinterpret_cast<const void *>(kernel), grid,
                                  block, ptrs, 0, s, nullptr, nullptr,
                                  int(flags)));
}

// Bytes [lo, hi) a view can touch (strides are never negative).
inline ByteRange view_bytes(const nt_view *v) {
  const int64_t es = int64_t(dtype_size(v->dtype));
  int64_t last = 0;
  for (int d = 0; d < v->ndim; ++d)
    last += (v->shape[d] - 1) * v->strides[d];
  ByteRange r;
  r.lo = reinterpret_cast<uintptr_t>(v->data) + uintptr_t(v->offset * es);
  r.hi = r.lo + uintptr_t((last + 1) * es);
  return r;
}

// A functor may declare `static constexpr bool heavy = true` when its
// arithmetic per element is long enough (tanh, sigmoid) to change which
// transposed-tile layout is fastest.
template <class F> constexpr bool ew_heavy() {
  if constexpr (requires { F::heavy; })
    return F::heavy;
  else
    return false;
}

template <class T> constexpr int ew_vec() {
  return sizeof(T) >= 16 ? 1 : int(16 / sizeof(T));
}

template <class TI, class TO, int NI, int NO, class F>
void launch_elementwise(const nt_view *const *ins, const nt_view *const *outs,
                        F f) {
  constexpr int NT = NI + NO;
  const nt_view *all[NT];
  for (int k = 0; k < NI; ++k)
    all[k] = ins[k];
  for (int m = 0; m < NO; ++m)
    all[NI + m] = outs[m];
  const int64_t n = numel(outs[0]);
  if (n == 0)
    return;
  // Barrier or not (launch_window.h): every operand's bytes.
  uint32_t flags;
  {
    ByteRange rd[NI > 0 ? NI : 1], wr[NO];
    for (int k = 0; k < NI; ++k)
      rd[k] = view_bytes(ins[k]);
    for (int m = 0; m < NO; ++m)
      wr[m] = view_bytes(outs[m]);
    flags = ew_launch_flags(rd, NI, wr, NO);
  }

  PtrPack<const TI, NI> pin{};
  PtrPack<TO, NO> pout{};
  for (int k = 0; k < NI; ++k)
    pin.p[k] = typed_ptr<const TI>(ins[k]);
  for (int m = 0; m < NO; ++m)
    pout.p[m] = typed_ptr<TO>(outs[m]);

  JointLayout L = coalesce(all, NT);
  hipStream_t s = stream();

  // ---- flat: every operand unit-stride (inputs may be stride-0 scalars).
  bool flat = L.ndim <= 1;
  uint32_t smask = 0;
  if (L.ndim == 0) {
    smask = (1u << NI) - 1;
  } else if (flat) {
    for (int k = 0; k < NT && flat; ++k) {
      const int64_t st = L.strides[k][0];
      if (st == 1)
        continue;
      if (st == 0 && k < NI)
        smask |= 1u << k;
      else
        flat = false;
    }
  }
  const bool ntl = ew_nontemporal();
  if (flat) {
    // Mixed widths (casts, comparisons): the wider type moves 16 bytes per
    // access (measured on [8192, 8192]: an fp32 -> fp64 cast 7.3 TB/s, a
    // comparison 6.3 TB/s; 16 bytes of the narrower type with two accesses
    // of the wider one ran at 5.8 and 5.6).
    constexpr int VBIG = ew_vec<TI>() < ew_vec<TO>() ? ew_vec<TI>()
                                                      : ew_vec<TO>();
    constexpr int UNROLL = NT_FLAT_UNROLL;
    bool aligned = true;
    for (int k = 0; k < NI; ++k)
      if (!(smask & (1u << k)) &&
          reinterpret_cast<uintptr_t>(pin.p[k]) % (sizeof(TI) * VBIG) != 0)
        aligned = false;
    for (int m = 0; m < NO; ++m)
      if (reinterpret_cast<uintptr_t>(pout.p[m]) % (sizeof(TO) * VBIG) != 0)
        aligned = false;
    const int VEC = aligned ? VBIG : 1;
    const int64_t nvec = n / VEC;
    // One work-item per UNROLL vector groups in a one-shot grid; a dispatch
    // holds fewer than 2^32 work-items, so a longer range (e.g. an
    // unaligned view past 2^32 elements) goes out in chunks of 2^30 groups,
    // the trailing partial group with the last chunk.
    constexpr int64_t CHUNK = int64_t(1) << 30;
    int64_t v0 = 0;
    do {
      const int64_t cv = std::min(CHUNK, nvec - v0);
      const int64_t cn = (v0 + cv == nvec) ? n - v0 * VEC : cv * VEC;
      PtrPack<const TI, NI> cin = pin;
      PtrPack<TO, NO> cout = pout;
      for (int k = 0; k < NI; ++k)
        if (!(smask & (1u << k)))
          cin.p[k] += v0 * VEC;
      for (int m = 0; m < NO; ++m)
        cout.p[m] += v0 * VEC;
      const int64_t blocks = std::max<int64_t>(
          1, (cv + FLAT_THREADS * UNROLL - 1) / (FLAT_THREADS * UNROLL));
      const dim3 grid{unsigned(blocks), 1u, 1u};
      // a workgroup's outputs lie within FLAT_THREADS * UNROLL vectors of
      // its base: within the device-scope stores' 2^31-byte range
      const bool through =
          smask == (NI > 0 ? (1u << NI) - 1 : 0u) &&
          int64_t(FLAT_THREADS) * UNROLL * VBIG * int64_t(sizeof(TO)) <= BUF_BYTES;
      if (aligned && ntl)
        ew_launch(ew_flat_kernel<TI, TO, NI, NO, VBIG, UNROLL, true, F>, grid,
                  FLAT_THREADS, s, flags, cin, smask, cout, cv, cn, through, f);
      else if (aligned)
        ew_launch(ew_flat_kernel<TI, TO, NI, NO, VBIG, UNROLL, false, F>, grid,
                  FLAT_THREADS, s, flags, cin, smask, cout, cv, cn, false, f);
      else
        ew_launch(ew_flat_kernel<TI, TO, NI, NO, 1, UNROLL, false, F>, grid,
                  FLAT_THREADS, s, flags, cin, smask, cout, cv, cn, false, f);
      NT_LAUNCH_CHECK();
      v0 += cv;
    } while (v0 < nvec);
    return;
  }

  // ---- rows: contiguous [R, C] outputs, inputs full / broadcast / scalar.
  if (L.ndim == 2) {
    constexpr int VBIG = ew_vec<TI>() < ew_vec<TO>() ? ew_vec<TI>()
                                                      : ew_vec<TO>();
    const int64_t R = L.shape[0], C = L.shape[1];
    bool rows = C % VBIG == 0 && n < (int64_t(1) << 32);
    uint32_t sm = 0, rb = 0, cb = 0;
    Strides2<NI> sin{};
    for (int m = 0; m < NO && rows; ++m)
      rows = L.strides[NI + m][0] == C && L.strides[NI + m][1] == 1 &&
             reinterpret_cast<uintptr_t>(pout.p[m]) % (sizeof(TO) * VBIG) == 0;
    for (int k = 0; k < NI && rows; ++k) {
      const int64_t sr = L.strides[k][0], sc = L.strides[k][1];
      sin.r[k] = sr;
      sin.c[k] = sc;
      const bool al =
          reinterpret_cast<uintptr_t>(pin.p[k]) % (sizeof(TI) * VBIG) == 0;
      if (sr == 0 && sc == 0)
        sm |= 1u << k;
      else if (sc == 0)
        cb |= 1u << k;
      else if (sr == 0 && sc == 1 && al)
        rb |= 1u << k;
      else if (!(sr == C && sc == 1 && al))
        rows = false;
    }
    // Worth it only when something is broadcast (otherwise the operands
    // would have coalesced to the flat case).
    if (rows && (rb | cb) != 0 && R > 0) {
      constexpr int RR = NT_ROWS_RR;
      const bool grouped = RR > 1 && R % RR == 0;
      const int64_t nvec = n / VBIG / (grouped ? RR : 1);
      const int64_t blocks = std::max<int64_t>(
          1, (nvec + NT_ROWS_THREADS - 1) / NT_ROWS_THREADS);
      const dim3 grid{unsigned(blocks), 1u, 1u};
      const FastDivU32 fdc{uint32_t(C)};
      if (grouped && ntl)
        ew_launch(ew_rows_kernel<TI, TO, NI, NO, VBIG, RR, true, F>, grid,
                  NT_ROWS_THREADS, s, flags, pin, sm, rb, cb, sin, pout,
                  uint32_t(nvec), fdc, uint32_t(C), f);
      else if (grouped)
        ew_launch(ew_rows_kernel<TI, TO, NI, NO, VBIG, RR, false, F>, grid,
                  NT_ROWS_THREADS, s, flags, pin, sm, rb, cb, sin, pout,
                  uint32_t(nvec), fdc, uint32_t(C), f);
      else if (ntl)
        ew_launch(ew_rows_kernel<TI, TO, NI, NO, VBIG, 1, true, F>, grid,
                  NT_ROWS_THREADS, s, flags, pin, sm, rb, cb, sin, pout,
                  uint32_t(nvec), fdc, uint32_t(C), f);
      else
        ew_launch(ew_rows_kernel<TI, TO, NI, NO, VBIG, 1, false, F>, grid,
                  NT_ROWS_THREADS, s, flags, pin, sm, rb, cb, sin, pout,
                  uint32_t(nvec), fdc, uint32_t(C), f);
      NT_LAUNCH_CHECK();
      return;
    }
  }

  // ---- tile2d: a 2-D iteration space, or a batch of 2-D planes (3-D after
  // coalescing, e.g. `x.transpose(1, 2)` of a [B, M, N] tensor).  st holds
  // each operand's (row, column) strides in the plane, bst its stride
  // between batch elements (nb of them).
  auto tile2d = [&](int64_t R0, int64_t C0, std::array<std::array<int64_t, 2>, NT> st,
                    int64_t nb, const std::array<int64_t, NT> &bst) -> bool {
    // Elements are independent, so the tile may walk the transposed index
    // space.  Column-major operands go through the LDS exchange; pick the
    // orientation in which that costs less.  An exchanged input costs two,
    // an exchanged output one (ties keep the orientation): measured in the
    // [4096, 4096] sweep, with each transposed kernel's time taken inside
    // the sweep, the binary forwards of two `.T` inputs run 6% faster
    // exchanging their output, the unary forwards 1-3%, and the backward of
    // an op with a saved output 3-7% faster exchanging its `.T` gradient
    // (read and written) than its upstream gradient and saved output.  A
    // backward whose saved tensors and gradients are `.T` views still
    // exchanges only the upstream gradient.  Functors marked heavy
    // (ew_heavy: tanh, sigmoid) keep the older weights, an exchanged output
    // costing three inputs, under which they exchange their input and
    // compute after the exchange: in that sweep their forwards ran 3-10%
    // slower exchanging the output.
    const int IN_COST = ew_heavy<F>() ? 1 : 2, OUT_COST = ew_heavy<F>() ? 3 : 1;
    int cost_keep = 0, cost_swap = 0;
    for (int k = 0; k < NT; ++k) {
      const int64_t sr = st[k][0], sc = st[k][1];
      const int wgt = k < NI ? IN_COST : OUT_COST;
      if (sc == 1 && sr != 0) // row-major now, exchanged after a swap
        cost_swap += wgt;
      else if (sr == 1 && sc != 0) // column-major now
        cost_keep += wgt;
    }
    const TileOverride &ov = tile_override();
    if (ov.orient == 2 || (ov.orient == 0 && cost_swap < cost_keep)) {
      std::swap(R0, C0);
      for (int k = 0; k < NT; ++k)
        std::swap(st[k][0], st[k][1]);
    }
    Strides2<NI> sin{};
    Strides2<NO> sout{};
    BatchStrides<NI, NO> bs{};
    uint32_t col_in = 0, col_out = 0, row_in = 0, row_out = 0, bcol_in = 0;
    const int64_t R = R0, C = C0;
    // Vector path: 4-element groups stay inside the matrix and aligned (in
    // every batch element).
    bool vec4 = R % 4 == 0 && C % 4 == 0 && sizeof(TI) <= 8 && sizeof(TO) <= 8;
    for (int k = 0; k < NT; ++k)
      if (bst[k] % 4 != 0)
        vec4 = false;
    auto classify = [&](int64_t sr, int64_t sc, const void *p, size_t es,
                        uint32_t bit, uint32_t &row, uint32_t &col) {
      const bool al = reinterpret_cast<uintptr_t>(p) % (4 * es) == 0;
      if (sc == 1) { // row-major rows
        row |= bit;
        if (!al || sr % 4 != 0)
          vec4 = false;
      } else if (sr == 1 && sc != 0) { // column-major (a transposed view)
        col |= bit;
        if (!al || sc % 4 != 0)
          vec4 = false;
      }
    };
    for (int k = 0; k < NI; ++k) {
      sin.r[k] = st[k][0];
      sin.c[k] = st[k][1];
      bs.in[k] = bst[k];
      classify(sin.r[k], sin.c[k], pin.p[k], sizeof(TI), 1u << k, row_in, col_in);
      if (sin.c[k] == 0 && sin.r[k] != 0)
        bcol_in |= 1u << k;
    }
    for (int m = 0; m < NO; ++m) {
      sout.r[m] = st[NI + m][0];
      sout.c[m] = st[NI + m][1];
      bs.out[m] = bst[NI + m];
      classify(sout.r[m], sout.c[m], pout.p[m], sizeof(TO), 1u << m, row_out, col_out);
    }
    // 16-byte tile kernel: TR x TC tiles, TR * TC / 16 work-items.
    auto tile4 = [&]<int TR, int TC>() {
      constexpr int64_t NTH = TR * TC / 16;
      const int64_t tr_n = (R + TR - 1) / TR, tc_n = (C + TC - 1) / TC;
      const int64_t blocks = tr_n * tc_n * nb;
      if (blocks * NTH >= (int64_t(1) << 32))
        return false;
      const dim3 grid{unsigned(blocks), 1u, 1u};
      const FastDivU32 tb(uint32_t(tr_n * tc_n));
      if (ntl)
        ew_launch(ew_tile4_kernel<TI, TO, NI, NO, true, TR, TC, F>, grid,
                  unsigned(NTH), s, flags, pin, sin, row_in, col_in, bcol_in,
                  pout, sout, row_out, col_out, R, C, tc_n, tb, bs, f);
      else
        ew_launch(ew_tile4_kernel<TI, TO, NI, NO, false, TR, TC, F>, grid,
                  unsigned(NTH), s, flags, pin, sin, row_in, col_in, bcol_in,
                  pout, sout, row_out, col_out, R, C, tc_n, tb, bs, f);
      NT_LAUNCH_CHECK();
      return true;
    };
    if (vec4) {
      // Tile shape by the streams in each layout, fp32 only (other types
      // keep 64 x 64 and one instantiation).  Chosen from each transposed
      // kernel of the [4096, 4096] sweep timed inside the sweep (the kernels
      // before and after it running as usual) in both orientations at
      // 64x64, 64x128, 128x64, 32x128, 16x256, 32x256, 64x256 and 128x128:
      //  * one exchanged stream and three or more straight ones (the binary
      //    backwards and the backwards of ops with a saved input, which
      //    exchange the upstream gradient): 32 x 256, i.e. the straight
      //    streams read 1-KB runs (1-2% faster than 128 x 64, 16 x 256 and
      //    64 x 256 within 1% of it, 16 x 512 slower);
      //  * one exchanged stream and at most two straight ones (forwards
      //    exchanging their output, the neg backward): 128 x 128 with 1024
      //    work-items (2-6% faster than 64 x 128 / 64 x 64), except for
      //    heavy functors, whose two resident workgroups per CU then wait on
      //    each other's compute (tanh / sigmoid forwards 10% slower): they
      //    keep 64 x 128;
      //  * two exchanged outputs and no exchanged input (an add / sub
      //    backward writing two `.T` gradients): 128 x 128 (36 us against
      //    40 us in 64 x 128);
      //  * two exchanged streams otherwise (the backward of an op with a
      //    saved output, exchanging its `.T` gradient in and out): 64 x 128;
      //  * more: 64 x 64.
      // Whole sweep 2% faster than the previous 128 x 64 / 64 x 128 / 64 x 64
      // rule.
      if constexpr (std::is_same_v<TI, float> && std::is_same_v<TO, float>) {
        const int n_col = __builtin_popcount(col_in) + __builtin_popcount(col_out);
        const int n_row = __builtin_popcount(row_in) + __builtin_popcount(row_out);
        if (ov.tr == 64 && ov.tc == 64)
          return tile4.template operator()<64, 64>();
        if (ov.tr == 64 && ov.tc == 128)
          return tile4.template operator()<64, 128>();
        if (ov.tr == 128 && ov.tc == 128)
          return tile4.template operator()<128, 128>();
        if (ov.tr == 32 && ov.tc == 256)
          return tile4.template operator()<32, 256>();
        if (n_col == 1 && n_row >= 3)
          return tile4.template operator()<32, 256>();
        if ((n_col == 1 || (n_col == 2 && col_in == 0)) && !ew_heavy<F>())
          return tile4.template operator()<128, 128>();
        if (n_col <= 2)
          return tile4.template operator()<64, 128>();
        return tile4.template operator()<64, 64>();
      } else {
        return tile4.template operator()<64, 64>();
      }
    }
    // element tiles: one plane only
    const int64_t tiles_r = (R + EW_TILE - 1) / EW_TILE;
    const int64_t tiles_c = (C + EW_TILE - 1) / EW_TILE;
    const int64_t blocks = tiles_r * tiles_c;
    if (nb == 1 && blocks * EW_THREADS < (int64_t(1) << 32)) {
      const dim3 grid{unsigned(blocks), 1u, 1u};
      ew_launch(ew_tile_kernel<TI, TO, NI, NO, F>, grid, EW_THREADS, s, flags,
                pin, sin, col_in, pout, sout, col_out, R, C, tiles_c, f);
      NT_LAUNCH_CHECK();
      return true;
    }
    return false;
  };
  if (L.ndim == 2) {
    std::array<std::array<int64_t, 2>, NT> st{};
    std::array<int64_t, NT> bst{};
    for (int k = 0; k < NT; ++k)
      st[k] = {L.strides[k][0], L.strides[k][1]};
    if (tile2d(L.shape[0], L.shape[1], st, 1, bst))
      return;
  } else if (L.ndim == 3) {
    // The batch axis is the one on which no operand has unit stride; the
    // other two (in order) form the plane.
    for (int z = 0; z < 3; ++z) {
      bool unit = false;
      for (int k = 0; k < NT; ++k)
        unit = unit || L.strides[k][z] == 1;
      if (unit)
        continue;
      const int pa = z == 0 ? 1 : 0, pb = z == 2 ? 1 : 2;
      std::array<std::array<int64_t, 2>, NT> st{};
      std::array<int64_t, NT> bst{};
      for (int k = 0; k < NT; ++k) {
        st[k] = {L.strides[k][pa], L.strides[k][pb]};
        bst[k] = L.strides[k][z];
      }
      if (tile2d(L.shape[pa], L.shape[pb], st, L.shape[z], bst))
        return;
      break;
    }
  }

  // ---- generic
  StridesN<NT> st{};
  ShapeN sh{};
  sh.ndim = L.ndim;
  for (int d = 0; d < L.ndim; ++d) {
    sh.shape[d] = L.shape[d];
    for (int k = 0; k < NT; ++k)
      st.s[k][d] = L.strides[k][d];
  }
  const bool idx32 = n < (int64_t(1) << 32);
  if (idx32)
    for (int d = 0; d < L.ndim; ++d)
      sh.fd[d] = FastDivU32(uint32_t(L.shape[d]));
  const int64_t want = (n + EW_THREADS * 4 - 1) / (EW_THREADS * 4);
  const int64_t blocks =
      std::max<int64_t>(1, std::min<int64_t>(want, int64_t(1) << 20));
  if (idx32)
    ew_launch(ew_generic_kernel<TI, TO, NI, NO, true, F>,
              dim3(unsigned(blocks)), EW_THREADS, s, flags, pin, pout, st, sh,
              n, f);
  else
    ew_launch(ew_generic_kernel<TI, TO, NI, NO, false, F>,
              dim3(unsigned(blocks)), EW_THREADS, s, flags, pin, pout, st, sh,
              n, f);
  NT_LAUNCH_CHECK();
}

} // namespace nt
