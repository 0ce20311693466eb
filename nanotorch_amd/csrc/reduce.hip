// Axis reductions (sum / max / min / argmax / argmin) and their backward.
//
// Semantics follow src/cpp/ops/reduction_ops.cu:
//  * the reduced axes form a "drop" view whose row-major order follows the
//    caller's axis tuple; the reduced index j of an element is its position
//    in that order (:187-217);
//  * sum accumulates in the output dtype, each element cast first (:66-67);
//  * max/min keep the first j on ties; the neutral elements are
//    (numeric_limits::lowest / max, j = INT64_MAX) (:13-40), so a slice whose
//    values are all below lowest() (i.e. -inf) reports lowest() and
//    INT64_MAX, as the reference does.
// The reference reduces each slice sequentially on the CPU and with a
// multi-pass shared-memory tree over 16-byte (idx, value) partials on CUDA.
//
// Kernels here, by layout of the slice elements in memory:
//  * row    -- each slice is one contiguous run (e.g. axis=-1, or a full
//              reduction of a contiguous tensor): workgroups stream the run
//              with 16-byte loads; a wave combines with cross-lane shuffles
//              and the four waves through LDS.  Long runs are split into S
//              segments whose partials a second kernel combines in order.
//  * column -- the kept axis is the contiguous one (e.g. axis=0 of a
//              row-major matrix): each lane owns 4 adjacent columns and walks
//              rows, so every wave load is 1 KB contiguous; rows are dealt
//              round-robin to S workgroups and a second kernel combines
//              partials.
//  * generic-- anything else: one workgroup per (slice, segment), elements
//              located by multiply-high unravel of j over the drop view.
// Max/min carry (value, first j, count of elements equal to the extremum);
// the count is what the backward needs (see nt_reduce_bwd).
//
// Sums are combined in a different order than the reference's sequential
// loop, so they agree to within rounding (|diff| <= 1e-5 * sum|x| is the
// parity bound); max/min/arg results are exact.
#include <limits>

#include "ew_engine.h"

namespace nt {

constexpr int RED_THREADS = 256;
constexpr int RED_WAVES = RED_THREADS / 64;

// Row kernel: 16-byte loads in flight per work-item, workgroups per CU for
// slices split over several workgroups.
#ifndef NT_ROW_UR
#define NT_ROW_UR 4 // 8: full sums 0.79 -> 0.76, max/min same; 2: full max 0.74 -> 0.55
#endif
#ifndef NT_ROW_WG_PER_CU
#define NT_ROW_WG_PER_CU 2 // measured: full sums 6.6 -> 6.8 TB/s against 4
#endif
// Column walk (reduce_col_kernel): rows per group for sums and for max/min,
// wave columns per workgroup on wide tensors, workgroups per CU for sums and
// for max/min, and the pipelined walk (the next group's loads issued before
// this group's arithmetic); rows are dealt round-robin to the segments.
// Measured on [8192, 8192] axis 0 with all of these: sums 0.81-0.83 of peak
// at 4 rows a group (0.79 at 6 and 0.79-0.81 at 8 without the pipeline,
// 0.75 at 6 with it), max/min 0.78-0.79 at 4 (0.73 at 6, 0.53 without the
// pipeline), two or four workgroups per CU 0.66 / 0.49 for max/min and
// 0.73 / 0.58 for sums.
#ifndef NT_COL_UR
#define NT_COL_UR 4
#endif
#ifndef NT_COL_UR_SEL
#define NT_COL_UR_SEL 4
#endif
#ifndef NT_COL_WC
#define NT_COL_WC 4
#endif
#ifndef NT_COL_WG_SUM
#define NT_COL_WG_SUM 1
#endif
#ifndef NT_COL_WG_SEL
#define NT_COL_WG_SEL 1
#endif
#ifndef NT_COL_PIPE
#define NT_COL_PIPE 1
#endif
// Workgroups per CU of the 2-D max/min backward.
#ifndef NT_SEL2D_WG
#define NT_SEL2D_WG 32 // 8: 0.70-0.74 of peak against 0.80-0.81
#endif
// Work-items per slice of the second pass when there are at most 64 slices.
#ifndef NT_COMBINE_WIDE
#define NT_COMBINE_WIDE 256 // 1024: same or slower; 64 or 128 with 8 loads in flight: slower
#endif

// ------------------------------------------------------------ accumulators

template <class O> struct SumAcc {
  O s;
  __device__ __forceinline__ void init() { s = O(0); }
  __device__ __forceinline__ void add(O x, int64_t) { s = s + x; }
  // `o` covers elements after this one's.
  __device__ __forceinline__ void merge(const SumAcc &o) { s = s + o.s; }
  __device__ __forceinline__ void shfl_merge(int off) {
    SumAcc o;
    o.s = __shfl_xor(s, off, 64);
    merge(o);
  }
};

template <class O, bool IS_MAX> struct SelAcc {
  O v;
  int32_t c; // before j: a float accumulator packs into 16 bytes
  int64_t j;
  __device__ __forceinline__ void init() {
    v = IS_MAX ? std::numeric_limits<O>::lowest()
               : std::numeric_limits<O>::max();
    j = std::numeric_limits<int64_t>::max();
    c = 0;
  }
  __device__ __forceinline__ static bool better(O a, O b) {
    if constexpr (IS_MAX)
      return a > b;
    else
      return a < b;
  }
  __device__ __forceinline__ static bool better_eq(O a, O b) {
    if constexpr (IS_MAX)
      return a >= b;
    else
      return a <= b;
  }
  // Branch-free update (selects, no divergent control flow).  Every kernel
  // feeds an accumulator its elements in increasing j, so on a tie the
  // stored, earlier index stays -- unless nothing equal has been counted yet
  // (c == 0: the neutral value with index INT64_MAX met an element equal to
  // it), when the element's index is the first.  In one expression: the
  // new count is 1 exactly when the element is better, or equal with
  // nothing counted, and that is when its index is taken (x >= v and the
  // new count is 1).  NaN compares false both ways and changes nothing.
  __device__ __forceinline__ void add(O x, int64_t jj) {
    const bool b = better(x, v);
    const bool ge = better_eq(x, v);
    const int32_t cn = b ? 1 : c + (ge ? 1 : 0);
    j = (ge && cn == 1) ? jj : j;
    c = cn;
    v = b ? x : v;
  }
  __device__ __forceinline__ void merge(const SelAcc &o) {
    if (better(o.v, v)) {
      v = o.v;
      j = o.j;
      c = o.c;
    } else if (o.v == v) {
      j = o.j < j ? o.j : j;
      c += o.c;
    }
  }
  __device__ __forceinline__ void shfl_merge(int off) {
    SelAcc o;
    if constexpr (std::is_same_v<O, bool>)
      o.v = bool(__shfl_xor(int(v), off, 64));
    else
      o.v = __shfl_xor(v, off, 64);
    o.j = __shfl_xor(j, off, 64);
    o.c = __shfl_xor(c, off, 64);
    merge(o);
  }
};

// Accumulators used inside a segment walk (reduce_col_kernel, and
// reduce_row_kernel when the segment is shorter than 2^31).  Sums use SumAcc
// itself.  Max/min keep the index as a 32-bit offset from the segment's
// first element -- one 32-bit select per element instead of a 64-bit pair --
// and widen it once at the end.  The update rule is SelAcc::add's.
template <class O, bool IS_MAX> struct SelAcc32 {
  O v;
  int32_t j;
  int32_t c;
  __device__ __forceinline__ void init() {
    v = IS_MAX ? std::numeric_limits<O>::lowest()
               : std::numeric_limits<O>::max();
    j = 0;
    c = 0;
  }
  // SelAcc::add's rule: two compares, an add-with-carry and three selects
  // per element (the 64-bit form with a separate equality test took about
  // twice as many instructions).
  __device__ __forceinline__ void add(O x, int32_t jj) {
    const bool b = SelAcc<O, IS_MAX>::better(x, v);
    const bool ge = SelAcc<O, IS_MAX>::better_eq(x, v);
    const int32_t cn = b ? 1 : c + (ge ? 1 : 0);
    j = (ge && cn == 1) ? jj : j;
    c = cn;
    v = b ? x : v;
  }
  // N elements at indices jb + off[0] < jb + off[1] < ..., in one step with
  // the result of N add() calls.  m is the chunk's best, taken with a
  // strict comparison in index order from the neutral value: it is the
  // first best element's value (a zero keeps the first zero's sign), and
  // NaN and elements beyond the neutral value never count.  cc counts the
  // elements equal to m and jf is the first one's offset.  Then, as add()
  // would have: a better m replaces the state, an equal one adds its count,
  // and an equal one meeting an empty state (the neutral value met its
  // equal) is taken with its first index.
  template <int N>
  __device__ __forceinline__ void add_chunk(const O (&x)[N], int32_t jb,
                                            const int32_t (&off)[N]) {
    O m = IS_MAX ? std::numeric_limits<O>::lowest()
                 : std::numeric_limits<O>::max();
#pragma unroll
    for (int k = 0; k < N; ++k)
      m = SelAcc<O, IS_MAX>::better(x[k], m) ? x[k] : m;
    int32_t cc = 0, jf = 0;
#pragma unroll
    for (int k = N - 1; k >= 0; --k) {
      const bool e = x[k] == m;
      cc += e ? 1 : 0;
      jf = e ? off[k] : jf;
    }
    const bool b = SelAcc<O, IS_MAX>::better(m, v);
    const bool eq = m == v;
    const bool take = b || (eq && c == 0);
    v = take ? m : v;
    j = take ? jb + jf : j;
    c = take ? cc : c + (eq ? cc : 0);
  }
};

template <class Acc> struct IsSel : std::false_type {};
template <class O, bool IS_MAX>
struct IsSel<SelAcc<O, IS_MAX>> : std::true_type {};

template <class Acc> struct ColLocal {
  using type = Acc;
  __device__ static Acc widen(const Acc &a, int64_t, int64_t = 1) { return a; }
};
template <class O, bool IS_MAX> struct ColLocal<SelAcc<O, IS_MAX>> {
  using type = SelAcc32<O, IS_MAX>;
  __device__ static SelAcc<O, IS_MAX> widen(const type &a, int64_t j0,
                                            int64_t mult = 1) {
    SelAcc<O, IS_MAX> r;
    r.v = a.v;
    // c == 0: no element was taken, the index stays the neutral INT64_MAX
    r.j = a.c == 0 ? std::numeric_limits<int64_t>::max() : j0 + a.j * mult;
    r.c = a.c;
    return r;
  }
};

// Writes the final accumulator of slice k.
// MODE 0: sum value; 1: extremum value (+ optional idx/count); 2: index.
template <int MODE> struct RedOut {
  void *val;
  int64_t *idx;
  int32_t *cnt;
  template <class O, class Acc>
  __device__ __forceinline__ void write(int64_t k, const Acc &a) const {
    if constexpr (MODE == 0) {
      static_cast<O *>(val)[k] = a.s;
    } else if constexpr (MODE == 1) {
      static_cast<O *>(val)[k] = a.v;
      if (idx)
        idx[k] = a.j;
      if (cnt)
        cnt[k] = a.c;
    } else {
      static_cast<int64_t *>(val)[k] = a.j;
    }
  }
};

template <class Acc> __device__ __forceinline__ void wave_reduce(Acc &a) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1)
    a.shfl_merge(off);
}

// Reduces the 4 waves' accumulators (wave order) into wave 0's lane 0 value,
// returned to every thread of wave 0.
template <class Acc>
__device__ __forceinline__ Acc block_reduce(Acc a, Acc *lds) {
  wave_reduce(a);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0)
    lds[w] = a;
  __syncthreads();
  Acc r = lds[0];
#pragma unroll
  for (int i = 1; i < RED_WAVES; ++i)
    r.merge(lds[i]);
  return r;
}

struct KeepDesc {
  int ndim;
  int64_t shape[NT_MAX_DIMS];
  int64_t strides[NT_MAX_DIMS];
  __device__ __forceinline__ int64_t offset_of(int64_t k) const {
    int64_t off = 0;
    for (int d = ndim - 1; d >= 0; --d) {
      const int64_t q = k / shape[d];
      off += (k - q * shape[d]) * strides[d];
      k = q;
    }
    return off;
  }
};

struct DropDesc {
  int ndim;
  int64_t shape[NT_MAX_DIMS];
  int64_t strides[NT_MAX_DIMS];
  FastDivU32 fd[NT_MAX_DIMS];
};

// ---------------------------------------------------------------- kernels

// Slices are contiguous runs of length D starting at x + keep.offset_of(k).
// Block b handles slice k = b / S, segment s = b % S.
template <class T, class O, class Acc, int VEC, int MODE, bool IDX32>
__global__ __launch_bounds__(RED_THREADS) void reduce_row_kernel(
    const T *__restrict__ x, KeepDesc keep, int64_t D, int64_t seg, int S,
    Acc *partial, RedOut<MODE> out) {
  __shared__ Acc lds[RED_WAVES];
  const int64_t k = int64_t(blockIdx.x) / S;
  const int s = int(int64_t(blockIdx.x) - k * S);
  const T *row = x + keep.offset_of(k);
  constexpr int UR = NT_ROW_UR;
  const int64_t step = int64_t(RED_THREADS) * VEC;
  // Chunks of CH elements: UR vector loads per work-item.
  constexpr int64_t CH = int64_t(UR) * RED_THREADS * VEC;
  // Sums: segment s is the range [s * seg, (s + 1) * seg).  Max/min: segment
  // s takes chunks s, s + S, s + 2S, ... of the slice, and the tail after
  // the last full chunk if it would take the next chunk, so that all
  // workgroups of a slice move down it together (measured on full [8192,
  // 8192] reductions, alternating on one box: max/min 0.72-0.73 -> 0.74-0.76
  // of peak; sums 0.80 -> 0.74, so sums keep the ranges).
  constexpr bool RR = IsSel<Acc>::value;
  const int64_t j0 = RR ? 0 : int64_t(s) * seg;
  const int64_t j1 = RR ? D : (j0 + seg < D ? j0 + seg : D);
  const int64_t ncf = (j1 - j0) / CH;
  const int64_t c0 = RR ? s : 0, cs = RR ? S : 1;
  const int64_t jt0 = j0 + ncf * CH;
  const int64_t jt1 = (!RR || ncf % S == s) ? j1 : jt0;
  // IDX32 (every index of the segment below 2^31 past j0): max/min
  // accumulate a 32-bit index relative to j0 and widen it once at the end.
  using LA = std::conditional_t<IDX32, typename ColLocal<Acc>::type, Acc>;
  using IT = std::conditional_t<IDX32, int32_t, int64_t>;
  // Max/min: the main loop feeds a[0] whole chunks (32-bit index) or, with
  // 64-bit indices, one accumulator per vector lane (element i of every
  // vector goes to a[i]) so the per-element select chains are independent;
  // the tail goes per lane too.  Each accumulator sees its elements in
  // increasing j, and the merge below keeps the smallest index on ties, so
  // the result is the single-chain one.  Sums keep one chain (their
  // rounding is order-dependent).
  constexpr int NA = IsSel<Acc>::value ? VEC : 1;
  LA a[NA];
#pragma unroll
  for (int q = 0; q < NA; ++q)
    a[q].init();
  using V = VecT<T, VEC>;
  // The full chunks (NT_ROW_UR independent vector loads in flight per
  // work-item), then the tail.
  for (int64_t c = c0; c < ncf; c += cs) {
    const int64_t j = j0 + c * CH + int64_t(threadIdx.x) * VEC;
    V v[UR];
#pragma unroll
    for (int u = 0; u < UR; ++u)
      v[u] = vload<true, T, VEC>(row + j + u * step);
    const IT jb = IDX32 ? IT(j - j0) : IT(j);
    if constexpr (IsSel<Acc>::value && IDX32) {
      // max/min: the UR * VEC elements as one chunk, in index order
      // (add_chunk: 6.6 VALU instructions per element against 8.5 for
      // per-element updates; full max/min 0.68-0.71 -> 0.73-0.75 of peak,
      // along a trailing axis unchanged; one chunk of UR elements per
      // vector lane took 10)
      O xs[UR * VEC];
      int32_t off[UR * VEC];
#pragma unroll
      for (int u = 0; u < UR; ++u)
#pragma unroll
        for (int i = 0; i < VEC; ++i) {
          xs[u * VEC + i] = static_cast<O>(v[u].v[i]);
          off[u * VEC + i] = u * int32_t(step) + i;
        }
      a[0].add_chunk(xs, int32_t(jb), off);
    } else {
#pragma unroll
      for (int u = 0; u < UR; ++u)
#pragma unroll
        for (int i = 0; i < VEC; ++i)
          a[i % NA].add(static_cast<O>(v[u].v[i]), jb + IT(u * step + i));
    }
  }
  for (int64_t j = jt0 + int64_t(threadIdx.x) * VEC; j < jt1; j += step) {
    const IT jb = IDX32 ? IT(j - j0) : IT(j);
    if (VEC > 1 && j + VEC <= jt1) {
      const V v = vload<true, T, VEC>(row + j);
#pragma unroll
      for (int i = 0; i < VEC; ++i)
        a[i % NA].add(static_cast<O>(v.v[i]), jb + IT(i));
    } else {
      for (int i = 0; i < VEC && j + i < jt1; ++i)
        a[i % NA].add(static_cast<O>(row[j + i]), jb + IT(i));
    }
  }
  Acc aw;
  if constexpr (IDX32)
    aw = ColLocal<Acc>::widen(a[0], j0);
  else
    aw = a[0];
#pragma unroll
  for (int q = 1; q < NA; ++q) {
    if constexpr (IDX32)
      aw.merge(ColLocal<Acc>::widen(a[q], j0));
    else
      aw.merge(a[q]);
  }
  Acc r = block_reduce(aw, lds);
  if (threadIdx.x == 0) {
    if (S == 1)
      out.template write<O>(k, r);
    else
      partial[k * S + s] = r;
  }
}

// x is [D, K] with K contiguous (stride 1) and row stride sd.  Block
// (bx, s) covers columns [bx * CB, +CB), CB = 64 * VEC * WC, and rows
// s, s + S, s + 2S, ...: WC waves stand side by side (lane l owns VEC
// adjacent columns, so a block reads CB * sizeof(T) contiguous bytes of each
// row) and the RED_WAVES / WC wave rows interleave the segment's rows, UR
// rows in flight per lane.  Partials go to partial[s * K + k] (coalesced),
// combined by reduce_col_combine_kernel.
template <class T, class O, class Acc, int VEC, int WC, int UR, int MODE>
__global__ __launch_bounds__(RED_THREADS) void reduce_col_kernel(
    const T *__restrict__ x, int64_t K, int64_t D, int64_t sd, int S,
    Acc *partial, RedOut<MODE> out) {
  constexpr int WR = RED_WAVES / WC;
  constexpr int CB = 64 * VEC * WC;
  __shared__ Acc lds[WR > 1 ? RED_WAVES : 1][64 * VEC];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wc = w % WC, wr = w / WC;
  const int s = blockIdx.y;
  const int64_t k0 =
      int64_t(blockIdx.x) * CB + int64_t(wc) * 64 * VEC + int64_t(lane) * VEC;
  // Segment s takes rows s, s + S, s + 2S, ... (relative row r is row
  // s + r S; D < 2^31, checked by the host), so all workgroups walk one
  // window of rows down the tensor together.  Contiguous row ranges per
  // segment spread the concurrent reads over S distant parts of the
  // tensor: axis-0 max / min / sum of [8192, 8192] ran at 0.69-0.72 of
  // peak that way, 0.78-0.79 round-robin.
  const int64_t j0 = s, jm = S;
  const int32_t nr = s < D ? int32_t((D - s + S - 1) / S) : 0;
  const T *base = x + j0 * sd + k0;
  sd *= S;
  using LA = typename ColLocal<Acc>::type;
  LA la[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i)
    la[i].init();
  using V = VecT<T, VEC>;
  if (k0 + VEC <= K) {
    int32_t jr = wr;
#if NT_COL_PIPE
    // Groups of UR rows (g-th group: rows wr + g*UR*WR + u*WR).  A wave
    // would otherwise leave the memory pipe idle while it works through a
    // group (max/min selects above all): the next group's loads go out
    // before this group's arithmetic, alternating two register sets (a copy
    // between them would wait for the loads in flight).  The last prefetch
    // re-reads the last group (clamped index, in bounds) and is discarded.
    constexpr int32_t GR = UR * WR;
    // wave-uniform loop control and addresses (scalar registers)
    const int32_t wru = __builtin_amdgcn_readfirstlane(wr);
    const int32_t nru = __builtin_amdgcn_readfirstlane(nr);
    const int32_t ng = nru - 1 - wru - (UR - 1) * WR >= 0
                           ? (nru - 1 - wru - (UR - 1) * WR) / GR + 1
                           : 0;
    if (ng > 0) {
      V va[UR], vb[UR];
      const int64_t rs = int64_t(WR) * sd, gs = int64_t(GR) * sd;
      const T *pa = base + int64_t(wru) * sd; // group 0
      auto load = [&](V *v, const T *p) {
#pragma unroll
        for (int u = 0; u < UR; ++u)
          v[u] = vload<true, T, VEC>(p + u * rs);
      };
      auto fold = [&](const V *v, int32_t g) {
        const int32_t jg = wru + g * GR;
#pragma unroll
        for (int u = 0; u < UR; ++u)
#pragma unroll
          for (int i = 0; i < VEC; ++i)
            la[i].add(static_cast<O>(v[u].v[i]), jg + u * WR);
      };
      auto at = [&](int32_t g) { return pa + int64_t(g < ng ? g : ng - 1) * gs; };
      load(va, pa);
      int32_t g = 0;
      for (; g + 1 < ng; g += 2) {
        load(vb, at(g + 1));
        // keep the scheduler from sinking these loads below the selects
        __builtin_amdgcn_sched_barrier(0);
        fold(va, g);
        load(va, at(g + 2)); // the last group again when g + 2 == ng
        __builtin_amdgcn_sched_barrier(0);
        fold(vb, g + 1);
      }
      if (g < ng)
        fold(va, g);
      jr = wru + ng * GR;
    }
#endif
    for (; jr + (UR - 1) * WR < nr; jr += UR * WR) {
      V v[UR];
#pragma unroll
      for (int u = 0; u < UR; ++u)
        v[u] = vload<true, T, VEC>(base + int64_t(jr + u * WR) * sd);
#pragma unroll
      for (int u = 0; u < UR; ++u)
#pragma unroll
        for (int i = 0; i < VEC; ++i)
          la[i].add(static_cast<O>(v[u].v[i]), jr + u * WR);
    }
    for (; jr < nr; jr += WR) {
      const V v = vload<true, T, VEC>(base + int64_t(jr) * sd);
#pragma unroll
      for (int i = 0; i < VEC; ++i)
        la[i].add(static_cast<O>(v.v[i]), jr);
    }
  } else if (k0 < K) {
    for (int32_t jr = wr; jr < nr; jr += WR)
      for (int i = 0; i < VEC; ++i)
        if (k0 + i < K)
          la[i].add(static_cast<O>(base[int64_t(jr) * sd + i]), jr);
  }
  Acc a[VEC];
#pragma unroll
  for (int i = 0; i < VEC; ++i)
    a[i] = ColLocal<Acc>::widen(la[i], j0, jm);
  if constexpr (WR > 1) {
    // Wave rows of one column group merge in wave-row order.
#pragma unroll
    for (int i = 0; i < VEC; ++i)
      lds[w][lane * VEC + i] = a[i];
    __syncthreads();
    if (wr == 0) {
#pragma unroll
      for (int i = 0; i < VEC; ++i)
#pragma unroll
        for (int rr = 1; rr < WR; ++rr)
          a[i].merge(lds[rr * WC + wc][lane * VEC + i]);
    }
  }
  if (wr == 0) {
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      const int64_t k = k0 + i;
      if (k < K) {
        if (S == 1)
          out.template write<O>(k, a[i]);
        else
          partial[int64_t(s) * K + k] = a[i];
      }
    }
  }
}

// Combines partial[s * K + k] over s for 64 columns per block: wave w
// merges s = w, w + 4, ... (UR loads in flight), then the four waves merge
// in order through LDS.
template <class O, class Acc, int MODE>
__global__ __launch_bounds__(RED_THREADS) void reduce_col_combine_kernel(
    const Acc *__restrict__ partial, int64_t K, int S, RedOut<MODE> out) {
  constexpr int UR = 4;
  __shared__ Acc lds[RED_WAVES][64];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t k = int64_t(blockIdx.x) * 64 + lane;
  Acc a;
  a.init();
  if (k < K) {
    int s = w;
    for (; s + RED_WAVES * (UR - 1) < S; s += RED_WAVES * UR) {
      Acc t[UR];
#pragma unroll
      for (int u = 0; u < UR; ++u)
        t[u] = partial[int64_t(s + RED_WAVES * u) * K + k];
#pragma unroll
      for (int u = 0; u < UR; ++u)
        a.merge(t[u]);
    }
    for (; s < S; s += RED_WAVES)
      a.merge(partial[int64_t(s) * K + k]);
  }
  lds[w][lane] = a;
  __syncthreads();
  if (w == 0 && k < K) {
    Acc r = lds[0][lane];
#pragma unroll
    for (int i = 1; i < RED_WAVES; ++i)
      r.merge(lds[i][lane]);
    out.template write<O>(k, r);
  }
}

template <class T, class O, class Acc, int MODE>
__global__ __launch_bounds__(RED_THREADS) void reduce_generic_kernel(
    const T *__restrict__ x, KeepDesc keep, DropDesc drop, int64_t D,
    int64_t seg, int S, bool idx32, Acc *partial, RedOut<MODE> out) {
  __shared__ Acc lds[RED_WAVES];
  const int64_t k = int64_t(blockIdx.x) / S;
  const int s = int(int64_t(blockIdx.x) - k * S);
  const T *base = x + keep.offset_of(k);
  const int64_t j0 = int64_t(s) * seg;
  const int64_t j1 = j0 + seg < D ? j0 + seg : D;
  Acc a;
  a.init();
  for (int64_t j = j0 + threadIdx.x; j < j1; j += RED_THREADS) {
    int64_t off = 0;
    if (idx32) {
      uint32_t rem = uint32_t(j);
      for (int d = drop.ndim - 1; d >= 0; --d) {
        const uint32_t q = drop.fd[d].div(rem);
        off += int64_t(rem - q * uint32_t(drop.shape[d])) * drop.strides[d];
        rem = q;
      }
    } else {
      int64_t rem = j;
      for (int d = drop.ndim - 1; d >= 0; --d) {
        const int64_t q = rem / drop.shape[d];
        off += (rem - q * drop.shape[d]) * drop.strides[d];
        rem = q;
      }
    }
    a.add(static_cast<O>(base[off]), j);
  }
  Acc r = block_reduce(a, lds);
  if (threadIdx.x == 0) {
    if (S == 1)
      out.template write<O>(k, r);
    else
      partial[k * S + s] = r;
  }
}

// Combines the S partials of slice k (one wave per slice), in segment order
// per lane, then across lanes.
// Combines partial[k * S + s] over s, one workgroup of NT work-items per
// slice k: item t merges s = t, t + NT, ..., then the waves merge in order.
template <class O, class Acc, int MODE, int NT>
__global__ __launch_bounds__(NT) void reduce_combine_kernel(
    const Acc *__restrict__ partial, int S, RedOut<MODE> out) {
  __shared__ Acc lds[NT / 64];
  const int64_t k = blockIdx.x;
  Acc a;
  a.init();
  for (int s = threadIdx.x; s < S; s += NT)
    a.merge(partial[k * S + s]);
  wave_reduce(a);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0)
    lds[w] = a;
  __syncthreads();
  if (threadIdx.x == 0) {
    Acc r = lds[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i)
      r.merge(lds[i]);
    out.template write<O>(k, r);
  }
}

// ------------------------------------------------------------------- plan

struct RedPlan {
  int64_t K = 1, D = 1;
  nt_view keep{}, drop{}; // coalesced, strides in elements; keep has offset
};

// Merges adjacent dims (in the order given) of a single view.
void coalesce_single(nt_view &v) {
  int out = 0;
  for (int d = 0; d < v.ndim; ++d) {
    if (v.shape[d] == 1)
      continue;
    if (out > 0 && v.strides[out - 1] == v.strides[d] * v.shape[d]) {
      v.shape[out - 1] *= v.shape[d];
      v.strides[out - 1] = v.strides[d];
      continue;
    }
    v.shape[out] = v.shape[d];
    v.strides[out] = v.strides[d];
    ++out;
  }
  v.ndim = out;
}

RedPlan make_plan(const nt_view *x, const int64_t *axes, int naxes) {
  RedPlan p;
  bool is_drop[NT_MAX_DIMS] = {};
  for (int i = 0; i < naxes; ++i) {
    const int64_t ax = axes[i];
    if (ax < 0 || ax >= x->ndim)
      fail(NT_ERR_INDEX, "reduction: axis out of range");
    if (is_drop[ax])
      fail(NT_ERR_VALUE, "reduction: redundant axes");
    is_drop[ax] = true;
  }
  p.keep.ndim = 0;
  for (int d = 0; d < x->ndim; ++d)
    if (!is_drop[d]) {
      p.keep.shape[p.keep.ndim] = x->shape[d];
      p.keep.strides[p.keep.ndim] = x->strides[d];
      p.keep.ndim++;
      p.K *= x->shape[d];
    }
  p.drop.ndim = naxes;
  for (int i = 0; i < naxes; ++i) {
    p.drop.shape[i] = x->shape[axes[i]];
    p.drop.strides[i] = x->strides[axes[i]];
    p.D *= x->shape[axes[i]];
  }
  coalesce_single(p.keep);
  coalesce_single(p.drop);
  return p;
}

KeepDesc to_keep_desc(const nt_view &v) {
  KeepDesc k{};
  k.ndim = v.ndim;
  for (int d = 0; d < v.ndim; ++d) {
    k.shape[d] = v.shape[d];
    k.strides[d] = v.strides[d];
  }
  return k;
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Partial results of one reduction: from the caching allocator (nt_reduce),
// or from the static scratch array whose device address `fixed` is
// (nt_reduce_noalloc), checked against its size.  Every partial slot is
// written by the first pass before the combine pass reads it, so the
// array's earlier contents never matter.
class PartialBuf {
public:
  PartialBuf(size_t nbytes, void *fixed)
      : alloc_(fixed != nullptr ? 0 : nbytes) {
    if (fixed != nullptr && nbytes > NT_NOALLOC_SCRATCH_BYTES)
      fail(NT_ERR_VALUE, "reduction needs " + std::to_string(nbytes) +
                             " bytes of partial results, more than the " +
                             std::to_string(NT_NOALLOC_SCRATCH_BYTES) +
                             "-byte allocation-free scratch");
    p_ = fixed != nullptr ? (nbytes ? fixed : nullptr) : alloc_.get();
  }
  template <class T> T *get() const { return static_cast<T *>(p_); }

private:
  DeviceScratch alloc_;
  void *p_;
};

template <class T, class O, class Acc, int MODE>
void run_reduce(const nt_view *x, const RedPlan &p, RedOut<MODE> out,
                void *fixed) {
  if (p.K == 0)
    return;
  const T *xp = typed_ptr<const T>(x);
  hipStream_t st = stream();
  const int64_t target_blocks = int64_t(device_cu_count()) * 8;
  constexpr int VEC = std::is_same_v<T, O> ? ew_vec<T>() : 1;
  constexpr bool FAST = std::is_same_v<T, O> &&
                        (std::is_same_v<T, float> || std::is_same_v<T, double>);

  // Second pass over partial[k * S + s]: few slices get 1024 work-items
  // each (a full reduction's S partials in two loads per item).
  auto finish = [&](Acc *partial, int S) {
    if (S > 1) {
      if (p.K <= 64)
        reduce_combine_kernel<O, Acc, MODE, NT_COMBINE_WIDE>
            <<<dim3(unsigned(p.K)), NT_COMBINE_WIDE, 0, st>>>(partial, S, out);
      else
        reduce_combine_kernel<O, Acc, MODE, RED_THREADS>
            <<<dim3(unsigned(p.K)), RED_THREADS, 0, st>>>(partial, S, out);
      NT_LAUNCH_CHECK();
    }
  };

  const bool drop_contig =
      p.drop.ndim == 0 || (p.drop.ndim == 1 && p.drop.strides[0] == 1);
  const bool col_layout = p.drop.ndim == 1 && p.keep.ndim == 1 &&
                          p.keep.strides[0] == 1 && p.drop.strides[0] != 1 &&
                          p.D < (int64_t(1) << 31);

  if (FAST && drop_contig) {
    // Vector loads need every slice start and segment start VEC-aligned.
    bool aligned = reinterpret_cast<uintptr_t>(xp) % (sizeof(T) * VEC) == 0;
    for (int d = 0; d < p.keep.ndim; ++d)
      if (p.keep.strides[d] % VEC != 0)
        aligned = false;
    // Long slices are split so that about NT_ROW_WG_PER_CU workgroups per
    // CU stream.
    const int64_t row_target = int64_t(device_cu_count()) * NT_ROW_WG_PER_CU;
    int64_t S = 1;
    if (p.K < row_target)
      S = std::min<int64_t>(ceil_div(row_target, p.K),
                            std::max<int64_t>(1, p.D / (RED_THREADS * 16)));
    S = std::max<int64_t>(1, std::min<int64_t>(S, 1 << 16));
    int64_t seg = ceil_div(p.D, S);
    seg = ceil_div(seg, VEC) * VEC;
    S = ceil_div(p.D, seg);
    PartialBuf partial_buf(S > 1 ? sizeof(Acc) * p.K * S : 0, fixed);
    Acc *partial = partial_buf.get<Acc>();
    const KeepDesc kd = to_keep_desc(p.keep);
    const int64_t blocks = p.K * S;
    if (blocks >= (int64_t(1) << 31))
      fail(NT_ERR_RUNTIME, "reduction too large");
    // a max/min segment spans the slice (round-robin chunks)
    const bool idx32 = (IsSel<Acc>::value ? p.D : seg) < (int64_t(1) << 31);
    const dim3 grid{unsigned(blocks), 1u, 1u};
    if (aligned && idx32)
      reduce_row_kernel<T, O, Acc, VEC, MODE, true>
          <<<grid, RED_THREADS, 0, st>>>(xp, kd, p.D, seg, int(S), partial, out);
    else if (aligned)
      reduce_row_kernel<T, O, Acc, VEC, MODE, false>
          <<<grid, RED_THREADS, 0, st>>>(xp, kd, p.D, seg, int(S), partial, out);
    else if (idx32)
      reduce_row_kernel<T, O, Acc, 1, MODE, true>
          <<<grid, RED_THREADS, 0, st>>>(xp, kd, p.D, seg, int(S), partial, out);
    else
      reduce_row_kernel<T, O, Acc, 1, MODE, false>
          <<<grid, RED_THREADS, 0, st>>>(xp, kd, p.D, seg, int(S), partial, out);
    NT_LAUNCH_CHECK();
    finish(partial, int(S));
    return;
  }

  if (FAST && col_layout) {
    const int64_t K = p.keep.shape[0], D = p.drop.shape[0];
    const int64_t sd = p.drop.strides[0];
    const bool aligned =
        reinterpret_cast<uintptr_t>(xp) % (sizeof(T) * VEC) == 0 &&
        sd % VEC == 0;
    const int vec = aligned ? VEC : 1;
    // Wide tensors: WC waves side by side (64 * vec * WC columns per
    // workgroup); narrow ones: 1 column group, 4 wave rows.
    constexpr int UR = IsSel<Acc>::value ? NT_COL_UR_SEL : NT_COL_UR;
    constexpr int WC = NT_COL_WC;
    const int wc = K >= WC * 64 * vec ? WC : 1;
    const int64_t bx = ceil_div(K, int64_t(64) * vec * wc);
    // About one (sum) or two (max/min, larger partials) workgroups per CU:
    // fewer, longer row walks with UR loads in flight measured faster than
    // many short ones, and keep the partials small.
    const int64_t col_target =
        int64_t(device_cu_count()) *
        (sizeof(Acc) <= 8 ? NT_COL_WG_SUM : NT_COL_WG_SEL);
    int64_t S = std::max<int64_t>(1, ceil_div(col_target, bx));
    S = std::min<int64_t>(S, std::max<int64_t>(1, D / (UR * (RED_WAVES / wc))));
    S = std::min<int64_t>(S, 65535);
    const int64_t seg = ceil_div(D, S);
    S = ceil_div(D, seg);
    PartialBuf partial_buf(S > 1 ? sizeof(Acc) * K * S : 0, fixed);
    Acc *partial = partial_buf.get<Acc>();
    if (bx >= (int64_t(1) << 31))
      fail(NT_ERR_RUNTIME, "reduction too large");
    const dim3 grid{unsigned(bx), unsigned(S), 1u};
    if (aligned && wc == WC)
      reduce_col_kernel<T, O, Acc, VEC, WC, UR, MODE>
          <<<grid, RED_THREADS, 0, st>>>(xp, K, D, sd, int(S), partial, out);
    else if (aligned)
      reduce_col_kernel<T, O, Acc, VEC, 1, UR, MODE>
          <<<grid, RED_THREADS, 0, st>>>(xp, K, D, sd, int(S), partial, out);
    else if (wc == WC)
      reduce_col_kernel<T, O, Acc, 1, WC, UR, MODE>
          <<<grid, RED_THREADS, 0, st>>>(xp, K, D, sd, int(S), partial, out);
    else
      reduce_col_kernel<T, O, Acc, 1, 1, UR, MODE>
          <<<grid, RED_THREADS, 0, st>>>(xp, K, D, sd, int(S), partial, out);
    NT_LAUNCH_CHECK();
    if (S > 1) {
      reduce_col_combine_kernel<O, Acc, MODE>
          <<<dim3(unsigned(ceil_div(K, 64))), RED_THREADS, 0, st>>>(
              partial, K, int(S), out);
      NT_LAUNCH_CHECK();
    }
    return;
  }

  // generic
  DropDesc dd{};
  dd.ndim = p.drop.ndim;
  const bool idx32 = p.D < (int64_t(1) << 32);
  for (int d = 0; d < p.drop.ndim; ++d) {
    dd.shape[d] = p.drop.shape[d];
    dd.strides[d] = p.drop.strides[d];
    if (idx32)
      dd.fd[d] = FastDivU32(uint32_t(p.drop.shape[d]));
  }
  int64_t S = 1;
  if (p.K < target_blocks)
    S = std::min<int64_t>(ceil_div(target_blocks, p.K),
                          std::max<int64_t>(1, p.D / (RED_THREADS * 8)));
  S = std::max<int64_t>(1, std::min<int64_t>(S, 1 << 16));
  const int64_t seg = ceil_div(p.D, S);
  S = ceil_div(p.D, seg);
  PartialBuf partial_buf(S > 1 ? sizeof(Acc) * p.K * S : 0, fixed);
  Acc *partial = partial_buf.get<Acc>();
  const int64_t blocks = p.K * S;
  if (blocks >= (int64_t(1) << 31))
    fail(NT_ERR_RUNTIME, "reduction too large");
  reduce_generic_kernel<T, O, Acc, MODE>
      <<<dim3(unsigned(blocks)), RED_THREADS, 0, st>>>(
          xp, to_keep_desc(p.keep), dd, p.D, seg, int(S), idx32, partial, out);
  NT_LAUNCH_CHECK();
  finish(partial, int(S));
}

// -------------------------------------------------------------- backward

// Max/min backward: gx[i] = g[k] * ((j == idx[k] && cnt[k] == 1) ? 1 : 0),
// where (k, j) are the kept / reduced coordinates of logical element i.
struct SelBwdDesc {
  int ndim;
  int64_t shape[NT_MAX_DIMS];
  FastDivU32 fd[NT_MAX_DIMS];
  int64_t gx_strides[NT_MAX_DIMS];
  int64_t kmul[NT_MAX_DIMS]; // contribution of each coord to k
  int64_t jmul[NT_MAX_DIMS]; // contribution of each coord to j
};

template <class T, bool ACC, bool IDX32>
__global__ __launch_bounds__(256) void sel_bwd_kernel(
    const T *__restrict__ g, const int64_t *__restrict__ idx,
    const int32_t *__restrict__ cnt, T *gx, SelBwdDesc dsc, int64_t n) {
  const int64_t stride = int64_t(gridDim.x) * 256;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < n;
       i += stride) {
    int64_t off = 0, k = 0, j = 0;
    if constexpr (IDX32) {
      uint32_t rem = uint32_t(i);
#pragma unroll
      for (int d = NT_MAX_DIMS - 1; d >= 0; --d)
        if (d < dsc.ndim) {
          const uint32_t q = dsc.fd[d].div(rem);
          const int64_t c = int64_t(rem - q * uint32_t(dsc.shape[d]));
          rem = q;
          off += c * dsc.gx_strides[d];
          k += c * dsc.kmul[d];
          j += c * dsc.jmul[d];
        }
    } else {
      int64_t rem = i;
#pragma unroll
      for (int d = NT_MAX_DIMS - 1; d >= 0; --d)
        if (d < dsc.ndim) {
          const int64_t q = rem / dsc.shape[d];
          const int64_t c = rem - q * dsc.shape[d];
          rem = q;
          off += c * dsc.gx_strides[d];
          k += c * dsc.kmul[d];
          j += c * dsc.jmul[d];
        }
    }
    const bool sel = (j == idx[k]) && (cnt[k] == 1);
    const T t = g[k] * (sel ? T(1) : T(0));
    if constexpr (ACC)
      gx[off] = gx[off] + t;
    else
      gx[off] = t;
  }
}

// Max/min backward when gx is contiguous and the reduced axes are the
// trailing (MODE 0: k = i / C, j = i % C), leading (MODE 1: k = i % C,
// j = i / C) or all (MODE 2: k = 0, j = i) dims in increasing order.  Each
// work-item writes 4 consecutive elements with one 16-byte store.
template <class T, bool ACC, int MODE>
__global__ __launch_bounds__(256) void sel_bwd_vec_kernel(
    const T *__restrict__ g, const int64_t *__restrict__ idx,
    const int32_t *__restrict__ cnt, T *gx, FastDivU32 fdC, uint32_t C,
    int64_t n4) {
  const int64_t stride = int64_t(gridDim.x) * 256;
  // q0: the block's first vector this round (uniform: the store base)
  for (int64_t q0 = int64_t(blockIdx.x) * 256; q0 < n4; q0 += stride) {
    const int64_t q = q0 + threadIdx.x;
    if (q >= n4)
      break;
    VecT<T, 4> o;
    VecT<T, 4> old;
    if constexpr (ACC)
      old = vload<true, T, 4>(gx + 4 * q);
    const uint32_t i0 = uint32_t(4 * q);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t i = i0 + e;
      int64_t k, j;
      if constexpr (MODE == 0) {
        const uint32_t qq = fdC.div(i);
        k = qq;
        j = i - qq * C;
      } else if constexpr (MODE == 1) {
        const uint32_t qq = fdC.div(i);
        k = i - qq * C;
        j = qq;
      } else {
        k = 0;
        j = i;
      }
      const bool sel = (j == idx[k]) && (cnt[k] == 1);
      const T t = g[k] * (sel ? T(1) : T(0));
      if constexpr (ACC)
        o.v[e] = old.v[e] + t;
      else
        o.v[e] = t;
    }
    vstore_out<true, 1, TK_SELVEC, T, 4>(gx + 4 * q0, 4 * int64_t(threadIdx.x),
                                         true, o);
  }
}

// Max/min backward on a contiguous [Rr, Cc] gx, Cc % 4 == 0.  MODE 0: slice
// k = row, reduced index j = column (trailing axes reduced); MODE 1: k =
// column, j = row (leading axes reduced).  Lane l of block (bx, by) owns
// columns 4 * (64 bx + l) .. +3 and the waves walk rows by * rpb + w, +4, ...
// The slice's (g, idx, count) is loaded once per row (MODE 0) or once per
// work-item (MODE 1), so the kernel is a plain 16-byte streaming write.
template <class T, bool ACC, int MODE>
__global__ __launch_bounds__(256) void sel_bwd_2d_kernel(
    const T *__restrict__ g, const int64_t *__restrict__ idx,
    const int32_t *__restrict__ cnt, T *gx, int64_t Rr, int64_t Cc,
    int64_t rpb) {
  // w is the same for every lane of a wave; readfirstlane tells the
  // compiler so, which keeps each row's store base below in scalar registers
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int64_t c = (int64_t(blockIdx.x) * 64 + lane) * 4;
  const int64_t r0 = int64_t(blockIdx.y) * rpb;
  const int64_t r1 = r0 + rpb < Rr ? r0 + rpb : Rr;
  const bool live = c < Cc;
  auto put = [&](int64_t r, const T (&t)[4]) {
    // row r from the block's first column: wave-uniform (r is)
    T *const rb = gx + r * Cc + int64_t(blockIdx.x) * 256;
    T *p = rb + 4 * lane;
    VecT<T, 4> o;
    if constexpr (ACC) {
      const VecT<T, 4> old = vload<true, T, 4>(p);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o.v[e] = old.v[e] + t[e];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o.v[e] = t[e];
    }
    // (streaming stores measured 0.75-0.77 -> 0.80-0.81 of peak against
    // plain ones for the axis-0 and axis-1 max backward on [8192, 8192])
    vstore_out<true, 1, TK_SEL2D, T, 4>(rb, 4 * lane, true, o);
  };
  if constexpr (MODE == 1) {
    // reduced axis leading: column c's g / idx / count, loaded once
    if (!live)
      return;
    T gk[4];
    int64_t ik[4];
    bool ok[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      gk[e] = g[c + e];
      ik[e] = idx[c + e];
      ok[e] = cnt[c + e] == 1;
    }
    for (int64_t r = r0 + w; r < r1; r += RED_WAVES) {
      T t[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        t[e] = gk[e] * ((ok[e] && r == ik[e]) ? T(1) : T(0));
      put(r, t);
    }
  } else {
    // reduced axis trailing: row r's g / idx / count.  The block stages
    // its rows' values in LDS (one coalesced load per chunk of 256 rows)
    // so that the store stream does not wait on a load per row.
    __shared__ T sg[256];
    __shared__ int64_t si[256];
    for (int64_t rc = r0; rc < r1; rc += 256) {
      const int64_t nrc = r1 - rc < 256 ? r1 - rc : 256;
      if (threadIdx.x < nrc) {
        const int64_t r = rc + threadIdx.x;
        sg[threadIdx.x] = g[r];
        // a tie (count != 1) routes nothing: no column matches -1
        si[threadIdx.x] = cnt[r] == 1 ? idx[r] : int64_t(-1);
      }
      __syncthreads();
      if (live)
        for (int q = w; q < nrc; q += RED_WAVES) {
          const T gr = sg[q];
          const int64_t ir = si[q];
          T t[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            t[e] = gr * ((c + e == ir) ? T(1) : T(0));
          put(rc + q, t);
        }
      __syncthreads();
    }
  }
}

template <class T, bool ACC> struct BcastBwd {
  T scale;
  bool divide;
  static constexpr int NI = ACC ? 2 : 1;
  __device__ __forceinline__ void operator()(const T (&x)[NI],
                                             T (&y)[1]) const {
    const T t = divide ? x[0] / scale : x[0];
    if constexpr (ACC)
      y[0] = x[1] + t;
    else
      y[0] = t;
  }
};

} // namespace nt

using namespace nt;

namespace {

// nt_reduce's body; fixed: the static scratch's device address for the
// allocation-free variant, nullptr to take partials from the allocator.
void reduce_impl(int32_t op, const nt_view *x, const int64_t *axes,
                 int32_t naxes, const nt_view *out, const nt_view *idx,
                 const nt_view *count, void *fixed) {
  {
    check_view(x, "reduction");
    check_view(out, "reduction");
    if (naxes < 0 || naxes > x->ndim)
      fail(NT_ERR_INDEX, "reduction: bad axis count");
    if (naxes > 0 && !axes)
      fail(NT_ERR_RUNTIME, "reduction: null axes");
    RedPlan p = make_plan(x, axes, naxes);
    if (numel(out) != p.K)
      fail(NT_ERR_RUNTIME, "reduction: output size mismatch");
    if (!is_contiguous(out))
      fail(NT_ERR_RUNTIME, "reduction: output must be contiguous");
    if (numel(x) == 0)
      fail(NT_ERR_RUNTIME, "reduction: empty input");
    if (op == NT_SUM) {
      RedOut<0> ro{nullptr, nullptr, nullptr};
      ro.val = static_cast<char *>(out->data) +
               out->offset * int64_t(dtype_size(out->dtype));
      dispatch_all(x->dtype, [&]<class T>() {
        dispatch_arith(out->dtype, [&]<class O>() {
          run_reduce<T, O, SumAcc<O>, 0>(x, p, ro, fixed);
        });
      });
      return;
    }
    const bool is_max = (op == NT_MAX || op == NT_ARGMAX);
    if (op == NT_MAX || op == NT_MIN) {
      if (out->dtype != x->dtype)
        fail(NT_ERR_RUNTIME, "reduction: max/min output dtype mismatch");
      RedOut<1> ro{nullptr, nullptr, nullptr};
      ro.val = static_cast<char *>(out->data) +
               out->offset * int64_t(dtype_size(out->dtype));
      if (idx) {
        check_view(idx, "reduction");
        if (idx->dtype != NT_INT64 || numel(idx) != p.K || !is_contiguous(idx))
          fail(NT_ERR_RUNTIME, "reduction: idx must be contiguous int64");
        ro.idx = typed_ptr<int64_t>(idx);
      }
      if (count) {
        check_view(count, "reduction");
        if (count->dtype != NT_INT32 || numel(count) != p.K ||
            !is_contiguous(count))
          fail(NT_ERR_RUNTIME, "reduction: count must be contiguous int32");
        ro.cnt = typed_ptr<int32_t>(count);
      }
      dispatch_all(x->dtype, [&]<class T>() {
        if (is_max)
          run_reduce<T, T, SelAcc<T, true>, 1>(x, p, ro, fixed);
        else
          run_reduce<T, T, SelAcc<T, false>, 1>(x, p, ro, fixed);
      });
      return;
    }
    if (op == NT_ARGMAX || op == NT_ARGMIN) {
      if (out->dtype != NT_INT64)
        fail(NT_ERR_RUNTIME, "reduction: argmax/argmin output must be int64");
      RedOut<2> ro{typed_ptr<int64_t>(out), nullptr, nullptr};
      dispatch_all(x->dtype, [&]<class T>() {
        if (is_max)
          run_reduce<T, T, SelAcc<T, true>, 2>(x, p, ro, fixed);
        else
          run_reduce<T, T, SelAcc<T, false>, 2>(x, p, ro, fixed);
      });
      return;
    }
    fail(NT_ERR_VALUE, "reduction: unknown op");
  }
}

} // namespace

extern "C" {

int nt_reduce(int32_t op, const nt_view *x, const int64_t *axes, int32_t naxes,
              const nt_view *out, const nt_view *idx, const nt_view *count) {
  return guard(
      [&] { reduce_impl(op, x, axes, naxes, out, idx, count, nullptr); });
}

int nt_reduce_noalloc(int32_t op, const nt_view *x, const int64_t *axes,
                      int32_t naxes, const nt_view *out, const nt_view *idx,
                      const nt_view *count) {
  return guard_initialised([&] {
    reduce_impl(op, x, axes, naxes, out, idx, count, noalloc_scratch());
  });
}

int nt_reduce_bwd(int32_t op, const nt_view *g, double scale, const nt_view *idx,
                  const nt_view *count, const int64_t *axes, int32_t naxes,
                  const nt_view *gx, int32_t accumulate) {
  return guard([&] {
    check_view(g, "reduction_bwd");
    check_view(gx, "reduction_bwd");
    require_same_dtype(g, gx, "reduction_bwd");
    if (naxes < 0 || naxes > gx->ndim || (naxes > 0 && !axes))
      fail(NT_ERR_INDEX, "reduction_bwd: bad axes");
    bool is_drop[NT_MAX_DIMS] = {};
    for (int i = 0; i < naxes; ++i) {
      if (axes[i] < 0 || axes[i] >= gx->ndim || is_drop[axes[i]])
        fail(NT_ERR_INDEX, "reduction_bwd: bad axes");
      is_drop[axes[i]] = true;
    }
    // Row-major multipliers of the kept coordinates (g is contiguous over
    // the kept axes) and of the reduced coordinates in axis-tuple order.
    int64_t kmul[NT_MAX_DIMS] = {}, jmul[NT_MAX_DIMS] = {};
    int64_t K = 1, D = 1;
    for (int d = gx->ndim - 1; d >= 0; --d)
      if (!is_drop[d]) {
        kmul[d] = K;
        K *= gx->shape[d];
      }
    for (int i = naxes - 1; i >= 0; --i) {
      jmul[axes[i]] = D;
      D *= gx->shape[axes[i]];
    }
    if (numel(g) != K || !is_contiguous(g))
      fail(NT_ERR_RUNTIME, "reduction_bwd: g must be contiguous over kept axes");
    const int64_t n = numel(gx);
    if (n == 0)
      return;
    const bool acc = accumulate != 0;
    if (op == NT_SUM || op == NT_MEAN) {
      nt_view gb = *gx;
      gb.data = g->data;
      gb.offset = g->offset;
      for (int d = 0; d < gx->ndim; ++d)
        gb.strides[d] = is_drop[d] ? 0 : kmul[d];
      dispatch_float(g->dtype, [&]<class T>() {
        const nt_view *outs[1] = {gx};
        if (acc) {
          const nt_view *ins[2] = {&gb, gx};
          launch_elementwise<T, T, 2, 1>(
              ins, outs, BcastBwd<T, true>{T(scale), op == NT_MEAN});
        } else {
          const nt_view *ins[1] = {&gb};
          launch_elementwise<T, T, 1, 1>(
              ins, outs, BcastBwd<T, false>{T(scale), op == NT_MEAN});
        }
      });
      return;
    }
    if (op != NT_MAX && op != NT_MIN)
      fail(NT_ERR_VALUE, "reduction_bwd: unknown op");
    check_view(idx, "reduction_bwd");
    check_view(count, "reduction_bwd");
    if (idx->dtype != NT_INT64 || count->dtype != NT_INT32 ||
        numel(idx) != K || numel(count) != K || !is_contiguous(idx) ||
        !is_contiguous(count))
      fail(NT_ERR_RUNTIME, "reduction_bwd: bad idx/count");
    // Vector path: contiguous, aligned gx whose reduced axes are the
    // trailing, leading or all dims, in increasing order.
    {
      bool inc = true;
      for (int i = 1; i < naxes; ++i)
        if (axes[i] != axes[i - 1] + 1)
          inc = false;
      const bool trailing = inc && naxes > 0 && axes[naxes - 1] == gx->ndim - 1;
      const bool leading = inc && naxes > 0 && axes[0] == 0;
      const size_t es = dtype_size(gx->dtype);
      const bool ok = is_contiguous(gx) && n % 4 == 0 &&
                      n < (int64_t(1) << 32) &&
                      reinterpret_cast<uintptr_t>(
                          static_cast<char *>(gx->data) + gx->offset * es) %
                              (4 * es) == 0;
      int mode = -1;
      int64_t Cdim = 1;
      if (ok && trailing && leading) {
        mode = 2;
      } else if (ok && trailing && D % 4 == 0) {
        mode = 0;
        Cdim = D;
      } else if (ok && leading && K % 4 == 0) {
        mode = 1;
        Cdim = K;
      }
      if (mode >= 0) {
        const FastDivU32 fd{static_cast<uint32_t>(Cdim)};
        const int64_t n4 = n / 4;
        // one work-item per 16-byte group (a one-shot grid, like the
        // elementwise engine's: a grid-stride loop over 16 workgroups per CU
        // wrote the full-reduction gradient at 4.3 TB/s, this at 6.6)
        const int64_t blocks = std::max<int64_t>(1, ceil_div(n4, 256));
        dispatch_float(g->dtype, [&]<class T>() {
          const T *gp = typed_ptr<const T>(g);
          const int64_t *ip = typed_ptr<const int64_t>(idx);
          const int32_t *cp = typed_ptr<const int32_t>(count);
          T *xp = typed_ptr<T>(gx);
          const dim3 grid{unsigned(blocks), 1u, 1u};
          hipStream_t st = stream();
          const uint32_t Cu = uint32_t(Cdim);
          if (mode == 2) {
            if (acc)
              sel_bwd_vec_kernel<T, true, 2>
                  <<<grid, 256, 0, st>>>(gp, ip, cp, xp, fd, Cu, n4);
            else
              sel_bwd_vec_kernel<T, false, 2>
                  <<<grid, 256, 0, st>>>(gp, ip, cp, xp, fd, Cu, n4);
          } else {
            const int64_t Cc = Cdim, Rr = n / Cdim;
            const int64_t bx = ceil_div(Cc, 256);
            const int64_t target = int64_t(device_cu_count()) * NT_SEL2D_WG;
            const int64_t by = std::max<int64_t>(
                1, std::min<int64_t>(ceil_div(target, bx), ceil_div(Rr, 16)));
            const int64_t rpb = ceil_div(Rr, by);
            const dim3 g2{unsigned(bx), unsigned(ceil_div(Rr, rpb)), 1u};
#define NT_SEL2D(ACC, MODE)                                                    \
  sel_bwd_2d_kernel<T, ACC, MODE><<<g2, 256, 0, st>>>(gp, ip, cp, xp, Rr, Cc, \
                                                      rpb)
            if (acc && mode == 0)
              NT_SEL2D(true, 0);
            else if (acc)
              NT_SEL2D(true, 1);
            else if (mode == 0)
              NT_SEL2D(false, 0);
            else
              NT_SEL2D(false, 1);
#undef NT_SEL2D
          }
          NT_LAUNCH_CHECK();
        });
        return;
      }
    }
    SelBwdDesc dsc{};
    dsc.ndim = gx->ndim;
    const bool idx32 = n < (int64_t(1) << 32);
    for (int d = 0; d < gx->ndim; ++d) {
      dsc.shape[d] = gx->shape[d];
      if (idx32)
        dsc.fd[d] = FastDivU32(uint32_t(gx->shape[d]));
      dsc.gx_strides[d] = gx->strides[d];
      dsc.kmul[d] = kmul[d];
      dsc.jmul[d] = jmul[d];
    }
    const int64_t blocks =
        std::max<int64_t>(1, std::min<int64_t>(ceil_div(n, 256 * 4), 1 << 20));
    dispatch_float(g->dtype, [&]<class T>() {
      const T *gp = typed_ptr<const T>(g);
      const int64_t *ip = typed_ptr<const int64_t>(idx);
      const int32_t *cp = typed_ptr<const int32_t>(count);
      T *op_ = typed_ptr<T>(gx);
      hipStream_t st = stream();
      if (acc) {
        if (idx32)
          sel_bwd_kernel<T, true, true>
              <<<dim3(unsigned(blocks)), 256, 0, st>>>(gp, ip, cp, op_, dsc, n);
        else
          sel_bwd_kernel<T, true, false>
              <<<dim3(unsigned(blocks)), 256, 0, st>>>(gp, ip, cp, op_, dsc, n);
      } else {
        if (idx32)
          sel_bwd_kernel<T, false, true>
              <<<dim3(unsigned(blocks)), 256, 0, st>>>(gp, ip, cp, op_, dsc, n);
        else
          sel_bwd_kernel<T, false, false>
              <<<dim3(unsigned(blocks)), 256, 0, st>>>(gp, ip, cp, op_, dsc, n);
      }
      NT_LAUNCH_CHECK();
    });
  });
}

} // extern "C"
