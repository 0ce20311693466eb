// Advanced (sequence / mask) indexing: gather from and scatter to a view
// along "fancy" axes selected by int64 index arrays.
//
// The plan (which axes are fancy, the output shape and where each output
// axis comes from) is the reference's _FancyAxes (src/nanotorch/core.py:667-
// 774), computed by the Python layer, which also normalises negative
// indices, checks bounds and turns boolean masks into index lists (those
// steps raise IndexError / RuntimeError exactly where the reference does).
// The reference runs both loops on the host only (src/cpp/ops/copy_ops.cu:
// 7-160, `_require_cpu`); here one work-item moves one element, or one
// 16-byte vector of the innermost axis when the layout allows:
//
//   gather : out[o] = x[src(o)],  o over the contiguous output
//   scatter: out[dst(s)] = src[s], s over the (broadcast) source
//
// With all index arrays broadcast to one index shape, output axis i either
// walks index axis out_axis_target[i] (fancy) or view axis out_axis_target[i]
// (basic); view axis d takes idx_p[flat index coordinate] when it is the
// p-th fancy axis.  A scatter whose index tuples repeat writes each target
// once, from the last occurrence in row-major order (the reference's
// sequential "last write wins"): the host marks, per index position,
// whether it is the last occurrence of its tuple (`keep`).
#include "ew_engine.h"


namespace nt {

constexpr int IDX_MAX_FANCY = NT_MAX_DIMS;
// Workgroups per CU of the grid-stride gather / scatter (32 measured 4%
// faster than 16 on a row gather; 64 no faster).
#ifndef NT_IDX_WG_PER_CU
#define NT_IDX_WG_PER_CU 32
#endif
// Workgroups per CU for whole-row gathers / scatters (each takes rows in a
// grid-stride loop).
#ifndef NT_IDX_ROW_WG_PER_CU
#define NT_IDX_ROW_WG_PER_CU 16
#endif

struct IndexPlan {
  int out_ndim;    // dims of the iteration space (gather: out, scatter: src)
  int view_ndim;   // dims of the indexed view
  int ind_ndim;    // dims of the broadcast index shape
  int nfancy;
  int64_t shape[NT_MAX_DIMS];      // iteration-space shape
  FastDivU32 fd[NT_MAX_DIMS];      // its divisors (32-bit indexing)
  int is_fancy[NT_MAX_DIMS];       // per iteration axis
  int target[NT_MAX_DIMS];         // index axis (fancy) or view axis (basic)
  int fancy_slot[NT_MAX_DIMS];     // per view axis: p, or -1 for basic
  int64_t view_shape[NT_MAX_DIMS];
  int64_t view_strides[NT_MAX_DIMS];
  int64_t view_offset;
  int64_t iter_strides[NT_MAX_DIMS]; // the other operand's strides over the
  int64_t iter_offset;               // iteration space (out: contiguous)
  int64_t ind_strides[IDX_MAX_FANCY][NT_MAX_DIMS]; // per index array
  const int64_t *ind[IDX_MAX_FANCY];
  const uint8_t *keep; // scatter: last-occurrence mask, contiguous over the
  int64_t keep_strides[NT_MAX_DIMS]; // index shape (may be null)
};

// Offsets of iteration element `it` in the indexed view and in the other
// operand; false when a scatter skips it (an earlier repeat of a tuple) or
// an index lies outside its axis (then *err is set; the host checks every
// index before the call, this keeps a bad C-ABI call from touching memory
// outside the view).
template <bool IDX32>
__device__ __forceinline__ bool index_offsets(const IndexPlan &p, int64_t it,
                                              int64_t &view_off,
                                              int64_t &iter_off, int *err) {
  int64_t loc_ind[NT_MAX_DIMS];
  int64_t loc_basic[NT_MAX_DIMS];
  int64_t io = p.iter_offset;
  if constexpr (IDX32) {
    uint32_t rem = uint32_t(it);
    for (int d = p.out_ndim - 1; d >= 0; --d) {
      const uint32_t q = p.fd[d].div(rem);
      const int64_t c = int64_t(rem - q * uint32_t(p.shape[d]));
      rem = q;
      io += c * p.iter_strides[d];
      if (p.is_fancy[d])
        loc_ind[p.target[d]] = c;
      else
        loc_basic[p.target[d]] = c;
    }
  } else {
    int64_t rem = it;
    for (int d = p.out_ndim - 1; d >= 0; --d) {
      const int64_t q = rem / p.shape[d];
      const int64_t c = rem - q * p.shape[d];
      rem = q;
      io += c * p.iter_strides[d];
      if (p.is_fancy[d])
        loc_ind[p.target[d]] = c;
      else
        loc_basic[p.target[d]] = c;
    }
  }
  if (p.keep) {
    int64_t ko = 0;
    for (int d = 0; d < p.ind_ndim; ++d)
      ko += loc_ind[d] * p.keep_strides[d];
    if (!p.keep[ko])
      return false;
  }
  int64_t vo = p.view_offset;
  for (int d = 0; d < p.view_ndim; ++d) {
    const int slot = p.fancy_slot[d];
    int64_t c;
    if (slot < 0) {
      c = loc_basic[d];
    } else {
      int64_t fo = 0;
      for (int e = 0; e < p.ind_ndim; ++e)
        fo += loc_ind[e] * p.ind_strides[slot][e];
      c = p.ind[slot][fo];
      if (c < 0 || c >= p.view_shape[d]) {
        *err = NT_ERR_INDEX; // the deferred-error word (host memory)
        iter_off = io;
        return false;
      }
    }
    vo += c * p.view_strides[d];
  }
  view_off = vo;
  iter_off = io;
  return true;
}

// Work-item g moves VEC consecutive elements of the innermost iteration
// axis (VEC > 1 only when that axis is basic, unit-stride in both operands
// and a multiple of VEC long, and every vector is aligned: then the group's
// offsets are those of its first element).
template <class T, bool IDX32, int VEC>
__global__ __launch_bounds__(256) void gather_kernel(const T *__restrict__ x,
                                                     T *__restrict__ out,
                                                     IndexPlan p, int64_t ngroups,
                                                     int *err) {
  using V = VecT<T, VEC>;
  const int64_t stride = int64_t(gridDim.x) * 256;
  for (int64_t g = int64_t(blockIdx.x) * 256 + threadIdx.x; g < ngroups;
       g += stride) {
    int64_t vo = 0, io = 0;
    const bool ok = index_offsets<IDX32>(p, g * VEC, vo, io, err);
    V v;
    if (ok) {
      v = *reinterpret_cast<const V *>(x + vo);
    } else {
#pragma unroll
      for (int j = 0; j < VEC; ++j)
        v.v[j] = T(0);
    }
    *reinterpret_cast<V *>(out + io) = v;
  }
}

template <class T, bool IDX32, int VEC>
__global__ __launch_bounds__(256) void scatter_kernel(const T *__restrict__ src,
                                                      T *__restrict__ out,
                                                      IndexPlan p, int64_t ngroups,
                                                      int *err) {
  using V = VecT<T, VEC>;
  const int64_t stride = int64_t(gridDim.x) * 256;
  for (int64_t g = int64_t(blockIdx.x) * 256 + threadIdx.x; g < ngroups;
       g += stride) {
    int64_t vo = 0, io = 0;
    if (index_offsets<IDX32>(p, g * VEC, vo, io, err))
      *reinterpret_cast<V *>(out + vo) = *reinterpret_cast<const V *>(src + io);
  }
}

// Whole rows: the view is [R, C] with unit-stride rows, one 1-D index array
// selects along axis 0, and the iteration space is [n, C] (a row gather
// out[i, :] = x[idx[i], :], or a row scatter x[idx[i], :] = src[i, :]).  A
// workgroup takes row i, loads idx[i] once and moves the row in VEC-element
// vectors; an index outside the axis is reported as in index_offsets (a
// gather writes a zero row) and a scatter skips rows the keep mask drops.
template <class T, int VEC, bool SCATTER>
__global__ __launch_bounds__(256) void row_index_kernel(T *view, T *iter,
                                                        IndexPlan p, int *err) {
  using V = VecT<T, VEC>;
  const int64_t n = p.shape[0], cv = p.shape[1] / VEC;
  for (int64_t i = blockIdx.x; i < n; i += gridDim.x) {
    if (SCATTER && p.keep && !p.keep[i * p.keep_strides[0]])
      continue;
    const int64_t r = p.ind[0][i * p.ind_strides[0][0]];
    V *it_row = reinterpret_cast<V *>(iter + p.iter_offset + i * p.iter_strides[0]);
    if (r < 0 || r >= p.view_shape[0]) {
      if (threadIdx.x == 0)
        *err = NT_ERR_INDEX; // the deferred-error word (host memory)
      if constexpr (!SCATTER) {
        V z;
#pragma unroll
        for (int j = 0; j < VEC; ++j)
          z.v[j] = T(0);
        for (int64_t v = threadIdx.x; v < cv; v += 256)
          it_row[v] = z;
      }
      continue;
    }
    V *vw_row = reinterpret_cast<V *>(view + p.view_offset + r * p.view_strides[0]);
    for (int64_t v = threadIdx.x; v < cv; v += 256) {
      if constexpr (SCATTER)
        vw_row[v] = it_row[v];
      else
        it_row[v] = vw_row[v];
    }
  }
}

namespace {

// Validates the plan's arrays and fills everything but the iteration
// operand.  `iter` is the iteration space (gather: out, scatter: src).
IndexPlan make_index_plan(const nt_view *view, const nt_view *iter,
                          int32_t nfancy, const int32_t *fancy_dims,
                          const nt_view *index_arrays,
                          const int32_t *out_axis_is_fancy,
                          const int32_t *out_axis_target,
                          const nt_view *keep) {
  IndexPlan p{};
  if (nfancy < 1 || nfancy > IDX_MAX_FANCY)
    fail(NT_ERR_RUNTIME, "indexing: bad number of index arrays");
  p.out_ndim = iter->ndim;
  p.view_ndim = view->ndim;
  p.nfancy = nfancy;
  p.ind_ndim = index_arrays[0].ndim;
  for (int d = 0; d < NT_MAX_DIMS; ++d)
    p.fancy_slot[d] = -1;
  for (int q = 0; q < nfancy; ++q) {
    const nt_view &iv = index_arrays[q];
    check_view(&iv, "indexing");
    if (iv.dtype != NT_INT64)
      fail(NT_ERR_RUNTIME, "indexing: index arrays must be int64");
    if (iv.ndim != p.ind_ndim)
      fail(NT_ERR_RUNTIME, "indexing: index arrays of different ranks");
    for (int d = 0; d < p.ind_ndim; ++d) {
      if (iv.shape[d] != index_arrays[0].shape[d])
        fail(NT_ERR_RUNTIME, "indexing: index arrays of different shapes");
      p.ind_strides[q][d] = iv.strides[d];
    }
    p.ind[q] = typed_ptr<const int64_t>(&iv);
    const int d = fancy_dims[q];
    if (d < 0 || d >= view->ndim || p.fancy_slot[d] != -1)
      fail(NT_ERR_RUNTIME, "indexing: bad fancy axis");
    p.fancy_slot[d] = q;
  }
  for (int i = 0; i < iter->ndim; ++i) {
    p.shape[i] = iter->shape[i];
    p.is_fancy[i] = out_axis_is_fancy[i] ? 1 : 0;
    p.target[i] = out_axis_target[i];
    const int lim = p.is_fancy[i] ? p.ind_ndim : view->ndim;
    if (p.target[i] < 0 || p.target[i] >= lim)
      fail(NT_ERR_RUNTIME, "indexing: bad axis plan");
    const int64_t ext = p.is_fancy[i] ? index_arrays[0].shape[p.target[i]]
                                      : view->shape[p.target[i]];
    if (ext != p.shape[i])
      fail(NT_ERR_RUNTIME, "indexing: shape does not match the axis plan");
    p.iter_strides[i] = iter->strides[i];
  }
  // every basic view axis and every index axis is walked by exactly one
  // iteration axis (otherwise a coordinate would be left undefined)
  int basic_seen[NT_MAX_DIMS] = {}, ind_seen[NT_MAX_DIMS] = {};
  for (int i = 0; i < iter->ndim; ++i) {
    if (p.is_fancy[i])
      ++ind_seen[p.target[i]];
    else if (p.fancy_slot[p.target[i]] >= 0)
      fail(NT_ERR_RUNTIME, "indexing: a basic axis of the plan is fancy");
    else
      ++basic_seen[p.target[i]];
  }
  for (int d = 0; d < view->ndim; ++d)
    if (p.fancy_slot[d] < 0 && basic_seen[d] != 1)
      fail(NT_ERR_RUNTIME, "indexing: axis plan does not cover the view");
  for (int d = 0; d < p.ind_ndim; ++d)
    if (ind_seen[d] != 1)
      fail(NT_ERR_RUNTIME, "indexing: axis plan does not cover the indices");
  p.iter_offset = iter->offset;
  for (int d = 0; d < view->ndim; ++d) {
    p.view_shape[d] = view->shape[d];
    p.view_strides[d] = view->strides[d];
  }
  p.view_offset = view->offset;
  p.keep = nullptr;
  if (keep) {
    check_view(keep, "indexing");
    if (keep->dtype != NT_BOOL || keep->ndim != p.ind_ndim)
      fail(NT_ERR_RUNTIME, "indexing: bad keep mask");
    for (int d = 0; d < p.ind_ndim; ++d) {
      if (keep->shape[d] != index_arrays[0].shape[d])
        fail(NT_ERR_RUNTIME, "indexing: bad keep mask");
      p.keep_strides[d] = keep->strides[d];
    }
    p.keep = reinterpret_cast<const uint8_t *>(
        static_cast<const char *>(keep->data) + keep->offset);
  }
  return p;
}

// Vector width for the plan: VEC elements of the innermost iteration axis
// per work-item when that axis is basic and unit-stride in both operands,
// its length is a multiple of VEC, and every vector start is VEC-aligned
// (every other stride a multiple of VEC, both bases aligned).
template <class T>
int index_vec(const nt_view *data, const nt_view *iter, const IndexPlan &p) {
  constexpr int V = ew_vec<T>();
  if (V == 1 || p.out_ndim == 0)
    return 1;
  const int last = p.out_ndim - 1;
  if (p.is_fancy[last] || p.iter_strides[last] != 1 ||
      p.view_strides[p.target[last]] != 1 || p.shape[last] % V != 0)
    return 1;
  for (int i = 0; i < last; ++i)
    if (p.iter_strides[i] % V != 0)
      return 1;
  for (int d = 0; d < p.view_ndim; ++d)
    if (p.view_strides[d] % V != 0 && d != p.target[last])
      return 1;
  const auto al = [&](const nt_view *v) {
    return (reinterpret_cast<uintptr_t>(v->data) + uintptr_t(v->offset) * sizeof(T)) %
               (V * sizeof(T)) == 0;
  };
  return al(data) && al(iter) ? V : 1;
}

// Queues the kernel and returns: an index outside its axis (possible only
// for a caller that skipped the host-side checks) is skipped -- a gather
// writes zeros there -- and stored in the deferred-error word, which the
// next nt_sync / device-to-host copy raises as NT_ERR_INDEX.
template <bool SCATTER>
void run_index(const nt_view *data, const nt_view *iter, const IndexPlan &base) {
  const int64_t n = numel(iter);
  if (n == 0)
    return;
  IndexPlan p = base;
  const bool idx32 = n < (int64_t(1) << 32);
  if (idx32)
    for (int d = 0; d < p.out_ndim; ++d)
      p.fd[d] = FastDivU32(uint32_t(p.shape[d]));
  hipStream_t st = stream();
  int *err = deferred_error_word();
  dispatch_all(data->dtype, [&]<class T>() {
    // raw storage pointers: the plan carries both offsets
    T *dptr = static_cast<T *>(const_cast<void *>(data->data));
    T *iptr = static_cast<T *>(const_cast<void *>(iter->data));
    const int vec = index_vec<T>(data, iter, p);
    constexpr int V = ew_vec<T>();
    if (vec > 1 && p.out_ndim == 2 && p.view_ndim == 2 && p.nfancy == 1 &&
        p.ind_ndim == 1 && p.is_fancy[0] && !p.is_fancy[1] &&
        p.target[0] == 0 && p.target[1] == 1 && p.fancy_slot[0] == 0 &&
        p.fancy_slot[1] < 0) {
      const dim3 rgrid{unsigned(std::min<int64_t>(
                           p.shape[0], int64_t(device_cu_count()) *
                                           NT_IDX_ROW_WG_PER_CU)),
                       1u, 1u};
      if constexpr (V > 1)
        row_index_kernel<T, V, SCATTER>
            <<<rgrid, 256, 0, st>>>(dptr, iptr, p, err);
      return;
    }
    const int64_t groups = n / vec;
    const dim3 grid{unsigned(std::min<int64_t>((groups + 255) / 256,
                                               int64_t(device_cu_count()) * NT_IDX_WG_PER_CU)),
                    1u, 1u};
#define NT_IDX_LAUNCH(K, A, B, I32, VV)                                        \
  K<T, I32, VV><<<grid, 256, 0, st>>>(A, B, p, groups, err)
    if constexpr (SCATTER) {
      if (vec > 1 && idx32)
        NT_IDX_LAUNCH(scatter_kernel, iptr, dptr, true, V);
      else if (vec > 1)
        NT_IDX_LAUNCH(scatter_kernel, iptr, dptr, false, V);
      else if (idx32)
        NT_IDX_LAUNCH(scatter_kernel, iptr, dptr, true, 1);
      else
        NT_IDX_LAUNCH(scatter_kernel, iptr, dptr, false, 1);
    } else {
      if (vec > 1 && idx32)
        NT_IDX_LAUNCH(gather_kernel, dptr, iptr, true, V);
      else if (vec > 1)
        NT_IDX_LAUNCH(gather_kernel, dptr, iptr, false, V);
      else if (idx32)
        NT_IDX_LAUNCH(gather_kernel, dptr, iptr, true, 1);
      else
        NT_IDX_LAUNCH(gather_kernel, dptr, iptr, false, 1);
    }
#undef NT_IDX_LAUNCH
  });
  NT_LAUNCH_CHECK();
}

} // namespace
} // namespace nt

using namespace nt;

extern "C" {

int nt_gather_axes(const nt_view *x, const nt_view *out, int32_t nfancy,
                   const int32_t *fancy_dims_in_src,
                   const nt_view *index_arrays,
                   const int32_t *out_axis_is_fancy,
                   const int32_t *out_axis_target) {
  return guard([&] {
    check_view(x, "gather_from_axes");
    check_view(out, "gather_from_axes");
    if (x->dtype != out->dtype)
      fail(NT_ERR_RUNTIME, "gather_from_axes: dtype mismatch");
    const IndexPlan p =
        make_index_plan(x, out, nfancy, fancy_dims_in_src, index_arrays,
                        out_axis_is_fancy, out_axis_target, nullptr);
    run_index<false>(x, out, p);
  });
}

int nt_scatter_axes(const nt_view *src, const nt_view *out, int32_t nfancy,
                    const int32_t *fancy_dims_in_src,
                    const nt_view *index_arrays,
                    const int32_t *out_axis_is_fancy,
                    const int32_t *out_axis_target, const nt_view *keep) {
  return guard([&] {
    check_view(src, "scatter_to_axes");
    check_view(out, "scatter_to_axes");
    if (src->dtype != out->dtype)
      fail(NT_ERR_RUNTIME, "scatter_to_axes: dtype mismatch");
    const IndexPlan p =
        make_index_plan(out, src, nfancy, fancy_dims_in_src, index_arrays,
                        out_axis_is_fancy, out_axis_target, keep);
    run_index<true>(out, src, p);
  });
}

} // extern "C"
