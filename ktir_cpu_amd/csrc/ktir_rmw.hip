// Ordered indirect read-modify-write of rows (scatter-accumulate through
// indirect access tiles), bit-exact against sequential execution.
//
// Reference order (grid.py:595-616, ops/memory_ops.py:868-964, memory.py:281-291):
// instances (core, loop iteration) run one after another; each one gathers
// K destination rows, combines them with K source rows, and scatters them
// back, where a destination repeated inside one instance keeps the value
// of its last position (computed from the row as it was before the instance).
//
//   pass 1 (one workgroup per instance): find the surviving (last) position of
//     every destination row inside the instance and push it on that row's
//     chain: link[e] = atomicExch(&head[row], e); non-survivors get -2.
//   pass 2 (one wavefront per entry): the entry whose link is -1 (the first
//     one pushed) owns the row: it walks the chain, orders the entries by e
//     (= instance order) and applies them one after another, so the floating
//     point accumulation order is exactly the reference's.
#include "ktir_common.h"

namespace ktir {

__device__ __forceinline__ int64_t read_index(uint64_t ptr, int dt, int64_t e, int64_t hi, bool* bad) {
  if (e < 0 || e >= hi) return 0;   // over-read of the index tensor reads zeros
  int64_t v;
  switch (dt) {
    case KTIR_I64: v = ((const int64_t*)ptr)[e]; break;
    case KTIR_I16: v = ((const int16_t*)ptr)[e]; break;
    case KTIR_I8: v = ((const int8_t*)ptr)[e]; break;
    default: v = ((const int32_t*)ptr)[e]; break;
  }
  if (v < 0) *bad = true;
  return v;
}

__device__ __forceinline__ float combine(int op, int order, int dt, float dst, float src) {
  float a = order ? src : dst, b = order ? dst : src;
  float r;
  switch (op) {
    case KTIR_OP_ADDF: r = __fadd_rn(a, b); break;
    case KTIR_OP_SUBF: r = __fsub_rn(a, b); break;
    case KTIR_OP_MULF: r = __fmul_rn(a, b); break;
    case KTIR_OP_MAXIMUMF: r = (a != a || b != b) ? __int_as_float(0x7fc00000) : fmaxf(a, b); break;
    case KTIR_OP_MINIMUMF: r = (a != a || b != b) ? __int_as_float(0x7fc00000) : fminf(a, b); break;
    case KTIR_OP_MAXNUMF: r = fmaxf(a, b); break;
    case KTIR_OP_MINNUMF: r = fminf(a, b); break;
    default: r = a;
  }
  return round_to(r, dt);
}

constexpr int RMW_MAXK = 1024;

__global__ __launch_bounds__(256) void rmw_link(const ktir_rmw_t d, int* err) {
  __shared__ int32_t rows[RMW_MAXK];
  const int64_t inst = blockIdx.x;
  const int64_t p0 = ((const int64_t*)d.dst_pos)[inst];
  bool bad = false;
  for (int k = threadIdx.x; k < d.K; k += blockDim.x) {
    int64_t r = read_index(d.dst_idx_ptr, d.dst_idx_dtype, p0 + k, d.dst_idx_hi, &bad);
    rows[k] = (r >= 0 && r < d.n_rows) ? (int32_t)r : -1;
  }
  if (bad) *err = 1;
  __syncthreads();
  for (int k = threadIdx.x; k < d.K; k += blockDim.x) {
    const int64_t e = inst * d.K + k;
    int32_t r = rows[k];
    bool last = r >= 0;
    for (int j = k + 1; j < d.K && last; ++j) last = rows[j] != r;
    ((int32_t*)d.link)[e] = last ? atomicExch(&((int32_t*)d.head)[r], (int32_t)e) : -2;
  }
}

// one wavefront per entry; lanes cover the row's D columns.  No barriers:
// every lane walks the (short) chain itself and visits its entries in
// ascending position order by repeated selection.
__global__ __launch_bounds__(256) void rmw_apply(const ktir_rmw_t d, int* err) {
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int64_t total = d.n_inst * d.K;
  const int64_t e = (int64_t)blockIdx.x * 4 + wave;
  if (e >= total) return;
  const int32_t* link = (const int32_t*)d.link;
  if (link[e] != -1) return;                       // not a row owner
  const int64_t inst = e / d.K, k = e - inst * d.K;
  bool bad = false;
  const int64_t r = read_index(d.dst_idx_ptr, d.dst_idx_dtype, ((const int64_t*)d.dst_pos)[inst] + k,
                               d.dst_idx_hi, &bad);
  const int32_t head = ((const int32_t*)d.head)[r];
  int m = 0;
  for (int32_t x = head; x >= 0; x = link[x]) ++m;
  const int64_t drow = d.dst_base + r * d.dst_row;
  for (int64_t c = lane; c < d.D; c += 64) {
    const int64_t de = drow + c * d.dst_col;
    const bool dok = de >= 0 && de < d.dst_hi;
    float v = dok ? load_elem(d.dst_ptr, de, d.dst_dtype) : 0.f;
    int32_t prev = -1;
    for (int i = 0; i < m; ++i) {
      int32_t ent = 0x7fffffff;
      for (int32_t x = head; x >= 0; x = link[x])
        if (x > prev && x < ent) ent = x;
      prev = ent;
      const int64_t ei = ent / d.K, ek = ent - ei * d.K;
      const int64_t s = read_index(d.src_idx_ptr, d.src_idx_dtype, ((const int64_t*)d.src_pos)[ei] + ek,
                                   d.src_idx_hi, &bad);
      const int64_t se = d.src_base + s * d.src_row + c * d.src_col;
      float g = (se >= 0 && se < d.src_hi) ? load_elem(d.src_ptr, se, d.src_dtype) : 0.f;
      v = combine(d.op, d.order, d.dt, v, g);
    }
    if (dok) store_elem(d.dst_ptr, de, d.dst_dtype, v);
  }
  if (bad) *err = 1;
}

}  // namespace ktir

using namespace ktir;

extern "C" int ktir_launch_row_rmw(const ktir_rmw_t* d) {
  if (!d || d->K < 1 || d->K > RMW_MAXK || d->D < 1 || d->n_inst < 0)
    return set_error(KTIR_E_ARG, "ktir_launch_row_rmw: bad descriptor");
  if (d->n_inst * d->K >= (int64_t)0x7fffffff || d->n_rows >= (int64_t)0x7fffffff)
    return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_row_rmw: too many entries");
  if (d->n_inst == 0) return KTIR_OK;
  // head table to -1 (all bytes 0xff)
  KTIR_HIP_CHECK(hipMemsetAsync((void*)d->head, 0xff, (size_t)d->n_rows * 4, stream()));
  int t1 = d->K >= 256 ? 256 : (int)((d->K + 63) / 64 * 64);
  hipLaunchKernelGGL(rmw_link, dim3((unsigned)d->n_inst), dim3(t1), 0, stream(), *d, device_error_flag());
  int64_t total = d->n_inst * d->K;
  hipLaunchKernelGGL(rmw_apply, dim3((unsigned)((total + 3) / 4)), dim3(256), 0, stream(), *d, device_error_flag());
  KTIR_HIP_CHECK(hipGetLastError());
  return KTIR_OK;
}
