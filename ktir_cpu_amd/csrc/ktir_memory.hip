// Indirect access tiles and last-writer-wins scatters.
//
// Reference: ops/memory_ops.py:224-576 builds, for every point of an indirect
// access tile's variable space, the parent-tensor coordinates: direct
// dimensions come from the iteration variables, indirect ones from values read
// out of index tensors (negative values raise IndexError, :378-382).  Here the
// host computes the data-independent parts (direct offsets and the positions
// of the index reads) and one kernel reads the index values on the device and
// forms flat element offsets.
//
// Scatter semantics (reference memory.py:281-291): a fancy-index write where a
// repeated destination keeps the value of the LAST position in enumeration
// order.  ktir_scatter_winners records, per destination element, the largest
// writing position; the store then writes only from that position.
#include "ktir_common.h"

namespace ktir {

__global__ void iat_offsets_kernel(const ktir_iat_t d, int* err) {
  const int64_t total = d.lanes * d.n;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    int64_t l = t / d.n, p = t - l * d.n;
    int64_t off = ((const int64_t*)d.dir)[l * d.dir_ls + p];
    for (int k = 0; k < d.n_ind; ++k) {
      int64_t e = ((const int64_t*)d.pos[k])[l * d.pos_ls[k] + p];
      if (d.pos_lane[k]) e += ((const int64_t*)d.pos_lane[k])[l];
      int64_t v = 0;
      if (e >= d.idx_lo[k] && e < d.idx_hi[k]) {
        switch (d.idx_dtype[k]) {
          case KTIR_I64: v = ((const int64_t*)d.idx_ptr[k])[e]; break;
          case KTIR_I16: v = ((const int16_t*)d.idx_ptr[k])[e]; break;
          case KTIR_I8: v = ((const int8_t*)d.idx_ptr[k])[e]; break;
          default: v = ((const int32_t*)d.idx_ptr[k])[e]; break;
        }
      }
      if (v < 0) {
        *err = 1;
        v = 0;
      }
      off += v * d.stride[k];
    }
    ((int64_t*)d.out)[t] = off;
  }
}

__global__ void winners_clear(const ktir_leaf_t L, int64_t lanes, int64_t n, int32_t* win) {
  const int64_t total = lanes * n;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    int64_t l = t / n, i = t - l * n;
    int64_t e = lane_offset(L, l) + ((const int64_t*)L.offsets)[l * L.offsets_lane_stride + i];
    if (e >= L.lo && e < L.hi) win[e - L.winner_base] = -1;
  }
}

__global__ void winners_max(const ktir_leaf_t L, int64_t lanes, int64_t n, int32_t* win) {
  const int64_t total = lanes * n;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    int64_t l = t / n, i = t - l * n;
    int64_t e = lane_offset(L, l) + ((const int64_t*)L.offsets)[l * L.offsets_lane_stride + i];
    if (e >= L.lo && e < L.hi) atomicMax(&win[e - L.winner_base], (int32_t)t);
  }
}

static unsigned grid_for(int64_t total) {
  int64_t b = (total + 255) / 256;
  if (b > 65536) b = 65536;
  return (unsigned)(b < 1 ? 1 : b);
}

}  // namespace ktir

using namespace ktir;

extern "C" int ktir_iat_offsets(const ktir_iat_t* d) {
  if (!d || d->n_ind < 0 || d->n_ind > 4) return set_error(KTIR_E_ARG, "ktir_iat_offsets: bad descriptor");
  int64_t total = d->lanes * d->n;
  if (total == 0) return KTIR_OK;
  hipLaunchKernelGGL(iat_offsets_kernel, dim3(grid_for(total)), dim3(256), 0, stream(), *d, device_error_flag());
  KTIR_HIP_CHECK(hipGetLastError());
  return KTIR_OK;
}

extern "C" int ktir_scatter_winners(const ktir_leaf_t* leaf, int64_t lanes, int64_t n, uint64_t winner) {
  if (!leaf || !leaf->offsets || !winner) return set_error(KTIR_E_ARG, "ktir_scatter_winners: needs offsets and table");
  if (lanes * n >= (int64_t)0x7fffffff) return set_error(KTIR_E_UNSUPPORTED, "scatter of %lld elements", (long long)(lanes * n));
  int64_t total = lanes * n;
  if (total == 0) return KTIR_OK;
  hipLaunchKernelGGL(winners_clear, dim3(grid_for(total)), dim3(256), 0, stream(), *leaf, lanes, n, (int32_t*)winner);
  hipLaunchKernelGGL(winners_max, dim3(grid_for(total)), dim3(256), 0, stream(), *leaf, lanes, n, (int32_t*)winner);
  KTIR_HIP_CHECK(hipGetLastError());
  return KTIR_OK;
}
