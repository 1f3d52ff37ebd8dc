// Batched matmul tiles: one [M,K] x [K,N] product per lane, optionally fused
// over an scf.for K loop (ksteps steps advancing A and B).
//
// Reference semantics (dialects/linalg_ops.py:307-369, ops/arith_ops.py:324-340):
// result = np.matmul(a, b).astype(a.dtype), then `outs += result`.  f16
// products are exact in f32 and accumulate in f32, so the MFMA path below
// (f16/bf16 operands, f32 accumulator) differs from the reference only in
// summation order, which the reference's own tests bound by tolerance.
#include "ktir_common.h"

namespace ktir {

// Generic path: 64x64 output tile per workgroup, 256 threads x (4x4) outputs,
// K staged through LDS in chunks of 16, f32 FMA.  Operands of any dtype are
// read through their leaves (bounds-checked like every other leaf read).
constexpr int GT = 64, GK = 16;

__global__ __launch_bounds__(256) void mm_generic(const ktir_mm_t d) {
  __shared__ float As[GK][GT + 1];
  __shared__ float Bs[GK][GT + 1];
  const int64_t tiles_m = (d.M + GT - 1) / GT, tiles_n = (d.N + GT - 1) / GT;
  const int64_t per_lane = tiles_m * tiles_n;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  for (int64_t w = blockIdx.x; w < d.lanes * per_lane; w += gridDim.x) {
    int64_t lane = w / per_lane, t = w - lane * per_lane;
    int64_t m0 = (t / tiles_n) * GT, n0 = (t % tiles_n) * GT;
    float acc[4][4];
    for (int i = 0; i < 4; ++i)
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
    const int64_t abase = lane_offset(d.a, lane), bbase = lane_offset(d.b, lane);
    for (int64_t s = 0; s < d.ksteps; ++s) {
      const int64_t ao = abase + s * d.a_kstep, bo = bbase + s * d.b_kstep;
      for (int64_t k0 = 0; k0 < d.K; k0 += GK) {
        for (int i = threadIdx.x; i < GK * GT; i += 256) {
          int kk = i / GT, mm = i % GT;
          int64_t gm = m0 + mm, gk = k0 + kk;
          float va = 0.f;
          if (gm < d.M && gk < d.K) {
            int64_t e = ao + gm * d.a.strides[0] + gk * d.a.strides[1];
            va = (e >= d.a.lo && e < d.a.hi) ? load_elem(d.a.ptr, e, d.a.dtype) : 0.f;
          }
          As[kk][mm] = va;
          int64_t gn = n0 + mm;
          float vb = 0.f;
          if (gn < d.N && gk < d.K) {
            int64_t e = bo + gk * d.b.strides[0] + gn * d.b.strides[1];
            vb = (e >= d.b.lo && e < d.b.hi) ? load_elem(d.b.ptr, e, d.b.dtype) : 0.f;
          }
          Bs[kk][mm] = vb;
        }
        __syncthreads();
        for (int kk = 0; kk < GK; ++kk) {
          float a[4], b[4];
          for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
          for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
          for (int i = 0; i < 4; ++i)
            for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
      }
    }
    const int64_t cbase = lane_offset(d.c, lane);
    const int64_t c0base = d.accumulate == 1 ? lane_offset(d.c0, lane) : 0;
    for (int i = 0; i < 4; ++i) {
      int64_t gm = m0 + ty * 4 + i;
      if (gm >= d.M) continue;
      for (int j = 0; j < 4; ++j) {
        int64_t gn = n0 + tx * 4 + j;
        if (gn >= d.N) continue;
        // np.matmul(...).astype(a.dtype): round the product to the result dtype
        // first, then accumulate into outs (the reference's two roundings).
        float v = round_to(acc[i][j], d.round_dt);
        if (d.accumulate == 1) {
          int64_t e0 = c0base + gm * d.c0.strides[0] + gn * d.c0.strides[1];
          float prev = (e0 >= d.c0.lo && e0 < d.c0.hi) ? load_elem(d.c0.ptr, e0, d.c0.dtype) : 0.f;
          v = round_to(__fadd_rn(prev, v), d.c.dtype);
        } else if (d.accumulate == 2) {
          v = round_to(__fadd_rn(0.f, v), d.c.dtype);
        }
        int64_t e = cbase + gm * d.c.strides[0] + gn * d.c.strides[1];
        if (e >= d.c.lo && e < d.c.hi) store_elem(d.c.ptr, e, d.c.dtype, v);
      }
    }
  }
}

}  // namespace ktir

using namespace ktir;

int ktir_launch_matmul_mfma(const ktir_mm_t* d, bool* handled);

extern "C" int ktir_launch_matmul(const ktir_mm_t* d) {
  if (!d || d->M < 0 || d->N < 0 || d->K < 0 || d->ksteps < 1) return set_error(KTIR_E_ARG, "ktir_launch_matmul: bad descriptor");
  if (d->lanes == 0 || d->M == 0 || d->N == 0) return KTIR_OK;
  bool handled = false;
  int rc = ktir_launch_matmul_mfma(d, &handled);
  if (rc != KTIR_OK || handled) return rc;
  int64_t work = d->lanes * ((d->M + GT - 1) / GT) * ((d->N + GT - 1) / GT);
  unsigned blocks = (unsigned)(work < 65536 ? work : 65536);
  hipLaunchKernelGGL(mm_generic, dim3(blocks), dim3(256), 0, stream(), *d);
  KTIR_HIP_CHECK(hipGetLastError());
  return KTIR_OK;
}
