// Paged attention: the online-softmax KV loop of the reference's unified
// attention example (examples/triton-ktir/paged_attention.mlir:194-392) as
// one launch.  Every iteration of the reference's loop reads one page of
// the K and V caches through the block table (an indirect access tile),
// computes S = scale * Q K^T over the page, masks key positions past each
// query row's position, and updates the row max m, row sum l and the f32
// accumulator; the reference runs each of those ops per core and iteration
// (dialects/linalg_ops.py:307-596, dialects/math_ops.py).
//
// One workgroup per lane (simulated core): Q (M x D, as f32) stays in LDS
// for the whole loop; per page the K and V tiles (N x D) are read once into
// LDS, S (M x N) is computed from LDS, each row's statistics by one thread,
// and the accumulator (M x D, at most 32 elements per thread) stays in
// registers.  Arithmetic is f32 in the order of the loop body: s = scale *
// (q . k), m' = max(m, max_c s), p = exp(s - m'), alpha = exp(m - m'),
// acc' = acc * alpha + p . v, l' = l * alpha + sum_c p.
#include <climits>
#include "ktir_common.h"

namespace ktir {

constexpr int PA_THREADS = 256;
constexpr int PA_ACC = 32;                 // accumulator elements per thread (M * D <= 8192)
constexpr int64_t PA_MAX_LDS = 160 * 1024;

__device__ __forceinline__ float max_nan(float a, float b) {
  // arith.maximumf: NaN if either operand is NaN (np.maximum)
  return (a != a || b != b) ? __int_as_float(0x7fc00000) : fmaxf(a, b);
}

__device__ __forceinline__ bool keep_pos(int p, int64_t k, int64_t q) {
  // the reference compares Python ints: unsigned predicates compare values
  switch (p) {
    case KTIR_CMP_EQ: return k == q;
    case KTIR_CMP_NE: return k != q;
    case KTIR_CMP_SLT: case KTIR_CMP_ULTI: return k < q;
    case KTIR_CMP_SLE: case KTIR_CMP_ULEI: return k <= q;
    case KTIR_CMP_SGT: case KTIR_CMP_UGTI: return k > q;
    case KTIR_CMP_SGE: case KTIR_CMP_UGEI: return k >= q;
  }
  return false;
}

__device__ __forceinline__ int64_t load_index(uint64_t ptr, int64_t e, int dt) {
  switch (dt) {
    case KTIR_I64: return ((const int64_t*)ptr)[e];
    case KTIR_I16: return ((const int16_t*)ptr)[e];
    case KTIR_I8: return ((const int8_t*)ptr)[e];
  }
  return ((const int32_t*)ptr)[e];
}

static int64_t pa_lds_floats(int64_t M, int64_t N, int64_t D) {
  return M * (D + 1) + N * (D + 1) + N * D + M * N + 3 * M;
}

__global__ __launch_bounds__(PA_THREADS) void pattn_kernel(const ktir_pattn_t d, int* err) {
  extern __shared__ float sm[];
  const int M = (int)d.M, N = (int)d.N, D = (int)d.D, DP = D + 1;
  float* Qs = sm;                  // [M][D + 1]
  float* Ks = Qs + M * DP;         // [N][D + 1]
  float* Vs = Ks + N * DP;         // [N][D]
  float* S = Vs + N * D;           // [M][N]
  float* mrow = S + M * N;         // [M]
  float* lrow = mrow + M;          // [M]
  float* arow = lrow + M;          // [M] alpha of the current page
  const int64_t lane = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t qb = ((const int64_t*)d.q_base)[lane];
  for (int i = tid; i < M * D; i += PA_THREADS) {
    const int r = i / D, c = i - r * D;
    const int64_t e = qb + (int64_t)r * d.q_row + c;
    Qs[r * DP + c] = (e >= d.q_lo && e < d.q_hi) ? load_elem(d.q_ptr, e, d.q_dtype) : 0.f;
  }
  for (int r = tid; r < M; r += PA_THREADS) {
    mrow[r] = d.m0;
    lrow[r] = d.l0;
  }
  float acc[PA_ACC];
#pragma unroll
  for (int k = 0; k < PA_ACC; ++k) acc[k] = 0.f;
  const int trips = ((const int32_t*)d.trips)[lane];
  const int64_t kb = ((const int64_t*)d.k_base)[lane], vb = ((const int64_t*)d.v_base)[lane];
  const int64_t tp = ((const int64_t*)d.tbl_pos)[lane];
  const int64_t qp0 = ((const int64_t*)d.qpos0)[lane], kp0 = ((const int64_t*)d.kpos0)[lane];
  __syncthreads();
  for (int j = 0; j < trips; ++j) {
    // the page of this iteration: an index read outside the table's
    // allocation reads 0, a negative index raises (after the launch)
    const int64_t te = tp + (int64_t)j * d.tbl_step;
    int64_t page = (te >= d.tbl_lo && te < d.tbl_hi) ? load_index(d.tbl_ptr, te, d.tbl_dtype) : 0;
    if (page < 0) {
      if (tid == 0) *err = 1;
      page = 0;
    }
    const int64_t k0 = kb + page * d.k_page, v0 = vb + page * d.v_page;
    for (int i = tid; i < N * D; i += PA_THREADS) {
      const int c = i / D, x = i - c * D;
      const int64_t ek = k0 + (int64_t)c * d.k_row + x, ev = v0 + (int64_t)c * d.v_row + x;
      Ks[c * DP + x] = (ek >= d.k_lo && ek < d.k_hi) ? load_elem(d.k_ptr, ek, d.kv_dtype) : 0.f;
      Vs[c * D + x] = (ev >= d.v_lo && ev < d.v_hi) ? load_elem(d.v_ptr, ev, d.kv_dtype) : 0.f;
    }
    __syncthreads();
    for (int i = tid; i < M * N; i += PA_THREADS) {
      const int r = i / N, c = i - r * N;
      const float* q = Qs + r * DP;
      const float* k = Ks + c * DP;
      float s = 0.f;
      for (int x = 0; x < D; ++x) s = __fmaf_rn(q[x], k[x], s);
      s = __fmul_rn(d.scale, s);
      if (d.causal) {
        const int64_t kpos = kp0 + (int64_t)j * d.kpos_step + c;
        const int64_t qpos = qp0 + r / d.row_div;
        if (!keep_pos(d.pred, kpos, qpos)) s = d.neg;
      }
      S[i] = s;
    }
    __syncthreads();
    for (int r = tid; r < M; r += PA_THREADS) {
      float* sr = S + r * N;
      float mx = -INFINITY;
      for (int c = 0; c < N; ++c) mx = max_nan(mx, sr[c]);
      const float mo = mrow[r];
      const float mn = max_nan(mo, mx);
      float sum = 0.f;
      for (int c = 0; c < N; ++c) {
        const float p = expf(__fsub_rn(sr[c], mn));
        sr[c] = p;
        sum = __fadd_rn(sum, p);
      }
      const float al = expf(__fsub_rn(mo, mn));
      arow[r] = al;
      lrow[r] = __fadd_rn(__fmul_rn(lrow[r], al), sum);
      mrow[r] = mn;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PA_ACC; ++k) {
      const int i = tid + k * PA_THREADS;
      if (i < M * D) {
        const int r = i / D, x = i - r * D;
        const float* p = S + r * N;
        float pv = 0.f;
        for (int c = 0; c < N; ++c) pv = __fmaf_rn(p[c], Vs[c * D + x], pv);
        acc[k] = __fadd_rn(__fmul_rn(acc[k], arow[r]), pv);
      }
    }
    __syncthreads();
  }
  for (int r = tid; r < M; r += PA_THREADS) {
    ((float*)d.m_out)[lane * M + r] = mrow[r];
    ((float*)d.l_out)[lane * M + r] = lrow[r];
  }
#pragma unroll
  for (int k = 0; k < PA_ACC; ++k) {
    const int i = tid + k * PA_THREADS;
    if (i < M * D) ((float*)d.acc_out)[lane * M * D + i] = acc[k];
  }
}

}  // namespace ktir

using namespace ktir;

extern "C" int ktir_launch_paged_attention(const ktir_pattn_t* d) {
  if (!d) return set_error(KTIR_E_ARG, "ktir_launch_paged_attention: null descriptor");
  if (d->M < 1 || d->N < 1 || d->D < 1 || d->M * d->D > (int64_t)PA_THREADS * PA_ACC || d->row_div < 1)
    return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_paged_attention: M=%lld N=%lld D=%lld row_div=%lld",
                     (long long)d->M, (long long)d->N, (long long)d->D, (long long)d->row_div);
  const int64_t lds = pa_lds_floats(d->M, d->N, d->D) * (int64_t)sizeof(float);
  if (lds > PA_MAX_LDS)
    return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_paged_attention: %lld bytes of LDS", (long long)lds);
  const int dts[2] = {d->q_dtype, d->kv_dtype};
  for (int dt : dts)
    if (dt != KTIR_F16 && dt != KTIR_BF16 && dt != KTIR_F32)
      return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_paged_attention: operand dtype %d", dt);
  if (d->tbl_dtype != KTIR_I32 && d->tbl_dtype != KTIR_I64 && d->tbl_dtype != KTIR_I16 && d->tbl_dtype != KTIR_I8)
    return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_paged_attention: index dtype %d", d->tbl_dtype);
  if (d->causal) {
    switch (d->pred) {
      case KTIR_CMP_EQ: case KTIR_CMP_NE: case KTIR_CMP_SLT: case KTIR_CMP_ULTI: case KTIR_CMP_SLE:
      case KTIR_CMP_ULEI: case KTIR_CMP_SGT: case KTIR_CMP_UGTI: case KTIR_CMP_SGE: case KTIR_CMP_UGEI: break;
      default: return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_paged_attention: mask predicate %d", d->pred);
    }
  }
  if (d->lanes == 0) return KTIR_OK;
  if (d->lanes > INT_MAX) return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_paged_attention: too many lanes");
  if (lds > 64 * 1024)
    KTIR_HIP_CHECK(hipFuncSetAttribute((const void*)pattn_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds));
  hipLaunchKernelGGL(pattn_kernel, dim3((unsigned)d->lanes), dim3(PA_THREADS), (size_t)lds, stream(), *d,
                     device_error_flag());
  KTIR_HIP_CHECK(hipGetLastError());
  return KTIR_OK;
}
