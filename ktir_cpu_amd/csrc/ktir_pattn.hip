// Paged attention: the online-softmax KV loop of the reference's unified
// attention example (examples/triton-ktir/paged_attention.mlir:194-392) as
// one launch.  Every iteration of the reference's loop reads one page of
// the K and V caches through the block table (an indirect access tile),
// computes S = scale * Q K^T over the page, masks key positions past each
// query row's position, and updates the row max m, row sum l and the f32
// accumulator; the reference runs each of those ops per core and iteration
// (dialects/linalg_ops.py:307-596, dialects/math_ops.py).
//
// One workgroup per lane (simulated core; the host orders workgroups so
// that the lanes reading one KV head's pages share an XCD and its L2):
// Q (M x D, as f32) stays in LDS
// for the whole loop; the next page's K and V tiles (N x D) are read into
// registers (16-byte loads) while the current page is computed, then
// written to LDS as f32; S (M x N) is computed from LDS by groups of lanes
// per (row, key) combined with shuffles, a row's statistics by N lanes with
// shuffles (or one thread per row), and the accumulator (M x D, at most 32
// elements per thread) stays in registers.  Arithmetic is f32 in the order of the loop body: s = scale *
// (q . k), m' = max(m, max_c s), p = exp(s - m'), alpha = exp(m - m'),
// acc' = acc * alpha + p . v, l' = l * alpha + sum_c p.
#include <climits>
#include "ktir_common.h"

namespace ktir {

constexpr int PA_THREADS = 256;
constexpr int PA_ACC = 32;                 // largest accumulator per thread (M * D <= 8192)
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

// Q and K rows are padded to D + 8 floats: 16-byte aligned rows for vector
// LDS reads, consecutive rows two 16-byte bank groups apart
static int64_t pa_lds_floats(int64_t M, int64_t N, int64_t D) {
  return M * (D + 8) + N * (D + 8) + N * D + M * N + 3 * M;
}

constexpr int PA_PF = 4;                   // largest prefetch: 8-element vectors per thread and tensor (N * D <= 8192)

// Prefetch of one page of K and V into registers: the vectorised form
// (flag `vec`: 16-bit elements, rows of whole 16-byte aligned 8-element
// vectors) issues 16-byte loads; a vector not wholly inside its allocation
// window, and the unaligned form, read element by element when the page is
// written to LDS.
template <int PF>
struct PagePf {
  uint4 k[PF], v[PF];
  int64_t k0, v0;
};

// sum over the 4-element groups g = p, p + TP, ... of q . k (16-byte aligned rows)
__device__ __forceinline__ float dot4(const float* q, const float* k, int p, int TP, int D) {
  const float4* q4 = (const float4*)q;
  const float4* k4 = (const float4*)k;
  float s0 = 0.f, s1 = 0.f;
#pragma unroll 4
  for (int g = p; g < D / 4; g += TP) {
    const float4 a = q4[g], b = k4[g];
    s0 = __fmaf_rn(a.x, b.x, s0);
    s1 = __fmaf_rn(a.y, b.y, s1);
    s0 = __fmaf_rn(a.z, b.z, s0);
    s1 = __fmaf_rn(a.w, b.w, s1);
  }
  return s0 + s1;
}

__device__ __forceinline__ int64_t page_of(const ktir_pattn_t& d, int64_t tp, int j, int* err, bool lead) {
  const int64_t te = tp + (int64_t)j * d.tbl_step;
  int64_t page = (te >= d.tbl_lo && te < d.tbl_hi) ? load_index(d.tbl_ptr, te, d.tbl_dtype) : 0;
  if (page < 0) {
    if (lead) *err = 1;
    page = 0;
  }
  return page;
}

__device__ __forceinline__ void unpack8(uint4 w, int dt, float* o) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (dt == KTIR_BF16) {
      o[2 * i] = __uint_as_float(u[i] << 16);
      o[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
    } else {
      o[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[i] & 0xffffu));
      o[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[i] >> 16));
    }
  }
}

template <int ACC, int PF>
__global__ __launch_bounds__(PA_THREADS) void pattn_kernel(const ktir_pattn_t d, int vec, int* err) {
  extern __shared__ float sm[];
  const int M = (int)d.M, N = (int)d.N, D = (int)d.D, DP = D + 8;
  float* Qs = sm;                  // [M][D + 8]
  float* Ks = Qs + M * DP;         // [N][D + 8]
  float* Vs = Ks + N * DP;         // [N][D]
  float* S = Vs + N * D;           // [M][N]
  float* mrow = S + M * N;         // [M]
  float* lrow = mrow + M;          // [M]
  float* arow = lrow + M;          // [M] alpha of the current page
  const int64_t lane = d.order ? ((const int32_t*)d.order)[blockIdx.x] : blockIdx.x;
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
  float acc[ACC];
#pragma unroll
  for (int k = 0; k < ACC; ++k) acc[k] = 0.f;
  const int trips = ((const int32_t*)d.trips)[lane];
  const int64_t kb = ((const int64_t*)d.k_base)[lane], vb = ((const int64_t*)d.v_base)[lane];
  const int64_t tp = ((const int64_t*)d.tbl_pos)[lane];
  const int64_t qp0 = ((const int64_t*)d.qpos0)[lane], kp0 = ((const int64_t*)d.kpos0)[lane];
  const int nvec = N * D / 8;      // 8-element vectors of one page tile (vectorised form)
  vec = vec && !(kb & 7) && !(vb & 7);   // this lane's tiles start on 16-byte boundaries
  // S = Q K^T: TP threads per (row, key) pair, each the 4-element groups
  // p, p + TP, ... of the dot product (16-byte LDS reads), combined by lane
  // shuffles (TP a power of two <= 64)
  int TP = PA_THREADS / (M * N);
  if (TP < 1) TP = 1;
  while (TP > 1 && (D % (4 * TP) || (TP & (TP - 1)))) TP >>= 1;
  // row statistics by N lanes per row when N is a power of two <= 64 and
  // the rows fit the workgroup at once; otherwise one thread per row
  const bool rows_par = (N & (N - 1)) == 0 && N <= 64 && M * N <= PA_THREADS;
  // S and the row statistics in one pass when every row's lanes lie in one
  // wavefront and all pairs fit the workgroup
  const bool fused = rows_par && N * TP <= 64 && M * N * TP <= PA_THREADS;
  PagePf<PF> pf;
  auto prefetch = [&](int j) {
    const int64_t page = page_of(d, tp, j, err, tid == 0);
    pf.k0 = kb + page * d.k_page;
    pf.v0 = vb + page * d.v_page;
    if (vec) {
#pragma unroll
      for (int u = 0; u < PF; ++u) {
        const int i = tid + u * PA_THREADS;
        if (i < nvec) {
          const int c = (i * 8) / D, x = i * 8 - c * D;
          const int64_t ek = pf.k0 + (int64_t)c * d.k_row + x, ev = pf.v0 + (int64_t)c * d.v_row + x;
          if (ek >= d.k_lo && ek + 8 <= d.k_hi) pf.k[u] = *(const uint4*)((const uint16_t*)d.k_ptr + ek);
          if (ev >= d.v_lo && ev + 8 <= d.v_hi) pf.v[u] = *(const uint4*)((const uint16_t*)d.v_ptr + ev);
        }
      }
    }
  };
  auto commit = [&]() {
    if (vec) {
#pragma unroll
      for (int u = 0; u < PF; ++u) {
        const int i = tid + u * PA_THREADS;
        if (i < nvec) {
          const int c = (i * 8) / D, x = i * 8 - c * D;
          const int64_t ek = pf.k0 + (int64_t)c * d.k_row + x, ev = pf.v0 + (int64_t)c * d.v_row + x;
          float kv[8], vv[8];
          if (ek >= d.k_lo && ek + 8 <= d.k_hi) {
            unpack8(pf.k[u], d.kv_dtype, kv);
          } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) kv[t] = (ek + t >= d.k_lo && ek + t < d.k_hi) ? load_elem(d.k_ptr, ek + t, d.kv_dtype) : 0.f;
          }
          if (ev >= d.v_lo && ev + 8 <= d.v_hi) {
            unpack8(pf.v[u], d.kv_dtype, vv);
          } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) vv[t] = (ev + t >= d.v_lo && ev + t < d.v_hi) ? load_elem(d.v_ptr, ev + t, d.kv_dtype) : 0.f;
          }
          float4* kd = (float4*)(Ks + c * DP + x);
          float4* vd = (float4*)(Vs + c * D + x);
          kd[0] = make_float4(kv[0], kv[1], kv[2], kv[3]);
          kd[1] = make_float4(kv[4], kv[5], kv[6], kv[7]);
          vd[0] = make_float4(vv[0], vv[1], vv[2], vv[3]);
          vd[1] = make_float4(vv[4], vv[5], vv[6], vv[7]);
        }
      }
    } else {
      for (int i = tid; i < N * D; i += PA_THREADS) {
        const int c = i / D, x = i - c * D;
        const int64_t ek = pf.k0 + (int64_t)c * d.k_row + x, ev = pf.v0 + (int64_t)c * d.v_row + x;
        Ks[c * DP + x] = (ek >= d.k_lo && ek < d.k_hi) ? load_elem(d.k_ptr, ek, d.kv_dtype) : 0.f;
        Vs[c * D + x] = (ev >= d.v_lo && ev < d.v_hi) ? load_elem(d.v_ptr, ev, d.kv_dtype) : 0.f;
      }
    }
  };
  if (trips > 0) prefetch(0);
  __syncthreads();
  for (int j = 0; j < trips; ++j) {
    commit();
    if (j + 1 < trips) prefetch(j + 1);    // next page's loads in flight during this page's compute
    __syncthreads();
    if (fused) {
      // one pass: lane group (pair, part) computes its part of s[r][c]; the
      // TP lanes of a pair sum by shuffles (each then holds s), the N pairs
      // of a row (N * TP consecutive lanes of one wavefront) take the row
      // max and the row sum by shuffles, counting each pair once
      const int pair = tid / TP, part = tid - pair * TP;
      const bool live = pair < M * N;
      const int r = live ? pair / N : 0, c = pair - r * N;
      float s = 0.f;
      if (live) {
        const float* q = Qs + r * DP;
        const float* k = Ks + c * DP;
        s = dot4(q, k, part, TP, D);
      }
      for (int o = 1; o < TP; o <<= 1) s += __shfl_xor(s, o);
      s = __fmul_rn(d.scale, s);
      if (d.causal) {
        const int64_t kpos = kp0 + (int64_t)j * d.kpos_step + c;
        const int64_t qpos = qp0 + r / d.row_div;
        if (!keep_pos(d.pred, kpos, qpos)) s = d.neg;
      }
      if (!live) s = -INFINITY;
      float mx = s;
      for (int o = TP; o < N * TP; o <<= 1) mx = max_nan(mx, __shfl_xor(mx, o));
      const float mo = live ? mrow[r] : 0.f;
      const float mn = max_nan(mo, mx);
      const float p = expf(__fsub_rn(s, mn));
      float sum = part == 0 ? p : 0.f;
      for (int o = 1; o < N * TP; o <<= 1) sum += __shfl_xor(sum, o);
      if (live && part == 0) S[pair] = p;
      if (live && part == 0 && c == 0) {
        const float al = expf(__fsub_rn(mo, mn));
        arow[r] = al;
        lrow[r] = __fadd_rn(__fmul_rn(lrow[r], al), sum);
        mrow[r] = mn;
      }
    } else {
    for (int base = 0; base < M * N * TP; base += PA_THREADS) {
      const int g = base + tid;
      const int pair = g / TP, part = g - pair * TP;
      float s = 0.f;
      if (pair < M * N) {
        const int r = pair / N, c = pair - r * N;
        const float* q = Qs + r * DP;
        const float* k = Ks + c * DP;
        s = dot4(q, k, part, TP, D);
      }
      for (int o = 1; o < TP; o <<= 1) s += __shfl_xor(s, o);
      if (pair < M * N && part == 0) {
        const int r = pair / N, c = pair - r * N;
        s = __fmul_rn(d.scale, s);
        if (d.causal) {
          const int64_t kpos = kp0 + (int64_t)j * d.kpos_step + c;
          const int64_t qpos = qp0 + r / d.row_div;
          if (!keep_pos(d.pred, kpos, qpos)) s = d.neg;
        }
        S[pair] = s;
      }
    }
    __syncthreads();
    if (rows_par) {
      const int r = tid / N, c = tid - r * N;
      const bool live = tid < M * N;
      const float sv = live ? S[tid] : -INFINITY;
      float mx = sv;
      for (int o = 1; o < N; o <<= 1) mx = max_nan(mx, __shfl_xor(mx, o));
      const float mo = live ? mrow[r] : 0.f;
      const float mn = max_nan(mo, mx);
      const float p = expf(__fsub_rn(sv, mn));
      float sum = p;
      for (int o = 1; o < N; o <<= 1) sum += __shfl_xor(sum, o);
      if (live) S[tid] = p;
      if (live && c == 0) {
        const float al = expf(__fsub_rn(mo, mn));
        arow[r] = al;
        lrow[r] = __fadd_rn(__fmul_rn(lrow[r], al), sum);
        mrow[r] = mn;
      }
    } else {
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
    }
    }
    __syncthreads();
    // the accumulator: group g = tid + k * 256 holds the 4 consecutive
    // elements 4g .. 4g + 3 of the row-major M x D block
#pragma unroll
    for (int k = 0; k < ACC / 4; ++k) {
      const int i = 4 * (tid + k * PA_THREADS);
      if (i < M * D) {
        const int r = i / D, x = i - r * D;
        const float* p = S + r * N;
        const float4* v4 = (const float4*)(Vs + x);
        float4 pv = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
        for (int c = 0; c < N; ++c) {
          const float pc = p[c];
          const float4 v = v4[c * (D / 4)];
          pv.x = __fmaf_rn(pc, v.x, pv.x);
          pv.y = __fmaf_rn(pc, v.y, pv.y);
          pv.z = __fmaf_rn(pc, v.z, pv.z);
          pv.w = __fmaf_rn(pc, v.w, pv.w);
        }
        const float al = arow[r];
        acc[4 * k] = __fadd_rn(__fmul_rn(acc[4 * k], al), pv.x);
        acc[4 * k + 1] = __fadd_rn(__fmul_rn(acc[4 * k + 1], al), pv.y);
        acc[4 * k + 2] = __fadd_rn(__fmul_rn(acc[4 * k + 2], al), pv.z);
        acc[4 * k + 3] = __fadd_rn(__fmul_rn(acc[4 * k + 3], al), pv.w);
      }
    }
    __syncthreads();
  }
  for (int r = tid; r < M; r += PA_THREADS) {
    ((float*)d.m_out)[lane * M + r] = mrow[r];
    ((float*)d.l_out)[lane * M + r] = lrow[r];
  }
#pragma unroll
  for (int k = 0; k < ACC / 4; ++k) {
    const int i = 4 * (tid + k * PA_THREADS);
    if (i < M * D)
      *(float4*)((float*)d.acc_out + lane * M * D + i) = make_float4(acc[4 * k], acc[4 * k + 1], acc[4 * k + 2], acc[4 * k + 3]);
  }
}

}  // namespace ktir

using namespace ktir;

extern "C" int ktir_launch_paged_attention(const ktir_pattn_t* d) {
  if (!d) return set_error(KTIR_E_ARG, "ktir_launch_paged_attention: null descriptor");
  if (d->M < 1 || d->N < 1 || d->D < 4 || d->D % 4 || d->M * d->D > (int64_t)PA_THREADS * PA_ACC || d->row_div < 1)
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
  // the vectorised page reads: 16-bit K / V, rows of whole 8-element
  // vectors, every row start a multiple of 8 elements, pointers 16-byte aligned
  int vec = (d->kv_dtype == KTIR_F16 || d->kv_dtype == KTIR_BF16) && d->D % 8 == 0 && d->N * d->D <= 8 * PA_THREADS * PA_PF
            && !((d->k_ptr | d->v_ptr) & 15) && !((d->k_row | d->v_row | d->k_page | d->v_page) & 7);
  const int64_t per = (d->M * d->D + PA_THREADS - 1) / PA_THREADS;
  const int64_t pfv = (d->N * d->D / 8 + PA_THREADS - 1) / PA_THREADS;
  auto go = [&](auto kern) -> int {
    if (lds > 64 * 1024)
      KTIR_HIP_CHECK(hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL(kern, dim3((unsigned)d->lanes), dim3(PA_THREADS), (size_t)lds, stream(), *d, vec,
                       device_error_flag());
    return 0;
  };
  // accumulator and prefetch sized to the tile: fewer VGPRs, more
  // workgroups per CU
  if (per <= 4 && pfv <= 1) go(pattn_kernel<4, 1>);
  else if (per <= 4 && pfv <= 2) go(pattn_kernel<4, 2>);
  else if (per <= 4) go(pattn_kernel<4, 4>);
  else if (per <= 8 && pfv <= 2) go(pattn_kernel<8, 2>);
  else if (per <= 8) go(pattn_kernel<8, 4>);
  else if (per <= 16) go(pattn_kernel<16, 4>);
  else go(pattn_kernel<32, 4>);
  KTIR_HIP_CHECK(hipGetLastError());
  return KTIR_OK;
}
