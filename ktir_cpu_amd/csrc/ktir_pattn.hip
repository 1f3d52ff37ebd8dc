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
    case KTIR_I64: return ((const KTIR_G(int64_t)*)ptr)[e];
    case KTIR_I16: return ((const KTIR_G(int16_t)*)ptr)[e];
    case KTIR_I8: return ((const KTIR_G(int8_t)*)ptr)[e];
  }
  return ((const KTIR_G(int32_t)*)ptr)[e];
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
  if (d.out_ptr) {
    // the loop's finalisation: acc / l rounded to the output's dtype
    const int64_t obase = ((const int64_t*)d.out_base)[lane];
#pragma unroll
    for (int k = 0; k < ACC / 4; ++k) {
      const int i = 4 * (tid + k * PA_THREADS);
      if (i < M * D) {
        const int r = i / D, x = i - r * D;
        const int64_t ob = obase + (int64_t)(r / d.out_grp) * d.out_gstride + (int64_t)(r % d.out_grp) * d.out_row + x;
#pragma unroll
        for (int u = 0; u < 4; ++u)
          if (ob + u >= d.out_lo && ob + u < d.out_hi) store_elem(d.out_ptr, ob + u, d.out_dtype, __fdiv_rn(acc[4 * k + u], lrow[r]));
      }
    }
  }
}

// ---- MFMA form ---------------------------------------------------------------
// The example's shape (pages of 16 keys, at most 16 query rows per lane, D a
// multiple of 32 up to 256, Q, K and V all f16 or all bf16) runs one
// wavefront per lane on the matrix cores, with no LDS and no barriers.  Per
// page, with lane l = 16 g + n (n = l % 16, g = l / 16):
//   S^T = K Q^T    D/32 v_mfma_f32_16x16x32: A = K (lane l: key n, the 8
//                  elements d = 32 t + 8 g ..), B = Q^T (lane l: query row
//                  n, the same d), so lane l ends up with s[row n][key 4 g + i],
//                  i < 4 (the 16 x 16 result layout: lane 16 g + n holds
//                  rows 4 g .. 4 g + 3 of column n);
//   row max / sum  the lane's 4 values, then lanes l ^ 16 and l ^ 32
//                  (v_permlane16_swap / v_permlane32_swap);
//   O^T += V^T P^T D/16 tiles of v_mfma_f32_16x16x16 with B = P^T (lane l:
//                  row n, keys 4 g + j: the lane's own S^T values after the
//                  softmax) and A = V^T whose columns interleave: tile t,
//                  lane n takes column (D/16) n + t, so a lane reads one
//                  contiguous (D/16)-element piece of each of its 4 key rows.
// O^T's result layout puts row n's columns (D/16)(4 g + i) + t in lane l,
// so alpha, m and l of a lane's rows are its own.  Products of 16-bit
// operands are exact in f32 and summed in f32; P enters P V as hi + lo in
// the operand type (about 16 significant bits instead of 11 / 8).  The
// page's K and V for page j + 1 are in flight (registers) while page j is
// computed, and the block table entry of page j + 2.
typedef _Float16 pa_h8 __attribute__((ext_vector_type(8)));
typedef __bf16 pa_b8 __attribute__((ext_vector_type(8)));
typedef _Float16 pa_h4 __attribute__((ext_vector_type(4)));
typedef short pa_s4 __attribute__((ext_vector_type(4)));
typedef float pa_f4 __attribute__((ext_vector_type(4)));
typedef float pa_f2 __attribute__((ext_vector_type(2)));
typedef _Float16 pa_h2 __attribute__((ext_vector_type(2)));
typedef __bf16 pa_b2 __attribute__((ext_vector_type(2)));
typedef uint32_t pa_u2 __attribute__((ext_vector_type(2)));
typedef uint32_t pa_u4 __attribute__((ext_vector_type(4)));

template <bool BF16>
__device__ __forceinline__ pa_f4 mfma_k32(const uint4& a, const uint4& b, pa_f4 c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(pa_b8, a), __builtin_bit_cast(pa_b8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(pa_h8, a), __builtin_bit_cast(pa_h8, b), c, 0, 0, 0);
}

template <bool BF16>
__device__ __forceinline__ pa_f4 mfma_k16(const uint2& a, const uint2& b, pa_f4 c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(pa_s4, a), __builtin_bit_cast(pa_s4, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(pa_h4, a), __builtin_bit_cast(pa_h4, b), c, 0, 0, 0);
}

// (a, b) rounded to nearest-even in the operand type, a in the low half
template <bool BF16>
__device__ __forceinline__ uint32_t pa_cvt2(float a, float b) {
  const pa_f2 v = {a, b};
  if constexpr (BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, pa_b2));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, pa_h2));
}

template <bool BF16>
__device__ __forceinline__ pa_f2 pa_uncvt2(uint32_t w) {
  if constexpr (BF16) return pa_f2{__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u)};
  else return __builtin_convertvector(__builtin_bit_cast(pa_h2, w), pa_f2);
}

// x of lanes l and l ^ 16 (v_permlane16_swap) / l and l ^ 32
// (v_permlane32_swap) as (lower lane's, upper lane's): the same pair, in the
// same order, in both lanes
__device__ __forceinline__ pa_f2 pair16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return pa_f2{__uint_as_float(r[0]), __uint_as_float(r[1])};
}
__device__ __forceinline__ pa_f2 pair32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return pa_f2{__uint_as_float(r[0]), __uint_as_float(r[1])};
}

// arith.maximumf over a row: NaN-propagating (v_maximum_f32)
__device__ __forceinline__ float pa_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// NW words (2 NW consecutive 16-bit elements) from element e: one vector
// load when `fast` (the caller has checked alignment and window), else
// element by element with zeros outside [lo, hi)
template <int NW>
__device__ __forceinline__ void pa_words(const KTIR_G(uint16_t) * p, int64_t e, bool fast, int64_t lo, int64_t hi,
                                         uint32_t* w) {
  if (fast) {
    if constexpr (NW == 1) {
      w[0] = *(const KTIR_G(uint32_t)*)(p + e);
    } else if constexpr (NW == 2) {
      const uint2 x = __builtin_bit_cast(uint2, *(const KTIR_G(pa_u2)*)(p + e));
      w[0] = x.x; w[1] = x.y;
    } else {
#pragma unroll
      for (int q = 0; q < NW / 4; ++q) {
        const pa_u4 x = *(const KTIR_G(pa_u4)*)(p + e + 8 * q);
        w[4 * q] = x[0]; w[4 * q + 1] = x[1]; w[4 * q + 2] = x[2]; w[4 * q + 3] = x[3];
      }
    }
    return;
  }
#pragma unroll
  for (int q = 0; q < NW; ++q) {
    const int64_t x = e + 2 * q;
    const uint32_t a = (x >= lo && x < hi) ? p[x] : 0u, b = (x + 1 >= lo && x + 1 < hi) ? p[x + 1] : 0u;
    w[q] = a | (b << 16);
  }
}

// one page's operands in registers: K chunks (lane l: key n, d = 32 t + 8 g
// .. + 8) and V pieces (key 4 g + j, columns (D/16) n .. + D/16: words
// 0 .. DT - 1 of v[j], 16 bytes per vector), kept in the vector types the
// loads return and the MFMAs read, so no register copies sit between them
template <int DT>
struct PaOps {
  pa_u4 k[DT];
  pa_u4 v[4][(DT + 3) / 4];
};

// word q (< DT) of V piece j
template <int DT>
__device__ __forceinline__ uint32_t pa_vword(const PaOps<DT>& o, int j, int q) {
  return o.v[j][q >> 2][q & 3];
}

// The page's K and V in their windows with 16-byte aligned rows: every
// piece is one vector load (the grouped loop runs only on such pages)
template <int DT>
__device__ __forceinline__ bool pa_fast(const ktir_pattn_t& d, int64_t k0, int64_t v0) {
  constexpr int D = 32 * DT;
  return !(k0 & 7) && !(v0 & 7) && k0 >= d.k_lo && k0 + 15 * d.k_row + D <= d.k_hi && v0 >= d.v_lo &&
         v0 + 15 * d.v_row + D <= d.v_hi;
}

// lane offsets (elements, from the page's first element) of its K chunks
// and V pieces; 32-bit: a page spans 16 rows
struct PaLaneOffs {
  uint32_t k, v[4];
};

// a fast page: uniform bases, 32-bit lane offsets, one vector load per piece
template <int DT>
__device__ __forceinline__ void pa_load_fast(const ktir_pattn_t& d, int64_t k0, int64_t v0, const PaLaneOffs& lo,
                                             PaOps<DT>& o) {
  const KTIR_G(uint16_t)* K = (const KTIR_G(uint16_t)*)d.k_ptr + k0;
  const KTIR_G(uint16_t)* V = (const KTIR_G(uint16_t)*)d.v_ptr + v0;
#pragma unroll
  for (int t = 0; t < DT; ++t) o.k[t] = *(const KTIR_G(pa_u4)*)(K + lo.k + 32 * t);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if constexpr (DT >= 4) {
#pragma unroll
      for (int q = 0; q < DT / 4; ++q) o.v[j][q] = *(const KTIR_G(pa_u4)*)(V + lo.v[j] + 8 * q);
    } else if constexpr (DT == 2) {
      const pa_u2 x = *(const KTIR_G(pa_u2)*)(V + lo.v[j]);
      o.v[j][0] = pa_u4{x[0], x[1], 0u, 0u};
    } else {
      o.v[j][0] = pa_u4{*(const KTIR_G(uint32_t)*)(V + lo.v[j]), 0u, 0u, 0u};
    }
  }
}

// any page: element loads, zeros outside the windows
template <int DT>
__device__ __forceinline__ void pa_load_any(const ktir_pattn_t& d, int64_t k0, int64_t v0, const PaLaneOffs& lo,
                                            PaOps<DT>& o) {
  const KTIR_G(uint16_t)* K = (const KTIR_G(uint16_t)*)d.k_ptr;
  const KTIR_G(uint16_t)* V = (const KTIR_G(uint16_t)*)d.v_ptr;
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    uint32_t w[4];
    pa_words<4>(K, k0 + lo.k + 32 * t, false, d.k_lo, d.k_hi, w);
    o.k[t] = pa_u4{w[0], w[1], w[2], w[3]};
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int q = 0; q < (DT + 3) / 4; ++q) {
      uint32_t w[4] = {0u, 0u, 0u, 0u};
      if constexpr (DT >= 4) pa_words<4>(V, v0 + lo.v[j] + 8 * q, false, d.v_lo, d.v_hi, w);
      else pa_words<DT>(V, v0 + lo.v[j], false, d.v_lo, d.v_hi, w);
      o.v[j][q] = pa_u4{w[0], w[1], w[2], w[3]};
    }
  }
}

// block-table entry of page j (< trips; 0 past the table's window; a
// negative entry reads page 0 and sets `bad`).  The load is unconditional
// (at the window's first entry when j is outside it) and its value is not
// used until pa_fix, so a chunk read ahead does not stall the pages in flight.
struct PaEntry {
  int64_t raw;
  bool in;
};

__device__ __forceinline__ PaEntry pa_entry_raw(const ktir_pattn_t& d, int64_t tp, int j, int trips) {
  if (d.tbl_hi <= d.tbl_lo) return PaEntry{0, false};
  const int64_t te = tp + (int64_t)j * d.tbl_step;
  const bool in = j < trips && te >= d.tbl_lo && te < d.tbl_hi;
  return PaEntry{load_index(d.tbl_ptr, in ? te : d.tbl_lo, d.tbl_dtype), in};
}

__device__ __forceinline__ int64_t pa_fix(const PaEntry& e, bool& bad) {
  const int64_t page = e.in ? e.raw : 0;
  bad |= page < 0;
  return page < 0 ? 0 : page;
}

// value of lane `src` (uniform) of a 64-bit per-lane value
__device__ __forceinline__ int64_t pa_readlane(int64_t v, int src) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, src), hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), src);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// e^x as 2^(x log2 e) on the hardware exp2 (v_exp_f32)
__device__ __forceinline__ float pa_exp(float x) { return __builtin_amdgcn_exp2f(__fmul_rn(x, 1.44269504088896341f)); }

// Pages move in groups of G: the next group's loads are issued, the current
// group's G pages are computed (one online-softmax step each, in order),
// then one wait for the next group.  A page that is not wholly inside its
// window or not 16-byte aligned ends the grouped loop; the lane's
// remaining pages then run one at a time with element loads.
template <bool BF16, int DT, int G>
__global__ __launch_bounds__(64) void pattn_mfma(const ktir_pattn_t d, int vec, int* err) {
  constexpr int D = 32 * DT, NT = 2 * DT;   // NT tiles of 16 columns
  const int l = threadIdx.x, n = l & 15, g = l >> 4;
  const int M = (int)d.M;
  const int64_t lane = d.order ? ((const int32_t*)d.order)[blockIdx.x] : blockIdx.x;
  const int trips = uni(((const int32_t*)d.trips)[lane]);
  const int64_t kb = uni(((const int64_t*)d.k_base)[lane]), vb = uni(((const int64_t*)d.v_base)[lane]);
  const int64_t tp = uni(((const int64_t*)d.tbl_pos)[lane]);
  const int64_t qp0 = uni(((const int64_t*)d.qpos0)[lane]), kp0 = uni(((const int64_t*)d.kpos0)[lane]);
  bool bad = false;
  PaLaneOffs lo;
  lo.k = (uint32_t)(n * d.k_row + 8 * g);
#pragma unroll
  for (int j = 0; j < 4; ++j) lo.v[j] = (uint32_t)((4 * g + j) * d.v_row + 2 * DT * n);
  // the table, 64 entries per register: entry c * 64 + l in lane l of chunk
  // c; chunk c + 1 is read when chunk c comes into use
  int64_t tcur = pa_fix(pa_entry_raw(d, tp, l, trips), bad);
  PaEntry tnext = pa_entry_raw(d, tp, 64 + l, trips);
  // page index of page jl (pages are asked for in increasing order, each once)
  auto page_at = [&](int jl) -> int64_t {
    if (jl > 0 && (jl & 63) == 0) {
      tcur = pa_fix(tnext, bad);
      tnext = pa_entry_raw(d, tp, jl + 64 + l, trips);
    }
    return pa_readlane(tcur, jl & 63);
  };
  // Q^T fragments: row n (zero past the M rows), d = 32 t + 8 g .. + 8
  uint32_t qf[DT][4];
  {
    const int64_t qb = uni(((const int64_t*)d.q_base)[lane]);
    const KTIR_G(uint16_t)* Q = (const KTIR_G(uint16_t)*)d.q_ptr;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const int64_t e = qb + (int64_t)n * d.q_row + 32 * t + 8 * g;
      const bool qv = vec && !(e & 7) && e >= d.q_lo && e + 8 <= d.q_hi;
      pa_words<4>(Q, e, qv, d.q_lo, d.q_hi, qf[t]);
      if (n >= M) qf[t][0] = qf[t][1] = qf[t][2] = qf[t][3] = 0u;
    }
  }
  // the position mask on d0 = kpos(key 4 g) - qpos(row n): key 4 g + i is
  // kept iff (lo - i <= d0 <= hi - i) != inv
  int64_t mlo = INT64_MIN, mhi = INT64_MAX;
  bool inv = false;
  if (d.causal) {
    switch (d.pred) {
      case KTIR_CMP_EQ: mlo = mhi = 0; break;
      case KTIR_CMP_NE: mlo = mhi = 0; inv = true; break;
      case KTIR_CMP_SLT: case KTIR_CMP_ULTI: mhi = -1; break;
      case KTIR_CMP_SLE: case KTIR_CMP_ULEI: mhi = 0; break;
      case KTIR_CMP_SGT: case KTIR_CMP_UGTI: mlo = 1; break;
      default: mlo = 0; break;                 // SGE / UGE (the launcher rejects others)
    }
  }
  int64_t lo_i[4], hi_i[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    lo_i[i] = mlo == INT64_MIN ? mlo : mlo - i;
    hi_i[i] = mhi == INT64_MAX ? mhi : mhi - i;
  }
  const int64_t dpos = kp0 - (qp0 + n / d.row_div) + 4 * g;
  // kpos - qpos over the wavefront's keys and rows of page 0 (rows past M
  // included): a page whose whole range lies inside [mlo, mhi] keeps every
  // key, so its mask is skipped
  const int64_t dmin0 = kp0 - (qp0 + 15 / d.row_div), dmax0 = kp0 + 15 - qp0;
  // m: the running row max (the reference's m).  P, l and O are kept
  // relative to mr <= m, moved up to m only when m passes mr by more than 8
  // (so P <= e^8) and once after the loop: the same quantities as the
  // loop body's per-page rescale by alpha = exp(m - m'), up to rounding.
  float m = d.m0, mr = d.m0, lsum = d.l0;
  pa_f4 o[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) o[t] = pa_f4{0.f, 0.f, 0.f, 0.f};

  auto step = [&](int j, const PaOps<DT>& cur) {
    pa_f4 st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < DT; ++t)
      st = mfma_k32<BF16>(__builtin_bit_cast(uint4, cur.k[t]), __builtin_bit_cast(uint4, qf[t]), st);
    float s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = __fmul_rn(d.scale, st[i]);
    const int64_t js = (int64_t)j * d.kpos_step;
    if (inv || dmin0 + js < mlo || dmax0 + js > mhi) {
      const int64_t d0 = dpos + js;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if ((d0 >= lo_i[i] && d0 <= hi_i[i]) == inv) s[i] = d.neg;
    }
    float mx = pa_max(pa_max(s[0], s[1]), pa_max(s[2], s[3]));
    pa_f2 pr = pair16(mx);
    mx = pa_max(pr.x, pr.y);
    pr = pair32(mx);
    m = pa_max(m, pa_max(pr.x, pr.y));
    const bool up = m > mr + 8.f;
    if (__builtin_amdgcn_ballot_w64(up)) {
      const float f = up ? pa_exp(__fsub_rn(mr, m)) : 1.f;
      mr = up ? m : mr;
      lsum = __fmul_rn(lsum, f);
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[t][i] = __fmul_rn(o[t][i], f);
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = pa_exp(__fsub_rn(s[i], mr));
    float sum = __fadd_rn(__fadd_rn(p[0], p[1]), __fadd_rn(p[2], p[3]));
    pr = pair16(sum);
    sum = __fadd_rn(pr.x, pr.y);
    pr = pair32(sum);
    lsum = __fadd_rn(lsum, __fadd_rn(pr.x, pr.y));
    // P^T in the operand type: f16 rounds once (P <= e^8 keeps 11
    // significant bits, as the flash attention kernel's f16 P V), bf16
    // carries hi + lo (about 16 bits instead of 8)
    const uint32_t h0 = pa_cvt2<BF16>(p[0], p[1]), h1 = pa_cvt2<BF16>(p[2], p[3]);
    const uint2 ph = make_uint2(h0, h1);
    uint2 pl = make_uint2(0u, 0u);
    if constexpr (BF16) {
      const pa_f2 a = pa_uncvt2<BF16>(h0), c = pa_uncvt2<BF16>(h1);
      pl = make_uint2(pa_cvt2<BF16>(__fsub_rn(p[0], a.x), __fsub_rn(p[1], a.y)),
                      pa_cvt2<BF16>(__fsub_rn(p[2], c.x), __fsub_rn(p[3], c.y)));
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int w = t >> 1;
      // 16-bit element t & 1 of keys 4 g .. 4 g + 3, two per word (v_perm_b32:
      // bytes 0-1 or 2-3 of each source)
      const uint32_t sel = (t & 1) ? 0x07060302u : 0x05040100u;
      const uint32_t a0 = __builtin_amdgcn_perm(pa_vword<DT>(cur, 1, w), pa_vword<DT>(cur, 0, w), sel);
      const uint32_t a1 = __builtin_amdgcn_perm(pa_vword<DT>(cur, 3, w), pa_vword<DT>(cur, 2, w), sel);
      const uint2 va = make_uint2(a0, a1);
      o[t] = mfma_k16<BF16>(va, ph, o[t]);
      if constexpr (BF16) o[t] = mfma_k16<BF16>(va, pl, o[t]);
    }
  };

  int j = 0;                                   // next page to compute
  const int64_t page0 = trips > 0 ? page_at(0) : 0;
  int64_t k0l = kb + page0 * d.k_page, v0l = vb + page0 * d.v_page;
  if (vec && trips > 0 && pa_fast<DT>(d, k0l, v0l)) {
    // group X's pages from page j0 on: true when every page below trips is
    // fast.  Every group issues the same loads (a page past trips or not
    // fast reads the last fast page again, and a false result leaves X
    // unused), so the loads in flight do not depend on the path taken.
    auto issue = [&](int j0, PaOps<DT>* X) -> bool {
      int64_t k0s[G], v0s[G];
      bool ok = true;
#pragma unroll
      for (int u = 0; u < G; ++u) {
        if (ok && j0 + u < trips && j0 + u > 0) {
          const int64_t page = page_at(j0 + u);
          const int64_t k0 = kb + page * d.k_page, v0 = vb + page * d.v_page;
          ok = pa_fast<DT>(d, k0, v0);
          if (ok) {
            k0l = k0;
            v0l = v0;
          }
        }
        k0s[u] = k0l;
        v0s[u] = v0l;
      }
#pragma unroll
      for (int u = 0; u < G; ++u) pa_load_fast<DT>(d, k0s[u], v0s[u], lo, X[u]);
      return ok;
    };
    PaOps<DT> A[G], B[G];
    bool okA = issue(0, A), okB;
    __builtin_amdgcn_s_waitcnt(0);
    // at the top: A holds pages j .. j + G - 1 (landed); okA: all of them valid
    while (true) {
      if (!okA) break;
      okB = issue(j + G, B);
#pragma unroll
      for (int u = 0; u < G; ++u)
        if (j + u < trips) step(j + u, A[u]);
      j += G;
      __builtin_amdgcn_s_waitcnt(0);
      if (j >= trips || !okB) break;
      okA = issue(j + G, A);
#pragma unroll
      for (int u = 0; u < G; ++u)
        if (j + u < trips) step(j + u, B[u]);
      j += G;
      __builtin_amdgcn_s_waitcnt(0);
      if (j >= trips) break;
    }
  }
  // page by page from page j (the whole loop when the pages are not
  // aligned, else from the first page that leaves its window), element
  // loads where a piece leaves the window
  for (; j < trips; ++j) {
    const int64_t page = uni(pa_fix(pa_entry_raw(d, tp, j, trips), bad));
    const int64_t k0 = kb + page * d.k_page, v0 = vb + page * d.v_page;
    PaOps<DT> one;
    if (vec && pa_fast<DT>(d, k0, v0)) pa_load_fast<DT>(d, k0, v0, lo, one);
    else pa_load_any<DT>(d, k0, v0, lo, one);
    step(j, one);
  }
  if (bad) *err = 1;
  // bring P, l and O from mr to m (m > mr only where the loop ran and m
  // moved by at most 8 since the last rebase)
  if (m > mr) {
    const float f = pa_exp(__fsub_rn(mr, m));
    lsum = __fmul_rn(lsum, f);
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[t][i] = __fmul_rn(o[t][i], f);
  }
  if (n < M) {
    if (g == 0) {
      ((float*)d.m_out)[lane * M + n] = m;
      ((float*)d.l_out)[lane * M + n] = lsum;
    }
    if (d.out_ptr) {
      // the loop's finalisation: acc / l rounded to the output's dtype
      const int64_t ob = ((const int64_t*)d.out_base)[lane] + (int64_t)(n / d.out_grp) * d.out_gstride +
                         (int64_t)(n % d.out_grp) * d.out_row;
      const bool w16 = d.out_dtype != KTIR_F32 && !(d.out_ptr & 15);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t e0 = ob + NT * (4 * g + i);
        float v[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) v[t] = __fdiv_rn(o[t][i], lsum);
        if constexpr (NT % 8 == 0) {
          // the row's NT consecutive elements as 16-byte stores when they
          // lie in the window on a 16-byte boundary
          if (w16 && !(e0 & 7) && e0 >= d.out_lo && e0 + NT <= d.out_hi) {
#pragma unroll
            for (int q = 0; q < NT / 8; ++q) {
              uint32_t w[4];
#pragma unroll
              for (int h = 0; h < 4; ++h)
                w[h] = d.out_dtype == KTIR_BF16
                           ? (__float_as_uint(round_bf16(v[8 * q + 2 * h])) >> 16) |
                                 (__float_as_uint(round_bf16(v[8 * q + 2 * h + 1])) & 0xffff0000u)
                           : pa_cvt2<false>(v[8 * q + 2 * h], v[8 * q + 2 * h + 1]);
              *(KTIR_G(pa_u4)*)((KTIR_G(uint16_t)*)d.out_ptr + e0 + 8 * q) = pa_u4{w[0], w[1], w[2], w[3]};
            }
            continue;
          }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t)
          if (e0 + t >= d.out_lo && e0 + t < d.out_hi) store_elem(d.out_ptr, e0 + t, d.out_dtype, v[t]);
      }
    }
    float* ao = (float*)d.acc_out + (lane * M + n) * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float* dst = ao + NT * (4 * g + i);
      if constexpr (NT % 4 == 0) {
#pragma unroll
        for (int q = 0; q < NT / 4; ++q)
          *(float4*)(dst + 4 * q) = make_float4(o[4 * q][i], o[4 * q + 1][i], o[4 * q + 2][i], o[4 * q + 3][i]);
      } else {
#pragma unroll
        for (int t = 0; t < NT; ++t) dst[t] = o[t][i];
      }
    }
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
  if (d->out_ptr && (d->out_grp < 1 || (d->out_dtype != KTIR_F16 && d->out_dtype != KTIR_BF16 && d->out_dtype != KTIR_F32)))
    return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_paged_attention: output dtype %d / group %lld", d->out_dtype,
                     (long long)d->out_grp);
  if (d->lanes == 0) return KTIR_OK;
  if (d->lanes > INT_MAX) return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_paged_attention: too many lanes");
  // the matrix-core form: pages of 16 keys, at most 16 rows, D = 32, 64,
  // 128 or 256, one 16-bit operand type
  const bool same16 = d->q_dtype == d->kv_dtype && (d->kv_dtype == KTIR_F16 || d->kv_dtype == KTIR_BF16);
  if (same16 && d->N == 16 && d->M <= 16 && (d->D == 32 || d->D == 64 || d->D == 128 || d->D == 256)) {
    // vector loads: 16-byte aligned operands, rows and pages a multiple of 8 elements
    const int mvec = !((d->q_ptr | d->k_ptr | d->v_ptr) & 15) &&
                     !((d->q_row | d->k_row | d->v_row | d->k_page | d->v_page) & 7);
    const bool bf = d->kv_dtype == KTIR_BF16;
    auto mgo = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3((unsigned)d->lanes), dim3(64), 0, stream(), *d, mvec, device_error_flag());
    };
    switch (d->D) {
      // one page per group measured fastest at D = 128 (56 us against 64 us
      // for two): the registers of a second page cost more than its overlap
      case 32: bf ? mgo(pattn_mfma<true, 1, 1>) : mgo(pattn_mfma<false, 1, 1>); break;
      case 64: bf ? mgo(pattn_mfma<true, 2, 1>) : mgo(pattn_mfma<false, 2, 1>); break;
      case 128: bf ? mgo(pattn_mfma<true, 4, 1>) : mgo(pattn_mfma<false, 4, 1>); break;
      case 256: bf ? mgo(pattn_mfma<true, 8, 1>) : mgo(pattn_mfma<false, 8, 1>); break;
    }
    KTIR_HIP_CHECK(hipGetLastError());
    return KTIR_OK;
  }
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
