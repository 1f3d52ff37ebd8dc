// Fused tile programs: the gfx950 replacement for the reference's per-op
// NumPy tile kernels (ops/memory_ops.py load/store, ops/arith_ops.py,
// ops/math_ops.py, dialects/linalg_ops.py broadcast/transpose/generic/reduce).
//
// The host compiles a chain of KTIR tile ops into a short program over 8
// virtual registers; every register holds V consecutive elements of one
// thread, and the register file stays in VGPRs (uniform dynamic indexing).
// Each float instruction rounds to its declared dtype, so f16/bf16 chains
// give NumPy's results (compute in f32, round to nearest even, per op).
//
// Two execution modes:
//  * flat: one thread per V consecutive elements of the [lanes, shape...]
//    iteration space; leaves are read with 64/128-bit accesses when aligned.
//  * rows: one workgroup per row; ELEM blocks stream over the row; RED/FOLD
//    run the reference's pairwise-halving tree fold (linalg_ops.py:86-133:
//    element i is combined with i + n/2, an odd tail is carried) in LDS.
#include "ktir_program_impl.h"

namespace ktir {

// Lean flat programs: every load is a prefetched strided leaf, the last
// instruction is the only store, and the rest are register ops.  Per vector
// a thread keeps just one element offset per leaf, so U vectors (all their
// loads in flight together) fit in few registers.
template <int V>
__device__ __forceinline__ void lean_load(const ktir_leaf_t& L, int64_t e0, float* out) {
  if ((L.flags & KTIR_LEAF_VEC) && e0 >= L.lo && e0 + V <= L.hi) {
    if (V == 4) {
      switch (L.dtype) {
        case KTIR_F16: {
          uint2 w = *(const uint2*)((const _Float16*)L.ptr + e0);
          const _Float16* h = (const _Float16*)&w;
          for (int v = 0; v < V; ++v) out[v] = (float)h[v];
          return;
        }
        case KTIR_BF16: {
          uint2 w = *(const uint2*)((const uint16_t*)L.ptr + e0);
          out[0] = __uint_as_float(w.x << 16);
          out[1] = __uint_as_float(w.x & 0xffff0000u);
          out[2] = __uint_as_float(w.y << 16);
          out[3] = __uint_as_float(w.y & 0xffff0000u);
          return;
        }
        case KTIR_F32: case KTIR_I32: {
          float4 w = *(const float4*)((const float*)L.ptr + e0);
          out[0] = w.x; out[1] = w.y; out[2] = w.z; out[3] = w.w;
          return;
        }
        default: break;
      }
    }
  }
  const int64_t s = L.strides[KTIR_MAX_DIMS - 1];
  for (int v = 0; v < V; ++v) {
    int64_t e = e0 + v * s;
    out[v] = (e >= L.lo && e < L.hi) ? load_elem(L.ptr, e, L.dtype) : 0.f;
  }
}

template <int V>
__device__ __forceinline__ void lean_store(const ktir_leaf_t& L, int64_t e0, const float* val) {
  if (V == 4 && (L.flags & KTIR_LEAF_VEC) && e0 >= L.lo && e0 + V <= L.hi) {
    switch (L.dtype) {
      case KTIR_F16: {
        _Float16 h[4] = {(_Float16)val[0], (_Float16)val[1], (_Float16)val[2], (_Float16)val[3]};
        *(uint2*)((_Float16*)L.ptr + e0) = *(const uint2*)h;
        return;
      }
      case KTIR_BF16: {
        uint32_t b[4];
        for (int v = 0; v < 4; ++v) b[v] = __float_as_uint(round_bf16(val[v])) >> 16;
        *(uint2*)((uint16_t*)L.ptr + e0) = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
        return;
      }
      case KTIR_F32: case KTIR_I32:
        *(float4*)((float*)L.ptr + e0) = make_float4(val[0], val[1], val[2], val[3]);
        return;
      default: break;
    }
  }
  const int64_t s = L.strides[KTIR_MAX_DIMS - 1];
  for (int v = 0; v < V; ++v) {
    int64_t e = e0 + v * s;
    if (e >= L.lo && e < L.hi) store_elem(L.ptr, e, L.dtype, val[v]);
  }
}

template <int V, int U, int NPF>
__global__ __launch_bounds__(256) void prog_lean(const ktir_prog_t P, const FlatDivs D, uint32_t total_vecs,
                                                 int st_leaf) {
  const int nd = P.ndim;
  const uint32_t nthreads = gridDim.x * blockDim.x;
  const int npf = P.n_pf;
  const int n_ops = P.n_instr - 1;                  // the last instruction is the store
  const ktir_instr_t st = P.instr[P.n_instr - 1];
  for (uint32_t base = blockIdx.x * blockDim.x + threadIdx.x; base < total_vecs; base += nthreads * U) {
    float pf[U][NPF][V];
    int64_t est[U], lane[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      uint32_t vid = base + u * nthreads;
      if (vid >= total_vecs) vid = base;
      // normalised index: dims shifted so the innermost is at KTIR_MAX_DIMS-1
      uint32_t idx[KTIR_MAX_DIMS] = {0, 0, 0, 0};
      const uint32_t row = fdiv(vid, D.nvi);
      idx[KTIR_MAX_DIMS - 1] = (vid - row * D.nvi.d) * V;
      uint32_t t = row;
#pragma unroll
      for (int d = KTIR_MAX_DIMS - 2; d >= 0; --d) {
        if (d < nd - 1) {
          uint32_t q = fdiv(t, D.dim[d]);
          idx[KTIR_MAX_DIMS - nd + d] = t - q * D.dim[d].d;
          t = q;
        }
      }
      lane[u] = t;
#pragma unroll
      for (int k = 0; k < NPF; ++k)
        if (k < npf) lean_load<V>(P.leaves[P.pf_leaf[k]], leaf_off(P.leaves[P.pf_leaf[k]], t, idx), pf[u][k]);
      est[u] = leaf_off(P.leaves[st_leaf], t, idx);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (base + u * nthreads >= total_vecs) continue;
      float r[KTIR_NREG][V];
#pragma unroll
      for (int k = 0; k < NPF; ++k)
        if (k < npf) FOR_V r[k][v] = pf[u][k][v];
      for (int pc = 0; pc < n_ops; ++pc)
        exec<V, KTIR_NREG, false>(P, P.instr[pc], r, lane[u], nullptr, 0, 0, false, true, nullptr, 0, 0);
      float out[V];
      FOR_V out[v] = r[st.a][v];
      lean_store<V>(P.leaves[st_leaf], est[u], out);
    }
  }
}

// U vectors per thread; the program's leaf loads (n_pf <= NPF) for all U
// vectors are issued before any instruction runs.
template <int V, int NR, int U, int NPF, bool FULL>
__global__ __launch_bounds__(256) void prog_flat(const ktir_prog_t P, const FlatDivs D, uint32_t total_vecs) {
  const int nd = P.ndim;
  const int64_t inner = P.shape[nd - 1];
  int64_t per_lane = 1;
  for (int d = 0; d < nd; ++d) per_lane *= P.shape[d];
  const uint32_t nthreads = gridDim.x * blockDim.x;
  const int npf = P.n_pf;
  for (uint32_t base = blockIdx.x * blockDim.x + threadIdx.x; base < total_vecs; base += nthreads * U) {
    int64_t idx[U][KTIR_MAX_DIMS];
    int64_t lane[U], flat[U];
    float pf[U][NPF][V];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t vid = base + u * nthreads;
      decompose(vid < total_vecs ? vid : base, D, nd, V, inner, idx[u], lane[u], flat[u]);
#pragma unroll
      for (int k = 0; k < NPF; ++k)
        if (k < npf && vid < total_vecs)
          leaf_load<V>(P.leaves[P.pf_leaf[k]], nd, lane[u], idx[u], flat[u], pf[u][k], false);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (base + u * nthreads >= total_vecs) continue;
      float r[NR][V];
#pragma unroll
      for (int k = 0; k < NPF; ++k)
        if (k < npf) FOR_V r[k][v] = pf[u][k][v];
      for (int pc = 0; pc < P.n_instr; ++pc)
        exec<V, NR, FULL>(P, P.instr[pc], r, lane[u], idx[u], flat[u], per_lane, false, true, nullptr, 0, inner);
    }
  }
}

template <int V>
__device__ void fold_row(float* red, int64_t n, int op, int dt) {
  // Pairwise halving (reference dialects/linalg_ops.py:114-131): combine
  // element i with element i + n/2; an odd last element is carried along.
  __syncthreads();
  while (n > 1) {
    int64_t half = n >> 1;
    for (int64_t i = threadIdx.x; i < half; i += blockDim.x) red[i] = binop_any(op, dt, red[i], red[i + half]);
    __syncthreads();
    if (n & 1) {
      if (threadIdx.x == 0) red[half] = red[n - 1];
      __syncthreads();
      n = half + 1;
    } else {
      n = half;
    }
  }
}

template <int V>
__global__ __launch_bounds__(256) void prog_rows(const ktir_prog_t P, int64_t total_rows) {
  // one row's values for the fold: `inner` floats of dynamic LDS, so short
  // rows leave room for many workgroups per CU
  extern __shared__ float red[];
  const int nd = P.ndim;
  const int64_t inner = P.shape[nd - 1];
  int64_t rows_per_lane = 1;
  for (int d = 0; d < nd - 1; ++d) rows_per_lane *= P.shape[d];
  const int64_t per_lane = rows_per_lane * inner;
  for (int64_t row = blockIdx.x; row < total_rows; row += gridDim.x) {
    int64_t lane = row / rows_per_lane;
    int64_t rr = row - lane * rows_per_lane;
    int64_t idx[KTIR_MAX_DIMS];
    int64_t t = rr;
    for (int d = nd - 2; d >= 0; --d) {
      int64_t q = t / P.shape[d];
      idx[d] = t - q * P.shape[d];
      t = q;
    }
    float r[KTIR_NREG][V];
    int pc = 0;
    while (pc < P.n_instr) {
      const ktir_instr_t in = P.instr[pc];
      if (in.op == KTIR_OP_ELEM) {
        int end = in.aux;
        for (int64_t c0 = (int64_t)threadIdx.x * V; c0 < inner; c0 += (int64_t)blockDim.x * V) {
          idx[nd - 1] = c0;
          for (int p = pc + 1; p < end; ++p)
            exec<V, KTIR_NREG, true>(P, P.instr[p], r, lane, idx, rr * inner + c0, per_lane, false, true, red, c0, inner);
        }
        pc = end + 1;
        continue;
      }
      if (in.op == KTIR_OP_FOLD) {
        fold_row<V>(red, inner, in.aux, in.dt);
        float x = red[0];
        __syncthreads();
        FOR_V r[in.dst][v] = x;
      } else {
        idx[nd - 1] = 0;
        exec<V, KTIR_NREG, true>(P, in, r, lane, idx, rr * inner, per_lane, true, threadIdx.x == 0, red, 0, inner);
      }
      ++pc;
    }
  }
}

}  // namespace ktir

using namespace ktir;

namespace ktir {
bool try_launch_map(const ktir_prog_t& Q, int64_t rows, int64_t inner);
bool try_launch_tile(const ktir_prog_t& Q, int64_t lanes, int64_t per_lane, int64_t inner);
bool try_launch_rows(const ktir_prog_t& P, int64_t rows, int64_t inner);
int64_t row_grid_limit(int64_t blocks);
}

extern "C" int ktir_launch_program(const ktir_prog_t* P) {
  if (!P || P->ndim < 1 || P->ndim > KTIR_MAX_DIMS || P->n_instr > KTIR_MAX_INSTR || P->n_leaves > KTIR_MAX_LEAVES)
    return set_error(KTIR_E_ARG, "ktir_launch_program: bad descriptor");
  int64_t per_lane = 1;
  for (int d = 0; d < P->ndim; ++d) {
    if (P->shape[d] < 0) return set_error(KTIR_E_ARG, "ktir_launch_program: negative extent");
    per_lane *= P->shape[d];
  }
  if (per_lane == 0 || P->lanes == 0) return KTIR_OK;
  const int64_t inner = P->shape[P->ndim - 1];
  const bool v4 = (inner % 4) == 0;
  if (P->mode == 0) {
    bool full = false;
    for (int i = 0; i < P->n_instr; ++i) full |= !simple_op(P->instr[i].op);
    const int V = inner % 4 == 0 ? 4 : 1;
    int64_t rows = P->lanes * (per_lane / inner);
    int64_t vecs = rows * (inner / V);
    if (vecs >= (int64_t)0x7fffffff)
      return set_error(KTIR_E_UNSUPPORTED, "program over %lld vectors", (long long)vecs);
    FlatDivs D;
    D.nvi = make_fastdiv((uint32_t)(inner / V));
    for (int d = 0; d < KTIR_MAX_DIMS; ++d) D.dim[d] = make_fastdiv(d < P->ndim - 1 ? (uint32_t)P->shape[d] : 1);
    D.rows_per_lane = (uint32_t)(per_lane / inner);
    // lean path: loads all prefetched (strided), one final store, register ops only
    bool lean = !full && P->n_instr >= 1 && P->instr[P->n_instr - 1].op == KTIR_OP_ST && P->n_pf <= 2;
    for (int i = 0; lean && i < P->n_instr - 1; ++i) {
      int op = P->instr[i].op;
      lean = op != KTIR_OP_LD && op != KTIR_OP_ST && op != KTIR_OP_IDX;
    }
    for (int k = 0; lean && k < P->n_pf; ++k) lean = P->leaves[P->pf_leaf[k]].offsets == 0;
    if (lean) {
      const ktir_leaf_t& sl = P->leaves[P->instr[P->n_instr - 1].aux];
      lean = sl.offsets == 0 && sl.winner == 0;
    }
    dim3 b(256);
    uint32_t nv = (uint32_t)vecs;
    if (!full && P->n_pf > 2 && try_launch_map(*P, rows, inner)) {   // three or four inputs in four registers
      KTIR_HIP_CHECK(hipGetLastError());
      return KTIR_OK;
    }
    if (!full && try_launch_tile(*P, P->lanes, per_lane, inner)) {
      KTIR_HIP_CHECK(hipGetLastError());
      return KTIR_OK;
    }
    if (lean) {
      if (try_launch_map(*P, rows, inner)) {
        KTIR_HIP_CHECK(hipGetLastError());
        return KTIR_OK;
      }
    }
    if (lean) {
      // leaf strides normalised to KTIR_MAX_DIMS dims (innermost last)
      ktir_prog_t Q = *P;
      for (int l = 0; l < Q.n_leaves; ++l) {
        int64_t st[KTIR_MAX_DIMS] = {0, 0, 0, 0};
        for (int d = 0; d < Q.ndim; ++d) st[KTIR_MAX_DIMS - Q.ndim + d] = P->leaves[l].strides[d];
        for (int d = 0; d < KTIR_MAX_DIMS; ++d) Q.leaves[l].strides[d] = st[d];
      }
      const int U = 4;
      int64_t blocks = (vecs + 256 * U - 1) / (256 * U);
      if (blocks > 1048576) blocks = 1048576;
      if (V == 4)
        hipLaunchKernelGGL((prog_lean<4, 4, 2>), dim3((unsigned)blocks), b, 0, stream(), Q, D, nv,
                           (int)P->instr[P->n_instr - 1].aux);
      else
        hipLaunchKernelGGL((prog_lean<1, 4, 2>), dim3((unsigned)blocks), b, 0, stream(), Q, D, nv,
                           (int)P->instr[P->n_instr - 1].aux);
    } else {
      const int U = 1;
      int64_t blocks = (vecs + 256 * U - 1) / (256 * U);
      if (blocks > 1048576) blocks = 1048576;
      dim3 g((unsigned)blocks);
      if (V == 4 && !full)
        hipLaunchKernelGGL((prog_flat<4, 8, 1, 4, false>), g, b, 0, stream(), *P, D, nv);
      else if (V == 4)
        hipLaunchKernelGGL((prog_flat<4, 8, 1, 4, true>), g, b, 0, stream(), *P, D, nv);
      else
        hipLaunchKernelGGL((prog_flat<1, 8, 1, 4, true>), g, b, 0, stream(), *P, D, nv);
    }
  } else {
    if (inner > KTIR_MAX_ROW)
      return set_error(KTIR_E_UNSUPPORTED, "row program: row of %lld elements exceeds %d", (long long)inner,
                       KTIR_MAX_ROW);
    int64_t rows = P->lanes * (per_lane / inner);
    if (try_launch_rows(*P, rows, inner)) {
      KTIR_HIP_CHECK(hipGetLastError());
      return KTIR_OK;
    }
    int64_t blocks = row_grid_limit(rows < 65536 ? rows : 65536);
    int64_t per = v4 ? inner / 4 : inner;
    int threads = per >= 256 ? 256 : (int)((per + 63) / 64 * 64);
    const size_t lds = (size_t)inner * sizeof(float);
    if (v4)
      hipLaunchKernelGGL(prog_rows<4>, dim3((unsigned)blocks), dim3(threads), lds, stream(), *P, rows);
    else
      hipLaunchKernelGGL(prog_rows<1>, dim3((unsigned)blocks), dim3(threads), lds, stream(), *P, rows);
  }
  KTIR_HIP_CHECK(hipGetLastError());
  return KTIR_OK;
}
