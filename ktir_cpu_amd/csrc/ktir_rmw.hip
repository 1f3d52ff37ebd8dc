// Ordered indirect read-modify-write of rows (scatter-accumulate through
// indirect access tiles), bit-exact against sequential execution.
//
// Reference order (grid.py:595-616, ops/memory_ops.py:868-964, memory.py:281-291):
// instances (core, loop iteration) run one after another; each one gathers
// K destination rows, combines them with K source rows, and scatters them
// back, where a destination repeated inside one instance keeps the value of
// its last position (computed from the row as it was before the instance).
//
//   pass 1 (one workgroup per instance): read the instance's K destination and
//     source indices, find the surviving (last) position of every destination
//     row inside the instance, and push survivors on the row's chain:
//     link[e] = atomicExch(&head[row], e).  The entry that finds the chain
//     empty becomes the row's owner and is appended to a compact owner list.
//   pass 2 (one half-wavefront per owner): a row with one entry is a single
//     load-combine-store; a longer chain is applied entry by entry in
//     ascending e, which is the reference's instance order, so the floating
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
  const int64_t q0 = ((const int64_t*)d.src_pos)[inst];
  bool bad = false;
  for (int k = threadIdx.x; k < d.K; k += blockDim.x) {
    int64_t r = read_index(d.dst_idx_ptr, d.dst_idx_dtype, p0 + k, d.dst_idx_hi, &bad);
    rows[k] = (r >= 0 && r < d.n_rows) ? (int32_t)r : -1;
  }
  __syncthreads();
  int32_t* owners = (int32_t*)d.owners;
  for (int k = threadIdx.x; k < d.K; k += blockDim.x) {
    const int64_t e = inst * d.K + k;
    const int32_t r = rows[k];
    bool last = r >= 0;
    for (int j = k + 1; j < d.K && last; ++j) last = rows[j] != r;
    int32_t prev = -2;
    if (last) {
      int64_t s = read_index(d.src_idx_ptr, d.src_idx_dtype, q0 + k, d.src_idx_hi, &bad);
      ((int32_t*)d.rows)[e] = r;
      ((int32_t*)d.srcs)[e] = (int32_t)(s < 0x7fffffff ? s : 0x7fffffff);
      prev = atomicExch(&((int32_t*)d.head)[r], (int32_t)e);
    }
    ((int32_t*)d.link)[e] = prev;
    // append owners (first pushed entry of a row) with one atomic per wavefront
    const bool own = prev == -1;
    const uint64_t mask = __ballot(own);
    if (mask) {
      const int leader = __ffsll((unsigned long long)mask) - 1;
      const int rank = __popcll(mask & ((1ull << (threadIdx.x & 63)) - 1));
      int32_t base = 0;
      if ((int)(threadIdx.x & 63) == leader) base = atomicAdd(&owners[0], __popcll(mask));
      base = __shfl(base, leader);
      if (own) owners[1 + base + rank] = (int32_t)e;
    }
  }
  if (bad) *err = 1;
}

// Apply one chain entry to the 4 columns [c, c+4) of the running row value.
__device__ __forceinline__ void apply_src(const ktir_rmw_t& d, int64_t s, int64_t c, float* v, bool vec) {
  const int64_t se = d.src_base + s * d.src_row + c * d.src_col;
  float g[4];
  if (vec && se >= 0 && se + 4 <= d.src_hi) {
    if (d.src_dtype == KTIR_F16) {
      uint2 w = *(const uint2*)((const _Float16*)d.src_ptr + se);
      const _Float16* h = (const _Float16*)&w;
      for (int i = 0; i < 4; ++i) g[i] = (float)h[i];
    } else {
      float4 w = *(const float4*)((const float*)d.src_ptr + se);
      g[0] = w.x; g[1] = w.y; g[2] = w.z; g[3] = w.w;
    }
  } else {
    for (int i = 0; i < 4; ++i) {
      int64_t x = se + i * d.src_col;
      g[i] = (c + i < d.D && x >= 0 && x < d.src_hi) ? load_elem(d.src_ptr, x, d.src_dtype) : 0.f;
    }
  }
  for (int i = 0; i < 4; ++i) v[i] = combine(d.op, d.order, d.dt, v[i], g[i]);
}

// One half-wavefront (32 lanes) per owner; each lane covers 4 columns per step.
__global__ __launch_bounds__(256) void rmw_apply(const ktir_rmw_t d) {
  const int32_t* owners = (const int32_t*)d.owners;
  const int32_t n_owners = owners[0];
  const int32_t* link = (const int32_t*)d.link;
  const int32_t* rows = (const int32_t*)d.rows;
  const int32_t* srcs = (const int32_t*)d.srcs;
  const int half = threadIdx.x / 32, hl = threadIdx.x % 32;
  const bool vec = d.dst_col == 1 && d.src_col == 1 && d.dst_dtype == KTIR_F32 &&
                   (d.src_dtype == KTIR_F16 || d.src_dtype == KTIR_F32) &&
                   (d.dst_base % 4 == 0) && (d.dst_row % 4 == 0) && (d.src_base % 4 == 0) && (d.src_row % 4 == 0);
  for (int64_t o = (int64_t)blockIdx.x * 8 + half; o < n_owners; o += (int64_t)gridDim.x * 8) {
    const int32_t e = owners[1 + o];
    const int32_t r = rows[e];
    const int32_t head = ((const int32_t*)d.head)[r];
    const int64_t drow = d.dst_base + (int64_t)r * d.dst_row;
    for (int64_t c = (int64_t)hl * 4; c < d.D; c += 128) {
      const int64_t de = drow + c * d.dst_col;
      float v[4];
      const bool dvec = vec && de >= 0 && de + 4 <= d.dst_hi;
      if (dvec) {
        float4 w = *(const float4*)((const float*)d.dst_ptr + de);
        v[0] = w.x; v[1] = w.y; v[2] = w.z; v[3] = w.w;
      } else {
        for (int i = 0; i < 4; ++i) {
          int64_t x = de + i * d.dst_col;
          v[i] = (c + i < d.D && x >= 0 && x < d.dst_hi) ? load_elem(d.dst_ptr, x, d.dst_dtype) : 0.f;
        }
      }
      if (head == e) {
        apply_src(d, srcs[e], c, v, vec);          // the row's only entry
      } else {
        // entries of the chain in ascending order (repeated selection)
        int32_t prev = -1;
        while (true) {
          int32_t ent = 0x7fffffff;
          for (int32_t x = head; x >= 0; x = link[x])
            if (x > prev && x < ent) ent = x;
          if (ent == 0x7fffffff) break;
          prev = ent;
          apply_src(d, srcs[ent], c, v, vec);
        }
      }
      if (dvec) {
        *(float4*)((float*)d.dst_ptr + de) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
        for (int i = 0; i < 4; ++i) {
          int64_t x = de + i * d.dst_col;
          if (c + i < d.D && x >= 0 && x < d.dst_hi) store_elem(d.dst_ptr, x, d.dst_dtype, v[i]);
        }
      }
    }
  }
}

}  // namespace ktir

using namespace ktir;

extern "C" int ktir_launch_row_rmw(const ktir_rmw_t* d) {
  if (!d || d->K < 1 || d->K > RMW_MAXK || d->D < 1 || d->n_inst < 0)
    return set_error(KTIR_E_ARG, "ktir_launch_row_rmw: bad descriptor");
  if (d->n_inst * d->K >= (int64_t)0x7fffffff || d->n_rows >= (int64_t)0x7fffffff)
    return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_row_rmw: too many entries");
  if (d->n_inst == 0) return KTIR_OK;
  KTIR_HIP_CHECK(hipMemsetAsync((void*)d->head, 0xff, (size_t)d->n_rows * 4, stream()));
  KTIR_HIP_CHECK(hipMemsetAsync((void*)d->owners, 0, 4, stream()));
  int t1 = d->K >= 256 ? 256 : (int)((d->K + 63) / 64 * 64);
  hipLaunchKernelGGL(rmw_link, dim3((unsigned)d->n_inst), dim3(t1), 0, stream(), *d, device_error_flag());
  int64_t total = d->n_inst * d->K;
  int64_t blocks = (total + 7) / 8;
  if (blocks > 16384) blocks = 16384;
  hipLaunchKernelGGL(rmw_apply, dim3((unsigned)blocks), dim3(256), 0, stream(), *d);
  KTIR_HIP_CHECK(hipGetLastError());
  return KTIR_OK;
}
