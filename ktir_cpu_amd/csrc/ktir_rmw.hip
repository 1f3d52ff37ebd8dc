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
      if (own) {
        int32_t* rec = owners + 4 + 4 * (int64_t)(base + rank);   // {entry, row, src, -}
        *(int4*)rec = make_int4((int32_t)e, r, ((int32_t*)d.srcs)[e], 0);
      }
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

// Two owners per half-wavefront (32 lanes x 4 columns cover a 128-wide row
// per step): the owner records, the chain heads and both rows of both owners
// are requested before anything is combined.
__device__ __forceinline__ void load4(const ktir_rmw_t& d, bool dst, int64_t e0, int64_t c, bool vec, float* v) {
  const uint64_t ptr = dst ? d.dst_ptr : d.src_ptr;
  const int dt = dst ? d.dst_dtype : d.src_dtype;
  const int64_t hi = dst ? d.dst_hi : d.src_hi, cs = dst ? d.dst_col : d.src_col;
  if (vec && e0 >= 0 && e0 + 4 <= hi) {
    if (dt == KTIR_F16) {
      uint2 w = *(const uint2*)((const _Float16*)ptr + e0);
      v[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.x & 0xffffu));
      v[1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.x >> 16));
      v[2] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.y & 0xffffu));
      v[3] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.y >> 16));
    } else {
      float4 w = *(const float4*)((const float*)ptr + e0);
      v[0] = w.x; v[1] = w.y; v[2] = w.z; v[3] = w.w;
    }
    return;
  }
  for (int i = 0; i < 4; ++i) {
    int64_t x = e0 + i * cs;
    v[i] = (c + i < d.D && x >= 0 && x < hi) ? load_elem(ptr, x, dt) : 0.f;
  }
}

__device__ __forceinline__ void store4(const ktir_rmw_t& d, int64_t e0, int64_t c, bool vec, const float* v) {
  if (vec && e0 >= 0 && e0 + 4 <= d.dst_hi) {
    *(float4*)((float*)d.dst_ptr + e0) = make_float4(v[0], v[1], v[2], v[3]);
    return;
  }
  for (int i = 0; i < 4; ++i) {
    int64_t x = e0 + i * d.dst_col;
    if (c + i < d.D && x >= 0 && x < d.dst_hi) store_elem(d.dst_ptr, x, d.dst_dtype, v[i]);
  }
}

__device__ __forceinline__ void apply_chain(const ktir_rmw_t& d, int32_t head, int64_t drow, int64_t c, bool vec,
                                         float* v) {
  const int32_t* link = (const int32_t*)d.link;
  const int32_t* srcs = (const int32_t*)d.srcs;
  int32_t prev = -1;
  while (true) {
    int32_t ent = 0x7fffffff;
    for (int32_t x = head; x >= 0; x = link[x])
      if (x > prev && x < ent) ent = x;
    if (ent == 0x7fffffff) break;
    prev = ent;
    float g[4];
    load4(d, false, d.src_base + (int64_t)srcs[ent] * d.src_row + c * d.src_col, c, vec, g);
    for (int i = 0; i < 4; ++i) v[i] = combine(d.op, d.order, d.dt, v[i], g[i]);
  }
}

__global__ __launch_bounds__(256) void rmw_apply(const ktir_rmw_t d) {
  const int32_t* owners = (const int32_t*)d.owners;
  const int32_t n_owners = owners[0];
  const int half = threadIdx.x / 32, hl = threadIdx.x % 32;
  const bool vec = d.dst_col == 1 && d.src_col == 1 && d.dst_dtype == KTIR_F32 &&
                   (d.src_dtype == KTIR_F16 || d.src_dtype == KTIR_F32) &&
                   (d.dst_base % 4 == 0) && (d.dst_row % 4 == 0) && (d.src_base % 4 == 0) && (d.src_row % 4 == 0);
  const int64_t step = (int64_t)gridDim.x * 16;
  for (int64_t o0 = (int64_t)blockIdx.x * 16 + half * 2; o0 < n_owners; o0 += step) {
    const bool two = o0 + 1 < n_owners;
    const int4 ra = *(const int4*)(owners + 4 + 4 * o0);
    const int4 rb = two ? *(const int4*)(owners + 4 + 4 * (o0 + 1)) : ra;
    const int32_t ha = ((const int32_t*)d.head)[ra.y];
    const int32_t hb = ((const int32_t*)d.head)[rb.y];
    const int64_t da = d.dst_base + (int64_t)ra.y * d.dst_row, db = d.dst_base + (int64_t)rb.y * d.dst_row;
    for (int64_t c = (int64_t)hl * 4; c < d.D; c += 128) {
      float va[4], vb[4], ga[4], gb[4];
      load4(d, true, da + c * d.dst_col, c, vec, va);
      load4(d, false, d.src_base + (int64_t)ra.z * d.src_row + c * d.src_col, c, vec, ga);
      if (two) {
        load4(d, true, db + c * d.dst_col, c, vec, vb);
        load4(d, false, d.src_base + (int64_t)rb.z * d.src_row + c * d.src_col, c, vec, gb);
      }
      if (ha == ra.x) {   // the row's only entry
        for (int i = 0; i < 4; ++i) va[i] = combine(d.op, d.order, d.dt, va[i], ga[i]);
      } else {
        apply_chain(d, ha, da, c, vec, va);
      }
      store4(d, da + c * d.dst_col, c, vec, va);
      if (two) {
        if (hb == rb.x) {
          for (int i = 0; i < 4; ++i) vb[i] = combine(d.op, d.order, d.dt, vb[i], gb[i]);
        } else {
          apply_chain(d, hb, db, c, vec, vb);
        }
        store4(d, db + c * d.dst_col, c, vec, vb);
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
  int64_t blocks = (total + 15) / 16;
  if (blocks > 16384) blocks = 16384;
  hipLaunchKernelGGL(rmw_apply, dim3((unsigned)blocks), dim3(256), 0, stream(), *d);
  KTIR_HIP_CHECK(hipGetLastError());
  return KTIR_OK;
}
