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
//     empty (link[e] == -1) is the row's owner; entries that do not survive
//     get link[e] = -2.
//   pass 2: every row with a chain is applied once.  A row with one entry is
//     a single load-combine-store; a longer chain is applied entry by entry
//     in ascending e, which is the reference's instance order, so the
//     floating point accumulation order is exactly the reference's.  The
//     common form (f32 rows, f16 / f32 sources) walks the head table in row
//     order; other forms give each owner entry half a wavefront.  Pass 2
//     resets every head it reads to -1, so the head table is all -1 between
//     calls (the caller fills it once).
#include "ktir_common.h"

namespace ktir {

typedef float gf4 __attribute__((ext_vector_type(4)));
typedef uint32_t gu2 __attribute__((ext_vector_type(2)));

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
  }
  if (bad) *err = 1;
}

// 4 columns [c, c+4) of a destination (dst) or source row
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

// RMW_NE entries per half-wavefront (32 lanes x 4 columns cover a 128-wide
// row per step): the entries' chain records are read together, then, for
// owners, the chain heads and all rows, before anything is combined.
constexpr int RMW_NE = 4;

__global__ __launch_bounds__(256) void rmw_apply(const ktir_rmw_t d, int64_t n_entries) {
  const int half = threadIdx.x / 32, hl = threadIdx.x % 32;
  const bool vec = d.dst_col == 1 && d.src_col == 1 && d.dst_dtype == KTIR_F32 &&
                   (d.src_dtype == KTIR_F16 || d.src_dtype == KTIR_F32) &&
                   (d.dst_base % 4 == 0) && (d.dst_row % 4 == 0) && (d.src_base % 4 == 0) && (d.src_row % 4 == 0);
  const int32_t* link = (const int32_t*)d.link;
  const int32_t* rows = (const int32_t*)d.rows;
  const int32_t* srcs = (const int32_t*)d.srcs;
  const int32_t* head = (const int32_t*)d.head;
  const int64_t step = (int64_t)gridDim.x * 8 * RMW_NE;
  for (int64_t e0 = ((int64_t)blockIdx.x * 8 + half) * RMW_NE; e0 < n_entries; e0 += step) {
    bool own[RMW_NE];
    int32_t r[RMW_NE], sr[RMW_NE], h[RMW_NE];
    // records of entries that do not survive are never read (their rows and
    // sources were not written): read all, use the owners'
#pragma unroll
    for (int j = 0; j < RMW_NE; ++j) {
      const int64_t e = e0 + j < n_entries ? e0 + j : e0;
      own[j] = e0 + j < n_entries && link[e] == -1;
      r[j] = rows[e];
      sr[j] = srcs[e];
    }
#pragma unroll
    for (int j = 0; j < RMW_NE; ++j) h[j] = own[j] ? head[r[j]] : 0;
    // the row's owner leaves its head empty again for the next call
#pragma unroll
    for (int j = 0; j < RMW_NE; ++j)
      if (own[j]) ((int32_t*)d.head)[r[j]] = -1;
    for (int64_t c = (int64_t)hl * 4; c < d.D; c += 128) {
      float v[RMW_NE][4], g[RMW_NE][4];
#pragma unroll
      for (int j = 0; j < RMW_NE; ++j) {
        if (!own[j]) continue;
        load4(d, true, d.dst_base + (int64_t)r[j] * d.dst_row + c * d.dst_col, c, vec, v[j]);
        load4(d, false, d.src_base + (int64_t)sr[j] * d.src_row + c * d.src_col, c, vec, g[j]);
      }
#pragma unroll
      for (int j = 0; j < RMW_NE; ++j) {
        if (!own[j]) continue;
        const int64_t de = d.dst_base + (int64_t)r[j] * d.dst_row;
        if (h[j] == (int32_t)(e0 + j)) {   // the row's only entry
          for (int i = 0; i < 4; ++i) v[j][i] = combine(d.op, d.order, d.dt, v[j][i], g[j][i]);
        } else {
          apply_chain(d, h[j], de, c, vec, v[j]);
        }
        store4(d, de + c * d.dst_col, c, vec, v[j]);
      }
    }
  }
}

// The common form: f32 destination rows and f16 / f32 source rows, unit
// column stride, 16-byte aligned rows, D a multiple of 128, f32 result.
// Destination-row order: wave w covers rows 64 w .. 64 w + 63 (one head
// entry per lane, read coalesced); the rows with a chain are compacted in
// LDS with their head entry's link and source, then applied by half
// wavefronts in ascending row order, so the row reads and writes of
// neighbouring wavefronts fall on neighbouring addresses.  Each head is reset
// to -1 once read.
template <int SDT>
__device__ __forceinline__ void rmw_src4(const ktir_rmw_t& d, int64_t se, float* g) {
  if (SDT == KTIR_F16) {
    const uint2 w = __builtin_bit_cast(uint2, *(const KTIR_G(gu2)*)((const KTIR_G(uint16_t)*)d.src_ptr + se));
    g[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.x & 0xffffu));
    g[1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.x >> 16));
    g[2] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.y & 0xffffu));
    g[3] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.y >> 16));
  } else {
    const gf4 w = *(const KTIR_G(gf4)*)((const KTIR_G(float)*)d.src_ptr + se);
    g[0] = w[0]; g[1] = w[1]; g[2] = w[2]; g[3] = w[3];
  }
}

template <int SDT>
__global__ __launch_bounds__(256) void rmw_apply_rows(const ktir_rmw_t d) {
  __shared__ int4 items[4][64];
  const int wv = threadIdx.x / 64, l = threadIdx.x % 64, half = l / 32, hl = l % 32;
  const int64_t r = ((int64_t)blockIdx.x * 4 + wv) * 64 + l;
  const int32_t h = r < d.n_rows ? ((const KTIR_G(int32_t)*)d.head)[r] : -1;
  const uint64_t mask = __ballot(h >= 0);
  const int n = __popcll(mask);
  if (h >= 0) {
    const int rank = __popcll(mask & ((1ull << l) - 1));
    const int32_t lk = ((const KTIR_G(int32_t)*)d.link)[h];
    const int32_t sr = ((const KTIR_G(int32_t)*)d.srcs)[h];
    items[wv][rank] = make_int4((int32_t)r, h, lk, sr);
    ((KTIR_G(int32_t)*)d.head)[r] = -1;
  }
  // the records are written and read by this wavefront only (its LDS
  // operations complete in order)
  __builtin_amdgcn_wave_barrier();
  const KTIR_G(float)* dst = (const KTIR_G(float)*)d.dst_ptr;
  for (int i = half; i < n; i += 2) {
    const int4 it = items[wv][i];
    const int64_t de = d.dst_base + (int64_t)it.x * d.dst_row;
    const int64_t se = d.src_base + (int64_t)it.w * d.src_row;
    // a source row outside its allocation (index past the table, or a
    // negative index that the host reports after the launch) reads zeros and
    // a destination row that ends past its allocation drops the columns
    // there (memory.py:243-305): such rows take the per-element path
    if (!(de >= 0 && de + d.D <= d.dst_hi && se >= 0 && se + d.D <= d.src_hi)) {
      for (int64_t c = (int64_t)hl * 4; c < d.D; c += 128) {
        float x[4], g[4];
        load4(d, true, de + c, c, true, x);
        if (it.z == -1) {
          load4(d, false, se + c, c, true, g);
          for (int q = 0; q < 4; ++q) x[q] = combine(d.op, d.order, KTIR_F32, x[q], g[q]);
        } else {
          apply_chain(d, it.y, de, c, true, x);
        }
        store4(d, de + c, c, true, x);
      }
      continue;
    }
    for (int64_t c = (int64_t)hl * 4; c < d.D; c += 128) {
      const gf4 v = *(const KTIR_G(gf4)*)(dst + de + c);
      float g[4];
      rmw_src4<SDT>(d, se + c, g);
      float x[4] = {v[0], v[1], v[2], v[3]};
      if (it.z == -1) {   // the head entry was also the chain's first: one entry
        for (int q = 0; q < 4; ++q) x[q] = combine(d.op, d.order, KTIR_F32, x[q], g[q]);
      } else {
        apply_chain(d, it.y, de, c, true, x);
      }
      *(KTIR_G(gf4)*)((KTIR_G(float)*)d.dst_ptr + de + c) = gf4{x[0], x[1], x[2], x[3]};
    }
  }
}

}  // namespace ktir

using namespace ktir;

static int rmw_check(const ktir_rmw_t* d, const char* who) {
  if (!d || d->K < 1 || d->K > RMW_MAXK || d->D < 1 || d->n_inst < 0)
    return set_error(KTIR_E_ARG, "%s: bad descriptor", who);
  if (d->n_inst * d->K >= (int64_t)0x7fffffff || d->n_rows >= (int64_t)0x7fffffff)
    return set_error(KTIR_E_UNSUPPORTED, "%s: too many entries", who);
  return KTIR_OK;
}

// The row-order apply kernel takes f32 destination rows, f16 / f32 source
// rows with unit column stride, positive row strides and 16-byte aligned
// rows of a multiple of 128 columns; everything else takes rmw_apply.
static bool rmw_rows_form(const ktir_rmw_t* d) {
  return d->dst_col == 1 && d->src_col == 1 && d->dst_dtype == KTIR_F32 && d->dt == KTIR_F32 &&
         (d->src_dtype == KTIR_F16 || d->src_dtype == KTIR_F32) && d->D % 128 == 0 && d->dst_row > 0 &&
         d->src_row >= 0 && d->dst_base % 4 == 0 && d->dst_row % 4 == 0 && d->src_base % 4 == 0 &&
         d->src_row % 4 == 0 && d->dst_ptr % 16 == 0 && d->src_ptr % 16 == 0;
}

extern "C" int ktir_rmw_variant(const ktir_rmw_t* d) {
  const int rc = rmw_check(d, "ktir_rmw_variant");
  if (rc != KTIR_OK) return rc;
  return rmw_rows_form(d) ? KTIR_RMW_ROWS : KTIR_RMW_GENERIC;
}

// The allocation-free form keeps the head, link, rows and srcs arrays in one
// file-scope device array: heads in a fixed region of RMW_NA_ROWS slots (all
// -1 between calls), then link, rows and srcs in fixed regions of
// RMW_NA_ENTRIES slots each, so no call's entries ever land in another call's
// heads.  In host code `scratch` names a host-side stand-in; its device
// address (one per device) comes from hipGetSymbolAddress, taken once per
// device by rmw_scratch_setup with that device current.
constexpr int64_t RMW_NA_ROWS = (int64_t)2 << 20;      // destination rows
constexpr int64_t RMW_NA_ENTRIES = (int64_t)1 << 20;   // n_inst * K
constexpr int64_t RMW_SCRATCH_WORDS = RMW_NA_ROWS + 3 * RMW_NA_ENTRIES;   // 20 MiB of int32
constexpr int RMW_MAX_DEVICES = 64;
__device__ __align__(256) int32_t scratch[RMW_SCRATCH_WORDS];
static int32_t* g_scratch[RMW_MAX_DEVICES];

__global__ __launch_bounds__(256) void rmw_fill(int32_t* p, int64_t n, int32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = v;
}

// Called by ktir_init with `device` current: the device address of this
// device's copy of `scratch`, and every head slot set to -1 (the head table is
// all -1 between calls: each launch resets the heads it uses).
int ktir::rmw_scratch_setup(int device) {
  if (device < 0 || device >= RMW_MAX_DEVICES)
    return set_error(KTIR_E_UNSUPPORTED, "ktir_init: device %d beyond the %d the RMW scratch table covers", device,
                     RMW_MAX_DEVICES);
  if (g_scratch[device]) return KTIR_OK;
  int32_t* ptr = nullptr;
  KTIR_HIP_CHECK(hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch)));
  hipLaunchKernelGGL(rmw_fill, dim3(1024), dim3(256), 0, stream(), ptr, RMW_NA_ROWS, (int32_t)-1);
  KTIR_HIP_CHECK(hipGetLastError());
  KTIR_HIP_CHECK(hipStreamSynchronize(stream()));
  g_scratch[device] = ptr;
  return KTIR_OK;
}

static int rmw_launch(const ktir_rmw_t* d);

extern "C" int ktir_launch_row_rmw_noalloc(const ktir_rmw_t* d) {
  const int rc = rmw_check(d, "ktir_launch_row_rmw_noalloc");
  if (rc != KTIR_OK) return rc;
  int dev = -1;
  KTIR_HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= RMW_MAX_DEVICES || !g_scratch[dev])
    return set_error(KTIR_E_ARG, "ktir_launch_row_rmw_noalloc: ktir_init was not called for device %d", dev);
  const int64_t entries = d->n_inst * d->K;
  if (d->n_rows > RMW_NA_ROWS || entries > RMW_NA_ENTRIES)
    return set_error(KTIR_E_UNSUPPORTED,
                     "ktir_launch_row_rmw_noalloc: %lld destination rows and %lld entries (n_inst * K) exceed "
                     "the scratch array's %lld rows and %lld entries (use ktir_launch_row_rmw with caller buffers)",
                     (long long)d->n_rows, (long long)entries, (long long)RMW_NA_ROWS, (long long)RMW_NA_ENTRIES);
  ktir_rmw_t w = *d;
  int32_t* base = g_scratch[dev];
  w.head = (uint64_t)base;
  w.link = (uint64_t)(base + RMW_NA_ROWS);
  w.rows = (uint64_t)(base + RMW_NA_ROWS + RMW_NA_ENTRIES);
  w.srcs = (uint64_t)(base + RMW_NA_ROWS + 2 * RMW_NA_ENTRIES);
  return rmw_launch(&w);
}

extern "C" int ktir_launch_row_rmw(const ktir_rmw_t* d) {
  const int rc = rmw_check(d, "ktir_launch_row_rmw");
  if (rc != KTIR_OK) return rc;
  return rmw_launch(d);
}

static int rmw_launch(const ktir_rmw_t* d) {
  if (d->n_inst == 0) return KTIR_OK;
  int t1 = d->K >= 256 ? 256 : (int)((d->K + 63) / 64 * 64);
  hipLaunchKernelGGL(rmw_link, dim3((unsigned)d->n_inst), dim3(t1), 0, stream(), *d, device_error_flag());
  const int64_t total = d->n_inst * d->K;
  if (rmw_rows_form(d)) {
    const int64_t blocks = (d->n_rows + 255) / 256;
    if (d->src_dtype == KTIR_F16)
      hipLaunchKernelGGL(rmw_apply_rows<KTIR_F16>, dim3((unsigned)blocks), dim3(256), 0, stream(), *d);
    else
      hipLaunchKernelGGL(rmw_apply_rows<KTIR_F32>, dim3((unsigned)blocks), dim3(256), 0, stream(), *d);
  } else {
    int64_t blocks = (total + 8 * RMW_NE - 1) / (8 * RMW_NE);
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(rmw_apply, dim3((unsigned)blocks), dim3(256), 0, stream(), *d, total);
  }
  KTIR_HIP_CHECK(hipGetLastError());
  return KTIR_OK;
}
