// Ordered indirect read-modify-write of rows (scatter-accumulate through
// indirect access tiles), bit-exact against sequential execution.
//
// Reference order (grid.py:595-616, ops/memory_ops.py:868-964, memory.py:281-291):
// instances (core, loop iteration) run one after another; each one gathers
// K destination rows, combines them with K source rows, and scatters them
// back, where a destination repeated inside one instance keeps the value of
// its last position (computed from the row as it was before the instance).
//
//   pass 1 (rmw_link, one workgroup per instance): the instance's last
//     position of every destination row survives (an LDS hash table with
//     open addressing keeps each row's largest position).  A survivor e of
//     row r exchanges itself into
//     head[r]; the entry that finds head[r] empty is the row's owner, and
//     every later arrival writes (its entry, its source row) into its
//     predecessor's successor slot.  The record of entry e is the pair
//     (r for an owner, -2 - r for a later arrival, -1 for an entry that does
//     not survive; the source row).
//   pass 2 (rmw_apply_rows / rmw_apply): the owner of each row reads its
//     record and its successor slot together, so a row with one or two
//     entries issues all its loads in one round trip; the entries are applied
//     in ascending e, which is the reference's instance order, so the
//     floating point accumulation order is exactly the reference's.  Longer
//     chains (rare) are walked.  Pass 2 leaves head[] and the successor slots
//     at -1 again, so they are -1 between calls (the caller fills them once).
#include "ktir_common.h"

namespace ktir {

typedef float gf4 __attribute__((ext_vector_type(4)));
typedef uint32_t gu2 __attribute__((ext_vector_type(2)));
typedef int32_t gi2 __attribute__((ext_vector_type(2)));
typedef int32_t gi4 __attribute__((ext_vector_type(4)));

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

// LDS hash slots for the last-position test: a power of two, at least 64
// and at least 4 per position (so at most a quarter of them are taken)
__host__ __device__ __forceinline__ int rmw_table_slots(int K) {
  int tb = 64;
  while (tb < 4 * K) tb <<= 1;
  return tb;
}

// The launch sizes the LDS to K (destination rows, source rows, then the
// hash table's keys and values), so that at the usual K = 128 (5 KB) many
// more workgroups share a CU than a fixed RMW_MAXK-sized table would allow.
// The table is open addressing with linear probing: a position claims its
// row's slot (compare-and-swap of the key from -1) or finds it, and raises
// the slot's value to its position; a lookup probes to the row's key.  Each
// row has exactly one slot, and with at most a quarter of the slots taken
// the probe sequences stay short (the table never fills, so they end).
__global__ __launch_bounds__(256) void rmw_link(const ktir_rmw_t d, int* err) {
  extern __shared__ int32_t rmw_lds[];
  const int K = (int)d.K;
  const int tb = rmw_table_slots(K);
  int32_t* rows = rmw_lds;
  int32_t* srcs = rmw_lds + K;
  int32_t* keys = rmw_lds + 2 * K;
  int32_t* last_pos = keys + tb;
  const int64_t inst = blockIdx.x;
  const int64_t p0 = ((const int64_t*)d.dst_pos)[inst];
  const int64_t q0 = ((const int64_t*)d.src_pos)[inst];
  const int tshift = 32 - __builtin_ctz(tb);
  const uint32_t tmask = (uint32_t)tb - 1;
  bool bad = false;
  for (int i = threadIdx.x; i < tb; i += blockDim.x) {
    keys[i] = -1;
    last_pos[i] = -1;
  }
  // both index views are read at every position, as the instance's gather
  // and scatter tiles read them (a negative value anywhere is an error)
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    const int64_t r = read_index(d.dst_idx_ptr, d.dst_idx_dtype, p0 + k, d.dst_idx_hi, &bad);
    const int64_t s = read_index(d.src_idx_ptr, d.src_idx_dtype, q0 + k, d.src_idx_hi, &bad);
    rows[k] = (r >= 0 && r < d.n_rows) ? (int32_t)r : -1;
    srcs[k] = (int32_t)(s < 0x7fffffff ? s : 0x7fffffff);
  }
  __syncthreads();
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    const int32_t r = rows[k];
    if (r < 0) continue;
    uint32_t h = ((uint32_t)r * 2654435761u) >> tshift;
    for (int probe = 0; probe < tb; ++probe, h = (h + 1) & tmask) {
      const int32_t owner = atomicCAS(&keys[h], -1, r);
      if (owner == -1 || owner == r) {
        atomicMax(&last_pos[h], k);
        break;
      }
    }
  }
  __syncthreads();
  int2* rec = (int2*)d.rows;
  int2* nxt = (int2*)d.link;
  for (int k = threadIdx.x; k < K; k += blockDim.x) {
    const int64_t e = inst * d.K + k;
    const int32_t r = rows[k];
    bool last = false;
    if (r >= 0) {
      uint32_t h = ((uint32_t)r * 2654435761u) >> tshift;
      for (int probe = 0; probe < tb && keys[h] != r; ++probe) h = (h + 1) & tmask;
      last = last_pos[h] == k;
    }
    int32_t code = -1, s32 = 0;
    if (last) {
      s32 = srcs[k];
      const int32_t prev = atomicExch(&((int32_t*)d.head)[r], (int32_t)e);
      // heads hold entries of this call only (-1 between calls); the bound
      // keeps a corrupted head from turning into a stray write
      if (prev >= 0 && prev < d.n_inst * d.K) nxt[prev] = make_int2((int32_t)e, s32);
      code = prev >= 0 ? -2 - r : r;
    }
    rec[e] = make_int2(code, s32);
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

// The rows form's element access (unit column stride, f32 destination, f16
// or f32 source): 4 columns [c, c + 4) from element e0, zeros outside
// [0, hi); the dtype is a template constant, so no per-element dtype switch.
template <int DT>
__device__ __forceinline__ void rows_get4(uint64_t ptr, int64_t e0, int64_t c, int64_t D, int64_t hi, float* v) {
  if (e0 >= 0 && e0 + 4 <= hi) {
    if (DT == KTIR_F16) {
      const uint2 w = __builtin_bit_cast(uint2, *(const KTIR_G(gu2)*)((const KTIR_G(uint16_t)*)ptr + e0));
      v[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.x & 0xffffu));
      v[1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.x >> 16));
      v[2] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.y & 0xffffu));
      v[3] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w.y >> 16));
    } else {
      const gf4 w = *(const KTIR_G(gf4)*)((const KTIR_G(float)*)ptr + e0);
      v[0] = w[0]; v[1] = w[1]; v[2] = w[2]; v[3] = w[3];
    }
    return;
  }
  for (int i = 0; i < 4; ++i) {
    const int64_t x = e0 + i;
    const bool in = c + i < D && x >= 0 && x < hi;
    v[i] = !in ? 0.f
               : (DT == KTIR_F16 ? (float)((const KTIR_G(_Float16)*)ptr)[x] : ((const KTIR_G(float)*)ptr)[x]);
  }
}

__device__ __forceinline__ void rows_put4(const ktir_rmw_t& d, int64_t e0, int64_t c, const float* v) {
  if (e0 >= 0 && e0 + 4 <= d.dst_hi) {
    *(KTIR_G(gf4)*)((KTIR_G(float)*)d.dst_ptr + e0) = gf4{v[0], v[1], v[2], v[3]};
    return;
  }
  for (int i = 0; i < 4; ++i) {
    const int64_t x = e0 + i;
    if (c + i < d.D && x >= 0 && x < d.dst_hi) ((KTIR_G(float)*)d.dst_ptr)[x] = v[i];
  }
}

// A chain of three or more entries (rare): starting from the owner (entry e,
// source s), the successor slots list the others in arrival order; apply
// them in ascending entry order by repeated selection (bounded walks).
// Each arrival links only to an earlier one, so chains are acyclic and at most
// n_entries long: that bound never cuts a chain short.
template <typename SRC4>
__device__ __forceinline__ void apply_long_chain(const ktir_rmw_t& d, int op, int32_t e, int32_t s, int2 nx, int dt,
                                                 float* x, SRC4 src4) {
  const int2* nxt = (const int2*)d.link;
  const int64_t bound = d.n_inst * d.K + 1;
  int32_t prevm = -1;
  for (int64_t it = 0; it < bound; ++it) {
    int32_t m = 0x7fffffff, sm = 0;
    if (e > prevm) { m = e; sm = s; }
    int64_t steps = 0;
    for (int2 t = nx; t.x >= 0 && t.x < bound - 1 && steps < bound; t = nxt[t.x], ++steps)
      if (t.x > prevm && t.x < m) { m = t.x; sm = t.y; }
    if (m == 0x7fffffff) break;
    prevm = m;
    float g[4];
    src4(sm, g);
    for (int q = 0; q < 4; ++q) x[q] = combine(op, d.order, dt, x[q], g[q]);
  }
}

// Lane 0 of the owner's half-wave leaves the row's head and successor slots
// empty again (after every lane has read them).
__device__ __forceinline__ void rmw_reset(const ktir_rmw_t& d, int32_t r, int32_t e, int2 nx, int hl) {
  __builtin_amdgcn_wave_barrier();
  if (hl != 0) return;
  ((int32_t*)d.head)[r] = -1;
  int2* nxt = (int2*)d.link;
  if (nx.x < 0) return;
  int32_t y = e;
  const int64_t bound = d.n_inst * d.K + 1;
  for (int64_t steps = 0; y >= 0 && y < bound - 1 && steps < bound; ++steps) {
    const int32_t y2 = nxt[y].x;
    nxt[y] = make_int2(-1, -1);
    y = y2;
  }
}

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

// A chain of three to RMW_CH entries whose rows lie inside their
// allocations: walk it once from the owner's third entry, keeping every
// (entry, source) pair, order the sources by ascending entry, then combine
// them in that order (instead of a walk per entry with a load after each).
// Returns false, having changed nothing, for a longer chain or a source row
// outside its allocation (the element-by-element path takes those).
constexpr int RMW_CH = 8;

template <int SDT, bool D128>
__device__ __forceinline__ bool apply_short_chain(const ktir_rmw_t& d, int op, int32_t r, int32_t e, int32_t s,
                                                  int2 nx, int2 n2, int64_t n_entries, int hl) {
  const KTIR_G(gi2)* nxt = (const KTIR_G(gi2)*)d.link;
  int32_t ce[RMW_CH], cs[RMW_CH];
  ce[0] = e; cs[0] = s;
  ce[1] = nx.x; cs[1] = nx.y;
  ce[2] = n2.x; cs[2] = n2.y;
  int L = 3;
  int2 t = n2;
#pragma unroll
  for (int q = 3; q <= RMW_CH; ++q) {
    const gi2 u = nxt[t.x];
    t = u.x >= 0 && u.x < n_entries ? make_int2(u.x, u.y) : make_int2(-1, -1);
    if (t.x < 0) break;
    if (q == RMW_CH) return false;       // longer than RMW_CH entries
    ce[q] = t.x;
    cs[q] = t.y;
    L = q + 1;
  }
  const int64_t D = D128 ? 128 : d.D;
#pragma unroll
  for (int q = 0; q < RMW_CH; ++q) {
    if (q >= L) break;
    const int64_t se = d.src_base + (int64_t)cs[q] * d.src_row;
    if (se < 0 || se + D > d.src_hi) return false;
  }
  const KTIR_G(float)* dst = (const KTIR_G(float)*)d.dst_ptr;
  const int64_t de = d.dst_base + (int64_t)r * d.dst_row;
  // the order of application: sources by ascending entry
  int32_t os[RMW_CH];
  int32_t prev = -1;
#pragma unroll
  for (int it = 0; it < RMW_CH; ++it) {
    int32_t m = 0x7fffffff, sm = 0;
#pragma unroll
    for (int q = 0; q < RMW_CH; ++q) {
      const bool take = q < L && ce[q] > prev && ce[q] < m;
      m = take ? ce[q] : m;
      sm = take ? cs[q] : sm;
    }
    prev = m;
    os[it] = sm;
  }
  for (int64_t c = (int64_t)hl * 4; c < D; c += 128) {
    const gf4 v = *(const KTIR_G(gf4)*)(dst + de + c);
    float x[4] = {v[0], v[1], v[2], v[3]};
#pragma unroll
    for (int it = 0; it < RMW_CH; ++it) {
      if (it >= L) break;
      float g[4];
      rmw_src4<SDT>(d, d.src_base + (int64_t)os[it] * d.src_row + c, g);
#pragma unroll
      for (int k = 0; k < 4; ++k) x[k] = combine(op, d.order, KTIR_F32, x[k], g[k]);
    }
    *(KTIR_G(gf4)*)((KTIR_G(float)*)d.dst_ptr + de + c) = gf4{x[0], x[1], x[2], x[3]};
  }
  // leave the row's head and every slot of the chain empty (after every lane
  // of the half-wave has read them)
  __builtin_amdgcn_wave_barrier();
  if (hl == 0) {
    ((KTIR_G(int32_t)*)d.head)[r] = -1;
    KTIR_G(gi2)* slot = (KTIR_G(gi2)*)d.link;
#pragma unroll
    for (int q = 0; q < RMW_CH; ++q)
      if (q < L) slot[ce[q]] = gi2{-1, -1};
  }
  return true;
}

// The common form: f32 destination rows and f16 / f32 source rows, unit
// column stride, 16-byte aligned rows, D a multiple of 128, f32 result.  A
// half-wave takes RMW_NE consecutive entries; lane l covers columns
// 4l .. 4l + 3 of each 128-column group.  An owner's record, its successor
// slot, its destination row and every source row of a one- or two-entry
// chain are loaded before anything is combined.  OPT >= 0 fixes the combining
// op at compile time (the launcher instantiates the add, the common case):
// the per-element op switch then disappears from the hot path, which keeps
// the kernel a fifth of its size; OPT = -1 reads the op from the descriptor.
constexpr int RMW_NE = 2;

template <int SDT, bool D128, int OPT>
__global__ __launch_bounds__(256) void rmw_apply_rows(const ktir_rmw_t d, int64_t n_entries) {
  const int op = OPT >= 0 ? OPT : d.op;
  const int64_t hw = ((int64_t)blockIdx.x * 256 + threadIdx.x) / 32;
  const int hl = threadIdx.x % 32;
  const int64_t e0 = hw * RMW_NE;
  // When the head table is at most 8 slots per entry, every thread first
  // sets four consecutive heads to -1 (the launch has 16 threads per entry,
  // so the grid covers the table): one coalesced pass instead of a 4-byte
  // write at a random address per owner.  Nothing in this kernel reads the
  // heads; rmw_link of this call has finished with them.
  const bool dense = d.n_rows <= 8 * n_entries;
  if (dense) {
    KTIR_G(int32_t)* hd = (KTIR_G(int32_t)*)d.head;
    const int64_t h0 = 4 * ((int64_t)blockIdx.x * 256 + threadIdx.x);
    if (h0 + 4 <= d.n_rows && (d.head & 15) == 0)
      *(KTIR_G(gi4)*)(hd + h0) = gi4{-1, -1, -1, -1};
    else
      for (int64_t i = h0; i < h0 + 4 && i < d.n_rows; ++i) hd[i] = -1;
  }
  if (e0 >= n_entries) return;
  const int64_t D = D128 ? 128 : d.D;
  const KTIR_G(gi2)* rec = (const KTIR_G(gi2)*)d.rows;
  KTIR_G(gi2)* nxt = (KTIR_G(gi2)*)d.link;
  KTIR_G(int32_t)* head = (KTIR_G(int32_t)*)d.head;
  int32_t r[RMW_NE], s[RMW_NE];
  int2 nx[RMW_NE], n2[RMW_NE];
  bool fast[RMW_NE];
#pragma unroll
  for (int j = 0; j < RMW_NE; ++j) {
    const int64_t e = e0 + j < n_entries ? e0 + j : e0;
    const gi2 t = rec[e], u = nxt[e];
    r[j] = e0 + j < n_entries ? t.x : -1;
    s[j] = t.y;
    // a successor outside this call's entries cannot occur when the slots
    // hold -1 on entry; such a value is never dereferenced
    nx[j] = u.x >= 0 && u.x < n_entries ? make_int2(u.x, u.y) : make_int2(-1, -1);
  }
#pragma unroll
  for (int j = 0; j < RMW_NE; ++j) {
    const int64_t de = d.dst_base + (int64_t)r[j] * d.dst_row;
    const int64_t se = d.src_base + (int64_t)s[j] * d.src_row;
    const int64_t se2 = d.src_base + (int64_t)nx[j].y * d.src_row;
    // every row the owner touches lies inside its allocation (else the
    // per-element path below: zeros past the end, dropped writes; memory.py:243-305)
    fast[j] = r[j] >= 0 && de >= 0 && de + D <= d.dst_hi && se >= 0 && se + D <= d.src_hi &&
              (nx[j].x < 0 || (se2 >= 0 && se2 + D <= d.src_hi));
  }
  const KTIR_G(float)* dst = (const KTIR_G(float)*)d.dst_ptr;
  for (int64_t c = (int64_t)hl * 4; c < D; c += 128) {
    gf4 v[RMW_NE];
    float g[RMW_NE][4], g2[RMW_NE][4];
    // the owner's rows, its successor's source row and the successor's own
    // successor slot (a third entry) are all read in this one round trip
#pragma unroll
    for (int j = 0; j < RMW_NE; ++j) {
      n2[j] = make_int2(-1, -1);
      if (!fast[j]) continue;
      v[j] = *(const KTIR_G(gf4)*)(dst + d.dst_base + (int64_t)r[j] * d.dst_row + c);
      rmw_src4<SDT>(d, d.src_base + (int64_t)s[j] * d.src_row + c, g[j]);
      if (nx[j].x >= 0) {
        rmw_src4<SDT>(d, d.src_base + (int64_t)nx[j].y * d.src_row + c, g2[j]);
        const gi2 t = nxt[nx[j].x];
        // checked like nx: a slot outside this call's entries is not followed
        n2[j] = t.x >= 0 && t.x < n_entries ? make_int2(t.x, t.y) : make_int2(-1, -1);
      }
    }
#pragma unroll
    for (int j = 0; j < RMW_NE; ++j) {
      if (!fast[j] || n2[j].x >= 0) continue;
      float x[4] = {v[j][0], v[j][1], v[j][2], v[j][3]};
      const bool second_first = nx[j].x >= 0 && nx[j].x < e0 + j;
      if (second_first)
        for (int q = 0; q < 4; ++q) x[q] = combine(op, d.order, KTIR_F32, x[q], g2[j][q]);
      for (int q = 0; q < 4; ++q) x[q] = combine(op, d.order, KTIR_F32, x[q], g[j][q]);
      if (nx[j].x >= 0 && !second_first)
        for (int q = 0; q < 4; ++q) x[q] = combine(op, d.order, KTIR_F32, x[q], g2[j][q]);
      if (hl == 0 && c + 128 >= D) {    // the row's last column group: leave its head and slot empty
        if (!dense) head[r[j]] = -1;
        if (nx[j].x >= 0) nxt[e0 + j] = gi2{-1, -1};
      }
      *(KTIR_G(gf4)*)((KTIR_G(float)*)d.dst_ptr + d.dst_base + (int64_t)r[j] * d.dst_row + c) =
          gf4{x[0], x[1], x[2], x[3]};
    }
  }
  // chains of three or more entries and rows reaching past their allocation
  // (rare): short chains at once, the rest element by element, then the
  // same resets
#pragma unroll
  for (int j = 0; j < RMW_NE; ++j) {
    if (r[j] < 0 || (fast[j] && n2[j].x < 0)) continue;
    const int32_t e = (int32_t)(e0 + j);
    if (fast[j] && apply_short_chain<SDT, D128>(d, op, r[j], e, s[j], nx[j], n2[j], n_entries, hl)) continue;
    const int64_t de = d.dst_base + (int64_t)r[j] * d.dst_row;
    for (int64_t c = (int64_t)hl * 4; c < D; c += 128) {
      float x[4];
      rows_get4<KTIR_F32>(d.dst_ptr, de + c, c, D, d.dst_hi, x);
      apply_long_chain(d, op, e, s[j], nx[j], KTIR_F32, x, [&](int32_t sm, float* gg) {
        rows_get4<SDT>(d.src_ptr, d.src_base + (int64_t)sm * d.src_row + c, c, D, d.src_hi, gg);
      });
      rows_put4(d, de + c, c, x);
    }
    rmw_reset(d, r[j], e, nx[j], hl);
  }
}

// Every other form (other dtypes, strided columns, any D): the same records,
// element by element (16-byte accesses where the layout allows).
__global__ __launch_bounds__(256) void rmw_apply(const ktir_rmw_t d, int64_t n_entries) {
  const int64_t hw = ((int64_t)blockIdx.x * 256 + threadIdx.x) / 32;
  const int hl = threadIdx.x % 32;
  const int64_t e0 = hw * RMW_NE;
  if (e0 >= n_entries) return;
  const bool vec = d.dst_col == 1 && d.src_col == 1 && d.dst_dtype == KTIR_F32 &&
                   (d.src_dtype == KTIR_F16 || d.src_dtype == KTIR_F32) &&
                   (d.dst_base % 4 == 0) && (d.dst_row % 4 == 0) && (d.src_base % 4 == 0) && (d.src_row % 4 == 0);
  const int2* rec = (const int2*)d.rows;
  const int2* nxt = (const int2*)d.link;
#pragma unroll
  for (int j = 0; j < RMW_NE; ++j) {
    if (e0 + j >= n_entries) break;
    const int32_t e = (int32_t)(e0 + j);
    const int2 re = rec[e];
    const int32_t r = re.x;
    if (r < 0) continue;
    const int32_t s = re.y;
    const int2 nx = nxt[e].x < n_entries ? nxt[e] : make_int2(-1, -1);
    const int64_t de = d.dst_base + (int64_t)r * d.dst_row;
    for (int64_t c = (int64_t)hl * 4; c < d.D; c += 128) {
      float x[4];
      load4(d, true, de + c * d.dst_col, c, vec, x);
      apply_long_chain(d, d.op, e, s, nx, d.dt, x, [&](int32_t sm, float* gg) {
        load4(d, false, d.src_base + (int64_t)sm * d.src_row + c * d.src_col, c, vec, gg);
      });
      store4(d, de + c * d.dst_col, c, vec, x);
    }
    rmw_reset(d, r, e, nx, hl);
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
// file-scope device array: heads in a fixed region of RMW_NA_ROWS slots and
// successor slots (link, two words per entry) in a fixed region, both -1
// between calls, then the entry records (two words per entry) in a fixed
// region, so no call's records ever land in another call's heads or links.  In host code `scratch` names a host-side stand-in; its device
// address (one per device) comes from hipGetSymbolAddress, taken once per
// device by rmw_scratch_setup with that device current.
constexpr int64_t RMW_NA_ROWS = (int64_t)2 << 20;      // destination rows
constexpr int64_t RMW_NA_ENTRIES = (int64_t)1 << 20;   // n_inst * K
constexpr int64_t RMW_SCRATCH_WORDS = RMW_NA_ROWS + 4 * RMW_NA_ENTRIES;   // 24 MiB of int32: heads, links, records
constexpr int RMW_MAX_DEVICES = 64;
__device__ __align__(256) int32_t scratch[RMW_SCRATCH_WORDS];
static int32_t* g_scratch[RMW_MAX_DEVICES];

__global__ __launch_bounds__(256) void rmw_fill(int32_t* p, int64_t n, int32_t v) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = v;
}

// Called by ktir_init with `device` current: the device address of this
// device's copy of `scratch`, and every head and link slot set to -1 (they
// are all -1 between calls: each launch resets the ones it uses).
int ktir::rmw_scratch_setup(int device) {
  if (device < 0 || device >= RMW_MAX_DEVICES)
    return set_error(KTIR_E_UNSUPPORTED, "ktir_init: device %d beyond the %d the RMW scratch table covers", device,
                     RMW_MAX_DEVICES);
  if (g_scratch[device]) return KTIR_OK;
  int32_t* ptr = nullptr;
  KTIR_HIP_CHECK(hipGetSymbolAddress((void**)&ptr, HIP_SYMBOL(scratch)));
  hipLaunchKernelGGL(rmw_fill, dim3(1024), dim3(256), 0, stream(), ptr, RMW_NA_ROWS + 2 * RMW_NA_ENTRIES,
                     (int32_t)-1);
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
  w.rows = (uint64_t)(base + RMW_NA_ROWS + 2 * RMW_NA_ENTRIES);
  w.srcs = 0;
  return rmw_launch(&w);
}

extern "C" int ktir_launch_row_rmw(const ktir_rmw_t* d) {
  const int rc = rmw_check(d, "ktir_launch_row_rmw");
  if (rc != KTIR_OK) return rc;
  if (d->n_inst > 0 && (!d->head || !d->link || !d->rows))
    return set_error(KTIR_E_ARG, "ktir_launch_row_rmw: head, link and rows scratch must be given "
                                 "(head: n_rows int32 of -1; link: 2 * n_inst * K int32 of -1)");
  return rmw_launch(d);
}

static int rmw_launch(const ktir_rmw_t* d) {
  if (d->n_inst == 0) return KTIR_OK;
  const int t1 = d->K >= 256 ? 256 : (int)((d->K + 63) / 64 * 64);
  const size_t lds = (size_t)(2 * d->K + 2 * rmw_table_slots((int)d->K)) * sizeof(int32_t);
  hipLaunchKernelGGL(rmw_link, dim3((unsigned)d->n_inst), dim3(t1), lds, stream(), *d, device_error_flag());
  const int64_t total = d->n_inst * d->K;
  const int64_t blocks = (total + 8 * RMW_NE - 1) / (8 * RMW_NE);
  if (rmw_rows_form(d)) {
    const bool d128 = d->D == 128, add = d->op == KTIR_OP_ADDF;
    const dim3 g((unsigned)blocks), b(256);
    if (d->src_dtype == KTIR_F16) {
      if (add) {
        if (d128) hipLaunchKernelGGL((rmw_apply_rows<KTIR_F16, true, KTIR_OP_ADDF>), g, b, 0, stream(), *d, total);
        else hipLaunchKernelGGL((rmw_apply_rows<KTIR_F16, false, KTIR_OP_ADDF>), g, b, 0, stream(), *d, total);
      } else {
        if (d128) hipLaunchKernelGGL((rmw_apply_rows<KTIR_F16, true, -1>), g, b, 0, stream(), *d, total);
        else hipLaunchKernelGGL((rmw_apply_rows<KTIR_F16, false, -1>), g, b, 0, stream(), *d, total);
      }
    } else {
      if (add) {
        if (d128) hipLaunchKernelGGL((rmw_apply_rows<KTIR_F32, true, KTIR_OP_ADDF>), g, b, 0, stream(), *d, total);
        else hipLaunchKernelGGL((rmw_apply_rows<KTIR_F32, false, KTIR_OP_ADDF>), g, b, 0, stream(), *d, total);
      } else {
        if (d128) hipLaunchKernelGGL((rmw_apply_rows<KTIR_F32, true, -1>), g, b, 0, stream(), *d, total);
        else hipLaunchKernelGGL((rmw_apply_rows<KTIR_F32, false, -1>), g, b, 0, stream(), *d, total);
      }
    }
  } else {
    hipLaunchKernelGGL(rmw_apply, dim3((unsigned)blocks), dim3(256), 0, stream(), *d, total);
  }
  KTIR_HIP_CHECK(hipGetLastError());
  return KTIR_OK;
}
