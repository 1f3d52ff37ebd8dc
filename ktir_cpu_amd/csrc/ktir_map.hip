// Streaming kernels for the most common fused program: one or two strided
// inputs (unit or zero inner stride), a chain of register ops, one strided
// output (an elementwise map, a copy, a cast, a broadcast).  Leaf and output dtypes are template
// parameters, so the memory path is straight-line code: each thread moves
// 8-element chunks with 16-byte accesses and has all its chunks' loads in
// flight before it computes.  The register ops still come from the
// program, evaluated per element with the same semantics as the general
// interpreter (ktir_program.hip).
#include "ktir_regops.h"

namespace ktir {

typedef float mf4 __attribute__((ext_vector_type(4)));
typedef uint32_t mu4 __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ void load8(const ktir_leaf_t& L, int64_t e0, float* out, bool bcast) {
  if (bcast) {   // inner stride 0: one element for the whole chunk
    const float v = (e0 >= L.lo && e0 < L.hi) ? load_elem(L.ptr, e0, DT) : 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = v;
    return;
  }
  if (e0 >= L.lo && e0 + 8 <= L.hi) {
    if (DT == KTIR_F16) {
      const uint4 w = __builtin_bit_cast(uint4, *(const KTIR_G(mu4)*)((const KTIR_G(uint16_t)*)L.ptr + e0));
      const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        out[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[i] & 0xffffu));
        out[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[i] >> 16));
      }
    } else if (DT == KTIR_BF16) {
      const uint4 w = __builtin_bit_cast(uint4, *(const KTIR_G(mu4)*)((const KTIR_G(uint16_t)*)L.ptr + e0));
      const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        out[2 * i] = __uint_as_float(u[i] << 16);
        out[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
      }
    } else {
      const mf4 w0 = *(const KTIR_G(mf4)*)((const KTIR_G(float)*)L.ptr + e0);
      const mf4 w1 = *(const KTIR_G(mf4)*)((const KTIR_G(float)*)L.ptr + e0 + 4);
      out[0] = w0[0]; out[1] = w0[1]; out[2] = w0[2]; out[3] = w0[3];
      out[4] = w1[0]; out[5] = w1[1]; out[6] = w1[2]; out[7] = w1[3];
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int64_t e = e0 + i;
    out[i] = (e >= L.lo && e < L.hi) ? load_elem(L.ptr, e, DT) : 0.f;
  }
}

template <int DT>
// 16-bit results go out with non-temporal (streaming) stores, which measured
// 6.1 against 5.0 TB/s for a 64 Mi-element f16 add; f32 results keep plain
// stores, which measured faster for an f32 copy (5.5 against 5.0 TB/s)
__device__ __forceinline__ void store8(const ktir_leaf_t& L, int64_t e0, const float* v) {
  if (e0 >= L.lo && e0 + 8 <= L.hi) {
    if (DT == KTIR_F16) {
      uint32_t u[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        u[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * i]) |
               ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * i + 1]) << 16);
      __builtin_nontemporal_store(mu4{u[0], u[1], u[2], u[3]}, (KTIR_G(mu4)*)((KTIR_G(uint16_t)*)L.ptr + e0));
    } else if (DT == KTIR_BF16) {
      uint32_t u[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        u[i] = (__float_as_uint(round_bf16(v[2 * i])) >> 16) | (__float_as_uint(round_bf16(v[2 * i + 1])) & 0xffff0000u);
      __builtin_nontemporal_store(mu4{u[0], u[1], u[2], u[3]}, (KTIR_G(mu4)*)((KTIR_G(uint16_t)*)L.ptr + e0));
    } else {
      *(KTIR_G(mf4)*)((KTIR_G(float)*)L.ptr + e0) = mf4{v[0], v[1], v[2], v[3]};
      *(KTIR_G(mf4)*)((KTIR_G(float)*)L.ptr + e0 + 4) = mf4{v[4], v[5], v[6], v[7]};
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int64_t e = e0 + i;
    if (e >= L.lo && e < L.hi) store_elem(L.ptr, e, DT, v[i]);
  }
}

// Four named registers selected by the (uniform) register number: no array,
// so nothing is spilled to scratch.
struct Reg4 {
  float r0, r1, r2, r3;
  __device__ __forceinline__ float get(int i) const { return i == 0 ? r0 : (i == 1 ? r1 : (i == 2 ? r2 : r3)); }
  __device__ __forceinline__ void set(int i, float v) {
    r0 = i == 0 ? v : r0;
    r1 = i == 1 ? v : r1;
    r2 = i == 2 ? v : r2;
    r3 = i == 3 ? v : r3;
  }
};

template <class RG>
__device__ __forceinline__ void exec_reg(const ktir_prog_t& P, const ktir_instr_t in, RG& R, int64_t lane) {
  const bool third = in.op == KTIR_OP_SELECT || in.op == KTIR_OP_FMA;
  R.set(in.dst, exec_val(P, in, R.get(in.a), R.get(in.b), third ? R.get(in.c) : 0.f, lane));
}

// One instruction over the 8 elements of a chunk; the opcode switch is
// taken once (it is uniform), the common ops run as straight loops.
template <class RG>
__device__ __forceinline__ void exec8(const ktir_prog_t& P, const ktir_instr_t in, RG (&R)[8], int64_t lane) {
  const int op = in.op, dt = in.dt;
#define EACH(expr)                                                          \
  _Pragma("unroll") for (int e = 0; e < 8; ++e) {                           \
    const float x = R[e].get(in.a), y = R[e].get(in.b);                     \
    (void)x; (void)y;                                                       \
    R[e].set(in.dst, (expr));                                               \
  }                                                                         \
  return;
  switch (op) {
    case KTIR_OP_ADDF: EACH(round_to(__fadd_rn(x, y), dt))
    case KTIR_OP_SUBF: EACH(round_to(__fsub_rn(x, y), dt))
    case KTIR_OP_MULF: EACH(round_to(mul_keep(x, y), dt))
    case KTIR_OP_DIVF: EACH(round_to(__fdiv_rn(x, y), dt))
    case KTIR_OP_CAST: EACH(cast_val(x, in.aux, dt))
    case KTIR_OP_CONST: EACH(__int_as_float(in.imm))
    case KTIR_OP_EXP: EACH(round_to(expf(x), dt))
    default: break;
  }
#undef EACH
#pragma unroll
  for (int e = 0; e < 8; ++e) exec_reg(P, in, R[e], lane);
}

// element offsets of chunk vid in the two inputs and the output
struct MapOffs {
  int64_t a, b, o, lane;
};

__device__ __forceinline__ MapOffs map_offsets(const ktir_prog_t& P, const FlatDivs& D, const ktir_leaf_t& LA,
                                               const ktir_leaf_t& LB, const ktir_leaf_t& LO, bool bca, bool bcb,
                                               uint32_t vid) {
  const int nd = P.ndim;
  uint32_t c[KTIR_MAX_DIMS] = {0, 0, 0, 0};
  const uint32_t row = fdiv(vid, D.nvi);
  const int64_t col = (int64_t)(vid - row * D.nvi.d) * 8;
  uint32_t t = row;
#pragma unroll
  for (int d = KTIR_MAX_DIMS - 2; d >= 0; --d) {
    if (d < nd - 1) {
      uint32_t q = fdiv(t, D.dim[d]);
      c[d] = t - q * D.dim[d].d;
      t = q;
    }
  }
  // inner strides are 1 (or 0 for a broadcast input) on this path (checked at launch)
  MapOffs m;
  m.a = lane_offset(LA, t) + (bca ? 0 : col);
  m.b = lane_offset(LB, t) + (bcb ? 0 : col);
  m.o = lane_offset(LO, t) + col;
#pragma unroll
  for (int d = 0; d < KTIR_MAX_DIMS - 1; ++d) {
    if (d < nd - 1) {
      m.a += (int64_t)c[d] * LA.strides[d];
      m.b += (int64_t)c[d] * LB.strides[d];
      m.o += (int64_t)c[d] * LO.strides[d];
    }
  }
  m.lane = t;
  return m;
}

// r = a OP b (or b OP a) over a chunk; the result rounded to dt unless the
// output store rounds to the same type
template <int DO>
__device__ __forceinline__ void map_binop(int op, int dt, bool swap, const float (&a)[8], const float (&b)[8],
                                          float (&r)[8]) {
  const bool round = dt != DO && dt != KTIR_F32;
  float p[8], q[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float ae = a[e], be = b[e];
    p[e] = swap ? be : ae;
    q[e] = swap ? ae : be;
  }
#define MB(expr)                                                 \
  _Pragma("unroll") for (int e = 0; e < 8; ++e) {                \
    const float x = p[e], y = q[e];                              \
    const float v = (expr);                                      \
    r[e] = round ? round_to(v, dt) : v;                          \
  }                                                              \
  return;
  switch (op) {
    case KTIR_OP_ADDF: MB(__fadd_rn(x, y))
    case KTIR_OP_SUBF: MB(__fsub_rn(x, y))
    case KTIR_OP_MULF: MB(mul_keep(x, y))
    case KTIR_OP_DIVF: MB(__fdiv_rn(x, y))
  }
#undef MB
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = binop_f_simple(op, dt, p[e], q[e]);
}

// A chunk's 8 elements as raw 16-byte words (one for 16-bit types, two for f32)
template <int DT>
struct Raw8 {
  mu4 w[DT == KTIR_F32 ? 2 : 1];
};

template <int DT>
__device__ __forceinline__ Raw8<DT> raw_load(uint64_t ptr, int64_t e0) {
  Raw8<DT> r;
  const KTIR_G(mu4)* p = (const KTIR_G(mu4)*)((const KTIR_G(uint8_t)*)ptr + e0 * (DT == KTIR_F32 ? 4 : 2));
  r.w[0] = p[0];
  if (DT == KTIR_F32) r.w[DT == KTIR_F32 ? 1 : 0] = p[1];
  return r;
}

template <int DT>
__device__ __forceinline__ void raw_decode(const Raw8<DT>& r, float (&out)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (DT == KTIR_F32) {
      out[i] = __uint_as_float(r.w[0][i]);
      out[4 + i] = __uint_as_float(r.w[DT == KTIR_F32 ? 1 : 0][i]);
    } else if (DT == KTIR_BF16) {
      out[2 * i] = __uint_as_float(r.w[0][i] << 16);
      out[2 * i + 1] = __uint_as_float(r.w[0][i] & 0xffff0000u);
    } else {
      out[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.w[0][i] & 0xffffu));
      out[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.w[0][i] >> 16));
    }
  }
}

// compute and store one chunk
template <int DO, int NIN>
__device__ __forceinline__ void map_chunk(const ktir_prog_t& P, const ktir_leaf_t& LO, int fast, int n_ops, int out_reg,
                                          const MapOffs& m, const float (&a)[8], const float (&b)[8]) {
  float out[8];
  if (NIN == 2 && fast >= 0) {
    map_binop<DO>(fast & 0xff, fast >> 16, (fast >> 8) & 1, a, b, out);
  } else {
    Reg4 R[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) R[e] = Reg4{a[e], NIN == 2 ? b[e] : 0.f, 0.f, 0.f};
    for (int pc = 0; pc < n_ops; ++pc) exec8(P, P.instr[pc], R, m.lane);
#pragma unroll
    for (int e = 0; e < 8; ++e) out[e] = R[e].get(out_reg);
  }
  store8<DO>(LO, m.o, out);
}

// Two chunks per thread per step (256 chunks apart), both chunks' loads
// issued before any compute.  `fast` >= 0: the program is one float binary
// op of the two inputs whose result is stored (op | swap << 8 | dt << 16),
// applied directly.
template <int DA, int DB, int DO, int NIN>
__global__ __launch_bounds__(256) void prog_map(const ktir_prog_t P, const FlatDivs D, uint32_t total, int st_leaf,
                                                int fast) {
  const ktir_leaf_t& LA = P.leaves[P.pf_leaf[0]];
  const ktir_leaf_t& LB = P.leaves[NIN == 2 ? P.pf_leaf[1] : P.pf_leaf[0]];
  const ktir_leaf_t& LO = P.leaves[st_leaf];
  const int nd = P.ndim;
  const int n_ops = P.n_instr - 1;
  const int out_reg = P.instr[n_ops].a;
  const bool bca = LA.strides[nd - 1] == 0, bcb = LB.strides[nd - 1] == 0;
  const uint32_t step = gridDim.x * 512;
  for (uint32_t v0 = blockIdx.x * 512 + threadIdx.x; v0 < total; v0 += step) {
    const uint32_t v1 = v0 + 256;
    const bool on1 = v1 < total;
    float a0[8], b0[8], a1[8], b1[8];
    const MapOffs m0 = map_offsets(P, D, LA, LB, LO, bca, bcb, v0);
    const MapOffs m1 = map_offsets(P, D, LA, LB, LO, bca, bcb, on1 ? v1 : v0);
    // one uniform test: every chunk of the wavefront inside its allocations
    // (then all raw loads are issued before anything is decoded)
    bool inb = on1 && !bca && (NIN == 1 || !bcb);
    inb = inb && m0.a >= LA.lo && m0.a + 8 <= LA.hi && m1.a >= LA.lo && m1.a + 8 <= LA.hi;
    if (NIN == 2) inb = inb && m0.b >= LB.lo && m0.b + 8 <= LB.hi && m1.b >= LB.lo && m1.b + 8 <= LB.hi;
    if (__all(inb)) {
      const Raw8<DA> ra0 = raw_load<DA>(LA.ptr, m0.a), ra1 = raw_load<DA>(LA.ptr, m1.a);
      Raw8<DB> rb0, rb1;
      if (NIN == 2) {
        rb0 = raw_load<DB>(LB.ptr, m0.b);
        rb1 = raw_load<DB>(LB.ptr, m1.b);
      }
      raw_decode<DA>(ra0, a0);
      raw_decode<DA>(ra1, a1);
      if (NIN == 2) {
        raw_decode<DB>(rb0, b0);
        raw_decode<DB>(rb1, b1);
      }
    } else {
      load8<DA>(LA, m0.a, a0, bca);
      if (NIN == 2) load8<DB>(LB, m0.b, b0, bcb);
      if (on1) {
        load8<DA>(LA, m1.a, a1, bca);
        if (NIN == 2) load8<DB>(LB, m1.b, b1, bcb);
      }
    }
    map_chunk<DO, NIN>(P, LO, fast, n_ops, out_reg, m0, a0, b0);
    if (on1) map_chunk<DO, NIN>(P, LO, fast, n_ops, out_reg, m1, a1, b1);
  }
}

// Three or four inputs of one dtype DI, four registers (the host's register
// allocation reuses an input's register once it is dead, so a RoPE half
// (x1 cos - x2 sin) fits), one store: the form of prog_map with NIN inputs,
// every array indexed by constants only (named per-chunk values).
struct MapOffs4 {
  int64_t in[4], o, lane;
};

__device__ __forceinline__ MapOffs4 map_offsets4(const ktir_prog_t& P, const FlatDivs& D, int nin,
                                                 const ktir_leaf_t& LO, uint32_t vid) {
  const int nd = P.ndim;
  uint32_t c[KTIR_MAX_DIMS] = {0, 0, 0, 0};
  const uint32_t row = fdiv(vid, D.nvi);
  const int64_t col = (int64_t)(vid - row * D.nvi.d) * 8;
  uint32_t t = row;
#pragma unroll
  for (int d = KTIR_MAX_DIMS - 2; d >= 0; --d) {
    if (d < nd - 1) {
      const uint32_t q = fdiv(t, D.dim[d]);
      c[d] = t - q * D.dim[d].d;
      t = q;
    }
  }
  MapOffs4 m;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const ktir_leaf_t& L = P.leaves[P.pf_leaf[k < nin ? k : nin - 1]];   // a fourth slot repeats the last input
    int64_t o = lane_offset(L, t) + (L.strides[nd - 1] == 0 ? 0 : col);
#pragma unroll
    for (int d = 0; d < KTIR_MAX_DIMS - 1; ++d)
      if (d < nd - 1) o += (int64_t)c[d] * L.strides[d];
    m.in[k] = o;
  }
  m.o = lane_offset(LO, t) + col;
#pragma unroll
  for (int d = 0; d < KTIR_MAX_DIMS - 1; ++d)
    if (d < nd - 1) m.o += (int64_t)c[d] * LO.strides[d];
  m.lane = t;
  return m;
}

template <int DI, int NIN>
__device__ __forceinline__ void map_run4(const ktir_prog_t& P, int n_ops, int out_reg, int64_t lane, const float (&x0)[8],
                                         const float (&x1)[8], const float (&x2)[8], const float (&x3)[8], float (&out)[8]) {
  Reg4 R[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) R[e] = Reg4{x0[e], x1[e], x2[e], NIN > 3 ? x3[e] : 0.f};
  for (int pc = 0; pc < n_ops; ++pc) exec8(P, P.instr[pc], R, lane);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = R[e].get(out_reg);
}

template <int DI, int DO, int NIN>
__global__ __launch_bounds__(256) void prog_map_n(const ktir_prog_t P, const FlatDivs D, uint32_t total, int st_leaf) {
  const ktir_leaf_t& LO = P.leaves[st_leaf];
  const ktir_leaf_t& L0 = P.leaves[P.pf_leaf[0]];
  const ktir_leaf_t& L1 = P.leaves[P.pf_leaf[1]];
  const ktir_leaf_t& L2 = P.leaves[P.pf_leaf[2]];
  const ktir_leaf_t& L3 = P.leaves[P.pf_leaf[NIN > 3 ? 3 : 2]];
  const int nd = P.ndim;
  const int n_ops = P.n_instr - 1;
  const int out_reg = P.instr[n_ops].a;
  const bool bc0 = L0.strides[nd - 1] == 0, bc1 = L1.strides[nd - 1] == 0, bc2 = L2.strides[nd - 1] == 0,
             bc3 = L3.strides[nd - 1] == 0;
  const uint32_t step = gridDim.x * 512;
  for (uint32_t v0 = blockIdx.x * 512 + threadIdx.x; v0 < total; v0 += step) {
    const bool on1 = v0 + 256 < total;
    const MapOffs4 m0 = map_offsets4(P, D, NIN, LO, v0);
    const MapOffs4 m1 = map_offsets4(P, D, NIN, LO, on1 ? v0 + 256 : v0);
    float a0[8], b0[8], c0[8], d0[8], a1[8], b1[8], c1[8], d1[8];
    auto in = [](const ktir_leaf_t& L, int64_t o) { return o >= L.lo && o + 8 <= L.hi; };
    bool inb = on1 && !bc0 && !bc1 && !bc2 && !bc3;
    inb = inb && in(L0, m0.in[0]) && in(L0, m1.in[0]) && in(L1, m0.in[1]) && in(L1, m1.in[1]) &&
          in(L2, m0.in[2]) && in(L2, m1.in[2]) && in(L3, m0.in[3]) && in(L3, m1.in[3]);
    if (__all(inb)) {
      const Raw8<DI> r00 = raw_load<DI>(L0.ptr, m0.in[0]), r01 = raw_load<DI>(L1.ptr, m0.in[1]),
                     r02 = raw_load<DI>(L2.ptr, m0.in[2]), r03 = raw_load<DI>(L3.ptr, m0.in[3]);
      const Raw8<DI> r10 = raw_load<DI>(L0.ptr, m1.in[0]), r11 = raw_load<DI>(L1.ptr, m1.in[1]),
                     r12 = raw_load<DI>(L2.ptr, m1.in[2]), r13 = raw_load<DI>(L3.ptr, m1.in[3]);
      raw_decode<DI>(r00, a0); raw_decode<DI>(r01, b0); raw_decode<DI>(r02, c0); raw_decode<DI>(r03, d0);
      raw_decode<DI>(r10, a1); raw_decode<DI>(r11, b1); raw_decode<DI>(r12, c1); raw_decode<DI>(r13, d1);
    } else {
      load8<DI>(L0, m0.in[0], a0, bc0); load8<DI>(L1, m0.in[1], b0, bc1);
      load8<DI>(L2, m0.in[2], c0, bc2); load8<DI>(L3, m0.in[3], d0, bc3);
      if (on1) {
        load8<DI>(L0, m1.in[0], a1, bc0); load8<DI>(L1, m1.in[1], b1, bc1);
        load8<DI>(L2, m1.in[2], c1, bc2); load8<DI>(L3, m1.in[3], d1, bc3);
      }
    }
    float out[8];
    map_run4<DI, NIN>(P, n_ops, out_reg, m0.lane, a0, b0, c0, d0, out);
    store8<DO>(LO, m0.o, out);
    if (on1) {
      map_run4<DI, NIN>(P, n_ops, out_reg, m1.lane, a1, b1, c1, d1, out);
      store8<DO>(LO, m1.o, out);
    }
  }
}

// The single-binary-op form in a kernel of its own (no interpreter, so few
// registers): MAP_BU chunks per thread per step, 256 chunks apart.  When the
// whole wavefront's chunks lie inside their allocations (one uniform test)
// all raw 16-byte loads are issued before anything is decoded; otherwise
// chunk by chunk with the per-element out-of-range rules.
constexpr int MAP_BU = 4;

template <int DA, int DB, int DO>
__global__ __launch_bounds__(256) void prog_map_bin(const ktir_prog_t P, const FlatDivs D, uint32_t total,
                                                    int st_leaf, int fast) {
  const ktir_leaf_t& LA = P.leaves[P.pf_leaf[0]];
  const ktir_leaf_t& LB = P.leaves[P.pf_leaf[1]];
  const ktir_leaf_t& LO = P.leaves[st_leaf];
  const int nd = P.ndim;
  const bool bca = LA.strides[nd - 1] == 0, bcb = LB.strides[nd - 1] == 0;
  const int op = fast & 0xff, dt = fast >> 16;
  const bool swap = (fast >> 8) & 1;
  const uint32_t step = gridDim.x * 256 * MAP_BU;
  for (uint32_t v0 = blockIdx.x * 256 * MAP_BU + threadIdx.x; v0 < total; v0 += step) {
    MapOffs m[MAP_BU];
    bool inb = !bca && !bcb;
#pragma unroll
    for (int u = 0; u < MAP_BU; ++u) {
      const uint32_t v = v0 + 256 * u;
      m[u] = map_offsets(P, D, LA, LB, LO, bca, bcb, v < total ? v : v0);
      inb = inb && v < total && m[u].a >= LA.lo && m[u].a + 8 <= LA.hi && m[u].b >= LB.lo && m[u].b + 8 <= LB.hi &&
            m[u].o >= LO.lo && m[u].o + 8 <= LO.hi;
    }
    if (__all(inb)) {
      Raw8<DA> ra[MAP_BU];
      Raw8<DB> rb[MAP_BU];
#pragma unroll
      for (int u = 0; u < MAP_BU; ++u) {
        ra[u] = raw_load<DA>(LA.ptr, m[u].a);
        rb[u] = raw_load<DB>(LB.ptr, m[u].b);
      }
#pragma unroll
      for (int u = 0; u < MAP_BU; ++u) {
        float a[8], b[8], out[8];
        raw_decode<DA>(ra[u], a);
        raw_decode<DB>(rb[u], b);
        map_binop<DO>(op, dt, swap, a, b, out);
        store8<DO>(LO, m[u].o, out);
      }
      continue;
    }
#pragma unroll
    for (int u = 0; u < MAP_BU; ++u) {
      if (v0 + 256 * u < total) {
        float a[8], b[8], out[8];
        load8<DA>(LA, m[u].a, a, bca);
        load8<DB>(LB, m[u].b, b, bcb);
        map_binop<DO>(op, dt, swap, a, b, out);
        store8<DO>(LO, m[u].o, out);
      }
    }
  }
}

template <int DA, int DB, int DO, int NIN>
static void launch_map(const ktir_prog_t& Q, const FlatDivs& D, uint32_t total, int st_leaf) {
  int64_t blocks = ((int64_t)total + 511) / 512;
  if (blocks > 1048576) blocks = 1048576;
  int fast = -1;
  if (NIN == 2 && Q.n_instr == 2) {
    const ktir_instr_t& x = Q.instr[0];
    const bool fop = x.op == KTIR_OP_ADDF || x.op == KTIR_OP_SUBF || x.op == KTIR_OP_MULF || x.op == KTIR_OP_DIVF ||
                     x.op == KTIR_OP_MAXIMUMF || x.op == KTIR_OP_MINIMUMF || x.op == KTIR_OP_MAXNUMF ||
                     x.op == KTIR_OP_MINNUMF;
    const bool fdt = x.dt == KTIR_F16 || x.dt == KTIR_BF16 || x.dt == KTIR_F32;
    if (fop && fdt && Q.instr[1].a == x.dst && ((x.a == 0 && x.b == 1) || (x.a == 1 && x.b == 0)))
      fast = x.op | ((x.a == 1) << 8) | (x.dt << 16);
  }
  if (fast >= 0) {
    int64_t nb = ((int64_t)total + 256 * MAP_BU - 1) / (256 * MAP_BU);
    if (nb > 1048576) nb = 1048576;
    hipLaunchKernelGGL((prog_map_bin<DA, DB, DO>), dim3((unsigned)nb), dim3(256), 0, stream(), Q, D, total, st_leaf,
                       fast);
    return;
  }
  hipLaunchKernelGGL((prog_map<DA, DB, DO, NIN>), dim3((unsigned)blocks), dim3(256), 0, stream(), Q, D, total,
                     st_leaf, fast);
}

template <int DA, int DB, int NIN>
static bool pick_out(int dout, const ktir_prog_t& Q, const FlatDivs& D, uint32_t total, int st) {
  switch (dout) {
    case KTIR_F16: launch_map<DA, DB, KTIR_F16, NIN>(Q, D, total, st); return true;
    case KTIR_BF16: launch_map<DA, DB, KTIR_BF16, NIN>(Q, D, total, st); return true;
    case KTIR_F32: launch_map<DA, DB, KTIR_F32, NIN>(Q, D, total, st); return true;
  }
  return false;
}

template <int DA, int NIN>
static bool pick_b(int db, int dout, const ktir_prog_t& Q, const FlatDivs& D, uint32_t total, int st) {
  if (NIN == 1) return pick_out<DA, DA, 1>(dout, Q, D, total, st);
  switch (db) {
    case KTIR_F16: return pick_out<DA, KTIR_F16, 2>(dout, Q, D, total, st);
    case KTIR_BF16: return pick_out<DA, KTIR_BF16, 2>(dout, Q, D, total, st);
    case KTIR_F32: return pick_out<DA, KTIR_F32, 2>(dout, Q, D, total, st);
  }
  return false;
}

template <int DI>
static bool pick_n(int dout, const ktir_prog_t& Q, const FlatDivs& D, uint32_t total, int st) {
  int64_t blocks = ((int64_t)total + 511) / 512;
  if (blocks > 1048576) blocks = 1048576;
  const dim3 g((unsigned)blocks), b(256);
#define KTIR_MAPN(DO)                                                                           \
  if (Q.n_pf == 3) hipLaunchKernelGGL((prog_map_n<DI, DO, 3>), g, b, 0, stream(), Q, D, total, st); \
  else hipLaunchKernelGGL((prog_map_n<DI, DO, 4>), g, b, 0, stream(), Q, D, total, st);           \
  return true;
  switch (dout) {
    case KTIR_F16: KTIR_MAPN(KTIR_F16)
    case KTIR_BF16: KTIR_MAPN(KTIR_BF16)
    case KTIR_F32: KTIR_MAPN(KTIR_F32)
  }
#undef KTIR_MAPN
  return false;
}

// Launch `Q` through a map kernel if it has the supported form.
bool try_launch_map(const ktir_prog_t& Q, int64_t rows, int64_t inner) {
  if (Q.mode != 0 || Q.n_pf < 1 || Q.n_pf > 4 || Q.n_instr < 1 || inner % 8) return false;
  const ktir_instr_t& st = Q.instr[Q.n_instr - 1];
  if (st.op != KTIR_OP_ST || st.a > 3) return false;
  for (int i = 0; i < Q.n_instr - 1; ++i) {
    const ktir_instr_t& in = Q.instr[i];
    const int op = in.op;
    if (op == KTIR_OP_LD || op == KTIR_OP_ST || op == KTIR_OP_IDX || !simple_op(op)) return false;
    if (in.dst > 3 || in.a > 3 || in.b > 3 || in.c > 3) return false;   // four registers
  }
  const int nd = Q.ndim;
  auto ok_leaf = [nd](const ktir_leaf_t& L, bool input) {
    const bool inner = (L.strides[nd - 1] == 1 && (L.flags & KTIR_LEAF_VEC8)) || (input && L.strides[nd - 1] == 0);
    return L.offsets == 0 && L.winner == 0 && inner &&
           (L.dtype == KTIR_F16 || L.dtype == KTIR_BF16 || L.dtype == KTIR_F32);
  };
  for (int k = 0; k < Q.n_pf; ++k)
    if (!ok_leaf(Q.leaves[Q.pf_leaf[k]], true)) return false;
  if (!ok_leaf(Q.leaves[st.aux], false)) return false;
  const int64_t chunks = rows * (inner / 8);
  if (chunks >= (int64_t)0x7fffffff || inner / 8 >= (int64_t)0x7fffffff) return false;
  FlatDivs D;
  D.nvi = make_fastdiv((uint32_t)(inner / 8));
  for (int d = 0; d < KTIR_MAX_DIMS; ++d) D.dim[d] = make_fastdiv(d < Q.ndim - 1 ? (uint32_t)Q.shape[d] : 1);
  D.rows_per_lane = 0;
  const int da = Q.leaves[Q.pf_leaf[0]].dtype;
  const int db = Q.n_pf == 2 ? Q.leaves[Q.pf_leaf[1]].dtype : da;
  const int dout = Q.leaves[st.aux].dtype;
  const uint32_t total = (uint32_t)chunks;
  if (Q.n_pf > 2) {
    for (int k = 1; k < Q.n_pf; ++k)
      if (Q.leaves[Q.pf_leaf[k]].dtype != da) return false;
    switch (da) {
      case KTIR_F16: return pick_n<KTIR_F16>(dout, Q, D, total, st.aux);
      case KTIR_BF16: return pick_n<KTIR_BF16>(dout, Q, D, total, st.aux);
      case KTIR_F32: return pick_n<KTIR_F32>(dout, Q, D, total, st.aux);
    }
    return false;
  }
  if (Q.n_pf == 1) {
    switch (da) {
      case KTIR_F16: return pick_b<KTIR_F16, 1>(db, dout, Q, D, total, st.aux);
      case KTIR_BF16: return pick_b<KTIR_BF16, 1>(db, dout, Q, D, total, st.aux);
      case KTIR_F32: return pick_b<KTIR_F32, 1>(db, dout, Q, D, total, st.aux);
    }
  } else {
    switch (da) {
      case KTIR_F16: return pick_b<KTIR_F16, 2>(db, dout, Q, D, total, st.aux);
      case KTIR_BF16: return pick_b<KTIR_BF16, 2>(db, dout, Q, D, total, st.aux);
      case KTIR_F32: return pick_b<KTIR_F32, 2>(db, dout, Q, D, total, st.aux);
    }
  }
  return false;
}

}  // namespace ktir
