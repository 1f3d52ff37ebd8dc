// Lane-tiled streaming kernel for flat programs: one simulated core's tile
// (a lane of the program's iteration space) is covered by whole workgroups,
// so the lane -- and with it every leaf's lane offset, read from an offset
// table when the lanes' tiles are not evenly spaced -- is uniform in a
// workgroup: scalar loads, no per-element dependent read before the data
// loads.  Covers what the map kernels (ktir_map.hip) do not: three or four
// inputs, or two stores (the two halves of a rotary embedding, several
// outputs of one expression).
//
// Registers: eight registers of four elements, selected by uniform branches
// on the run-time register number (TileRegs); each thread takes two
// 4-element chunks per step and issues all of both chunks' loads before it
// computes.  Semantics per element are those of the general
// interpreter (ktir_program_impl.h) through exec_val (ktir_regops.h).
#include "ktir_regops.h"

namespace ktir {

struct TileDims {
  FastDiv cpr;                     // 4-element chunks per row (inner / 4)
  FastDiv dim[KTIR_MAX_DIMS];      // extents of the outer dims of one lane
  FastDiv bpl;                     // workgroups per lane
  uint32_t chunks;                 // chunks per lane
};

constexpr int TILE_U = 2;          // chunks per thread per step

typedef float tf4 __attribute__((ext_vector_type(4)));
typedef uint32_t tu2 __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ void load4(const ktir_leaf_t& L, int64_t e0, bool bcast, float (&out)[4]) {
  if (bcast) {
    const float v = (e0 >= L.lo && e0 < L.hi) ? load_elem(L.ptr, e0, DT) : 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = v;
    return;
  }
  if (e0 >= L.lo && e0 + 4 <= L.hi) {
    if (DT == KTIR_F32) {
      const tf4 w = *(const KTIR_G(tf4)*)((const KTIR_G(float)*)L.ptr + e0);
      out[0] = w[0]; out[1] = w[1]; out[2] = w[2]; out[3] = w[3];
    } else {
      const tu2 w = *(const KTIR_G(tu2)*)((const KTIR_G(uint16_t)*)L.ptr + e0);
      const uint32_t u[2] = {w[0], w[1]};
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        if (DT == KTIR_BF16) {
          out[2 * i] = __uint_as_float(u[i] << 16);
          out[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
        } else {
          out[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[i] & 0xffffu));
          out[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u[i] >> 16));
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t e = e0 + i;
    out[i] = (e >= L.lo && e < L.hi) ? load_elem(L.ptr, e, DT) : 0.f;
  }
}

template <int DT>
__device__ __forceinline__ void store4(const ktir_leaf_t& L, int64_t e0, const float (&v)[4]) {
  if (e0 >= L.lo && e0 + 4 <= L.hi) {
    if (DT == KTIR_F32) {
      *(KTIR_G(tf4)*)((KTIR_G(float)*)L.ptr + e0) = tf4{v[0], v[1], v[2], v[3]};
    } else {
      uint32_t u[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        if (DT == KTIR_BF16)
          u[i] = (__float_as_uint(round_bf16(v[2 * i])) >> 16) | (__float_as_uint(round_bf16(v[2 * i + 1])) & 0xffff0000u);
        else
          u[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * i]) |
                 ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * i + 1]) << 16);
      }
      *(KTIR_G(tu2)*)((KTIR_G(uint16_t)*)L.ptr + e0) = tu2{u[0], u[1]};
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t e = e0 + i;
    if (e >= L.lo && e < L.hi) store_elem(L.ptr, e, DT, v[i]);
  }
}

// element offset (before the lane offset) of chunk q of a lane in a leaf
__device__ __forceinline__ int64_t tile_off(const ktir_leaf_t& L, int nd, const TileDims& T, uint32_t q) {
  const uint32_t row = fdiv(q, T.cpr);
  int64_t o = L.strides[nd - 1] == 0 ? 0 : (int64_t)(q - row * T.cpr.d) * 4 * L.strides[nd - 1];
  uint32_t t = row;
#pragma unroll
  for (int d = KTIR_MAX_DIMS - 2; d >= 0; --d) {
    if (d < nd - 1) {
      const uint32_t qq = fdiv(t, T.dim[d]);
      o += (int64_t)(t - qq * T.dim[d].d) * L.strides[d];
      t = qq;
    }
  }
  return o;
}

// Eight registers of four elements selected by a uniform branch on the
// (uniform) register number.  The empty volatile asm in every case keeps
// the compiler from folding the branches back into an indexed access
// (indexed register moves or scratch) or a select chain: an access costs a
// few scalar instructions and four moves.
struct TileRegs {
  tf4 r[8];
  __device__ __forceinline__ void get(int i, float (&o)[4]) const {
    tf4 t;
    switch (i) {
#define KTIR_TR_GET(k) case k: t = r[k]; __asm__ volatile("" : "+v"(t)); break;
      KTIR_TR_GET(0) KTIR_TR_GET(1) KTIR_TR_GET(2) KTIR_TR_GET(3)
      KTIR_TR_GET(4) KTIR_TR_GET(5) KTIR_TR_GET(6) default: KTIR_TR_GET(7)
#undef KTIR_TR_GET
    }
    o[0] = t[0]; o[1] = t[1]; o[2] = t[2]; o[3] = t[3];
  }
  __device__ __forceinline__ void set(int i, const float (&v)[4]) {
    tf4 t = {v[0], v[1], v[2], v[3]};
    switch (i) {
#define KTIR_TR_SET(k) case k: __asm__ volatile("" : "+v"(t)); r[k] = t; break;
      KTIR_TR_SET(0) KTIR_TR_SET(1) KTIR_TR_SET(2) KTIR_TR_SET(3)
      KTIR_TR_SET(4) KTIR_TR_SET(5) KTIR_TR_SET(6) default: KTIR_TR_SET(7)
#undef KTIR_TR_SET
    }
  }
};

template <int DI, int DO, int NIN>
__global__ __launch_bounds__(256) void prog_tile(const ktir_prog_t P, const TileDims T) {
  const int nd = P.ndim;
  const uint32_t lane = fdiv(blockIdx.x, T.bpl);
  const uint32_t blk = blockIdx.x - lane * T.bpl.d;
  int64_t lo[NIN];
  bool bc[NIN];
#pragma unroll
  for (int k = 0; k < NIN; ++k) {
    const ktir_leaf_t& L = P.leaves[P.pf_leaf[k]];
    lo[k] = lane_offset(L, lane);
    bc[k] = L.strides[nd - 1] == 0;
  }
  float in[TILE_U][NIN][4];
  uint32_t q[TILE_U];
#pragma unroll
  for (int u = 0; u < TILE_U; ++u) {
    q[u] = (blk * TILE_U + u) * 256 + threadIdx.x;
    if (q[u] >= T.chunks) continue;
#pragma unroll
    for (int k = 0; k < NIN; ++k) {
      const ktir_leaf_t& L = P.leaves[P.pf_leaf[k]];
      load4<DI>(L, lo[k] + tile_off(L, nd, T, q[u]), bc[k], in[u][k]);
    }
  }
#pragma unroll
  for (int u = 0; u < TILE_U; ++u) {
    if (q[u] >= T.chunks) continue;
    TileRegs R;
#pragma unroll
    for (int k = 0; k < NIN; ++k) R.set(k, in[u][k]);
    for (int pc = 0; pc < P.n_instr; ++pc) {
      const ktir_instr_t ins = P.instr[pc];
      float a[4], b[4], c[4], v[4];
      R.get(ins.a, a);
      if (ins.op == KTIR_OP_ST) {
        const ktir_leaf_t& L = P.leaves[ins.aux];
        store4<DO>(L, lane_offset(L, lane) + tile_off(L, nd, T, q[u]), a);
        continue;
      }
      R.get(ins.b, b);
      const int op = ins.op, dt = ins.dt;
      switch (op) {
#define KTIR_T4(expr)                                 \
  _Pragma("unroll") for (int e = 0; e < 4; ++e) {     \
    const float x = a[e], y = b[e];                   \
    (void)y;                                          \
    v[e] = (expr);                                    \
  }                                                   \
  break;
        case KTIR_OP_ADDF: KTIR_T4(round_to(__fadd_rn(x, y), dt))
        case KTIR_OP_SUBF: KTIR_T4(round_to(__fsub_rn(x, y), dt))
        case KTIR_OP_MULF: KTIR_T4(round_to(mul_keep(x, y), dt))
        case KTIR_OP_DIVF: KTIR_T4(round_to(__fdiv_rn(x, y), dt))
        case KTIR_OP_EXP: KTIR_T4(round_to(expf(x), dt))
#undef KTIR_T4
        default: {
          const bool third = op == KTIR_OP_SELECT || op == KTIR_OP_FMA;
          if (third) R.get(ins.c, c);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = exec_val(P, ins, a[e], b[e], third ? c[e] : 0.f, lane);
        }
      }
      R.set(ins.dst, v);
    }
  }
}

template <int DI, int DO>
static void launch_tile(const ktir_prog_t& Q, const TileDims& T, uint32_t blocks) {
  switch (Q.n_pf) {
    case 1: hipLaunchKernelGGL((prog_tile<DI, DO, 1>), dim3(blocks), dim3(256), 0, stream(), Q, T); break;
    case 2: hipLaunchKernelGGL((prog_tile<DI, DO, 2>), dim3(blocks), dim3(256), 0, stream(), Q, T); break;
    case 3: hipLaunchKernelGGL((prog_tile<DI, DO, 3>), dim3(blocks), dim3(256), 0, stream(), Q, T); break;
    default: hipLaunchKernelGGL((prog_tile<DI, DO, 4>), dim3(blocks), dim3(256), 0, stream(), Q, T); break;
  }
}

// Launch `Q` through prog_tile if it has the form: a flat program whose
// loads are all prefetched (1 to 4 inputs of one float dtype, inner stride
// 1 on 4-aligned chunks or 0), register ops only, one or two stores to
// leaves of one float dtype (inner stride 1, 4-aligned), the last
// instruction a store; at least 512 elements per lane.  The one-store,
// one- and two-input programs stay with the map kernels.
bool try_launch_tile(const ktir_prog_t& Q, int64_t lanes, int64_t per_lane, int64_t inner) {
  if (Q.mode != 0 || Q.n_pf < 1 || Q.n_pf > 4 || Q.n_instr < 1 || inner % 4 || per_lane < 512) return false;
  if (Q.instr[Q.n_instr - 1].op != KTIR_OP_ST) return false;
  const int nd = Q.ndim;
  int n_st = 0, dout = -1;
  for (int i = 0; i < Q.n_instr; ++i) {
    const ktir_instr_t& in = Q.instr[i];
    if (in.dst >= 8 || in.a >= 8 || in.b >= 8 || in.c >= 8) return false;
    if (in.op == KTIR_OP_ST) {
      const ktir_leaf_t& L = Q.leaves[in.aux];
      if (L.offsets || L.winner || L.strides[nd - 1] != 1 || !(L.flags & KTIR_LEAF_VEC)) return false;
      if (dout >= 0 && L.dtype != dout) return false;
      dout = L.dtype;
      ++n_st;
      continue;
    }
    if (in.op == KTIR_OP_LD || in.op == KTIR_OP_IDX || !simple_op(in.op)) return false;
  }
  if (n_st > 2 || (Q.n_pf <= 2 && n_st < 2)) return false;
  const int din = Q.leaves[Q.pf_leaf[0]].dtype;
  for (int k = 0; k < Q.n_pf; ++k) {
    const ktir_leaf_t& L = Q.leaves[Q.pf_leaf[k]];
    const bool in_ok = (L.strides[nd - 1] == 1 && (L.flags & KTIR_LEAF_VEC)) || L.strides[nd - 1] == 0;
    if (L.offsets || L.winner || !in_ok || L.dtype != din) return false;
  }
  const int64_t chunks = per_lane / 4;
  const int64_t bpl = (chunks + 256 * TILE_U - 1) / (256 * TILE_U);
  if (chunks >= (int64_t)0x7fffffff || lanes * bpl >= (int64_t)0x7fffffff) return false;
  TileDims T;
  T.cpr = make_fastdiv((uint32_t)(inner / 4));
  for (int d = 0; d < KTIR_MAX_DIMS; ++d) T.dim[d] = make_fastdiv(d < nd - 1 ? (uint32_t)Q.shape[d] : 1);
  T.bpl = make_fastdiv((uint32_t)bpl);
  T.chunks = (uint32_t)chunks;
  const uint32_t blocks = (uint32_t)(lanes * bpl);
#define KTIR_TILE_OUT(DI)                                                      \
  switch (dout) {                                                              \
    case KTIR_F16: launch_tile<DI, KTIR_F16>(Q, T, blocks); return true;       \
    case KTIR_BF16: launch_tile<DI, KTIR_BF16>(Q, T, blocks); return true;     \
    case KTIR_F32: launch_tile<DI, KTIR_F32>(Q, T, blocks); return true;       \
  }                                                                            \
  return false;
  switch (din) {
    case KTIR_F16: KTIR_TILE_OUT(KTIR_F16)
    case KTIR_BF16: KTIR_TILE_OUT(KTIR_BF16)
    case KTIR_F32: KTIR_TILE_OUT(KTIR_F32)
  }
#undef KTIR_TILE_OUT
  return false;
}

}  // namespace ktir
