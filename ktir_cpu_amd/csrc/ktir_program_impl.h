// Device-side pieces shared by the fused-program kernels: operator
// semantics, leaf access, the register interpreter, launch-time division.
#pragma once
#include "ktir_common.h"

namespace ktir {

// ---- scalar operator semantics (shared with the fold) ---------------------

__device__ __forceinline__ float py_fmod(float x, float y) {
  // NumPy float remainder: result takes the sign of the divisor.
  float r = fmodf(x, y);
  if (r != 0.f) {
    if ((y < 0.f) != (r < 0.f)) r += y;
  } else {
    r = copysignf(0.f, y);
  }
  return r;
}

__device__ __forceinline__ float erf_as(float x, int dt) {
  // Reference ops/math_ops.py:100-106 (Abramowitz & Stegun 7.1.26), evaluated
  // by NumPy in the tile dtype: every constant and intermediate is rounded to dt.
#define R(e) round_to((e), dt)
  float a = fabsf(x);
  float t = R(R(1.0f) / R(R(1.0f) + R(R(0.3275911f) * a)));
  float p = R(t * R(1.061405429f));
  p = R(t * R(R(-1.453152027f) + p));
  p = R(t * R(R(1.421413741f) + p));
  p = R(t * R(R(-0.284496736f) + p));
  p = R(t * R(R(0.254829592f) + p));
  float e = R(expf(R(R(-a) * a)));
  float s = (x > 0.f) ? 1.f : ((x < 0.f) ? -1.f : x);
  return R(s * R(R(1.0f) - R(p * e)));
#undef R
}

__device__ __forceinline__ float binop_f(int op, int dt, float x, float y) {
  float r;
  switch (op) {
    case KTIR_OP_ADDF: r = __fadd_rn(x, y); break;
    case KTIR_OP_SUBF: r = __fsub_rn(x, y); break;
    case KTIR_OP_MULF: r = mul_keep(x, y); break;
    case KTIR_OP_DIVF: r = __fdiv_rn(x, y); break;
    case KTIR_OP_REMF: r = py_fmod(x, y); break;
    case KTIR_OP_MAXIMUMF: r = (x != x || y != y) ? __int_as_float(0x7fc00000) : fmaxf(x, y); break;
    case KTIR_OP_MINIMUMF: r = (x != x || y != y) ? __int_as_float(0x7fc00000) : fminf(x, y); break;
    case KTIR_OP_MAXNUMF: r = fmaxf(x, y); break;
    case KTIR_OP_MINNUMF: r = fminf(x, y); break;
    case KTIR_OP_POWF: r = powf(x, y); break;
    default: r = 0.f;
  }
  return round_to(r, dt);
}

// Integer semantics are NumPy's on int32 tiles, as the reference computes
// them on an x86-64 host:
// * floor_divide / remainder by 0 give 0; INT_MIN // -1 wraps to INT_MIN;
// * divsi and ceildivsi go through float64 (trunc / ceil of a / b, exact for
//   int32 operands), and a float64 that int32 cannot hold (a / 0 = +-inf or
//   NaN, INT_MIN / -1 = 2^31) converts to INT_MIN, as cvttsd2si does;
// * remsi is a - divsi(a, b) * b in wrapping int32 (so remsi(a, 0) = a);
// * shifts by an amount outside [0, 32) give 0 (shli, shrui) or the sign
//   fill (shrsi).
__device__ __forceinline__ int neg_i(int x) { return (int)(0u - (uint32_t)x); }

__device__ __forceinline__ int floordiv_i(int x, int y) {
  if (y == 0) return 0;
  if (y == -1) return neg_i(x);
  int q = x / y;
  if ((x % y != 0) && ((x < 0) != (y < 0))) --q;
  return q;
}

__device__ __forceinline__ int truncdiv_i(int x, int y) {
  if (y == 0 || (y == -1 && x == INT_MIN)) return INT_MIN;
  return y == -1 ? -x : x / y;
}

__device__ __forceinline__ int truncrem_i(int x, int y) {
  return (int)((uint32_t)x - (uint32_t)truncdiv_i(x, y) * (uint32_t)y);
}

__device__ __forceinline__ int ceildiv_i(int x, int y) {
  if (y == 0 || (y == -1 && x == INT_MIN)) return INT_MIN;
  if (y == -1) return -x;
  int q = x / y;
  if ((x % y != 0) && ((x < 0) == (y < 0))) ++q;
  return q;
}

__device__ __forceinline__ int shl_i(int x, int y) { return (uint32_t)y < 32u ? (int)((uint32_t)x << y) : 0; }
__device__ __forceinline__ int shrs_i(int x, int y) { return (uint32_t)y < 32u ? x >> y : (x < 0 ? -1 : 0); }
__device__ __forceinline__ int shru_i(int x, int y) { return (uint32_t)y < 32u ? (int)((uint32_t)x >> y) : 0; }

__device__ __forceinline__ int binop_i(int op, int x, int y) {
  switch (op) {
    case KTIR_OP_ADDI: return (int)((uint32_t)x + (uint32_t)y);
    case KTIR_OP_SUBI: return (int)((uint32_t)x - (uint32_t)y);
    case KTIR_OP_MULI: return (int)((uint32_t)x * (uint32_t)y);
    case KTIR_OP_DIVSI: return truncdiv_i(x, y);
    case KTIR_OP_REMSI: return truncrem_i(x, y);
    case KTIR_OP_FLOORDIVSI: return floordiv_i(x, y);
    case KTIR_OP_FLOORREMSI: return y ? (int)((uint32_t)x - (uint32_t)floordiv_i(x, y) * (uint32_t)y) : 0;
    case KTIR_OP_CEILDIVSI: return ceildiv_i(x, y);
    case KTIR_OP_ANDI: return x & y;
    case KTIR_OP_ORI: return x | y;
    case KTIR_OP_XORI: return x ^ y;
    case KTIR_OP_SHLI: return shl_i(x, y);
    case KTIR_OP_SHRSI: return shrs_i(x, y);
    case KTIR_OP_SHRUI: return shru_i(x, y);
    case KTIR_OP_MAXSI: return x > y ? x : y;
    case KTIR_OP_MINSI: return x < y ? x : y;
  }
  return 0;
}

__device__ __forceinline__ float binop_any(int op, int dt, float x, float y) {
  if (op >= KTIR_OP_ADDI) return __int_as_float(binop_i(op, __float_as_int(x), __float_as_int(y)));
  return binop_f(op, dt, x, y);
}

__device__ __forceinline__ int cmp_f(int p, float x, float y) {
  bool un = (x != x) || (y != y);
  switch (p) {
    case KTIR_CMP_FALSE: return 0;
    case KTIR_CMP_OEQ: return x == y;
    case KTIR_CMP_OGT: return x > y;
    case KTIR_CMP_OGE: return x >= y;
    case KTIR_CMP_OLT: return x < y;
    case KTIR_CMP_OLE: return x <= y;
    case KTIR_CMP_ONE: return (x != y) && !un;
    case KTIR_CMP_ORD: return !un;
    case KTIR_CMP_UEQ: return (x == y) || un;
    case KTIR_CMP_UGT: return (x > y) || un;
    case KTIR_CMP_UGE: return (x >= y) || un;
    case KTIR_CMP_ULT: return (x < y) || un;
    case KTIR_CMP_ULE: return (x <= y) || un;
    case KTIR_CMP_UNE: return x != y;
    case KTIR_CMP_UNO: return un;
    case KTIR_CMP_TRUE: return 1;
  }
  return 0;
}

__device__ __forceinline__ int cmp_i(int p, int x, int y) {
  // The reference compares Python ints, so unsigned predicates compare values.
  switch (p) {
    case KTIR_CMP_EQ: return x == y;
    case KTIR_CMP_NE: return x != y;
    case KTIR_CMP_SLT: case KTIR_CMP_ULTI: return x < y;
    case KTIR_CMP_SLE: case KTIR_CMP_ULEI: return x <= y;
    case KTIR_CMP_SGT: case KTIR_CMP_UGTI: return x > y;
    case KTIR_CMP_SGE: case KTIR_CMP_UGEI: return x >= y;
  }
  return 0;
}

__device__ __forceinline__ float cast_val(float x, int src, int dst) {
  bool fs = is_float_dt(src), fd = is_float_dt(dst);
  if (fs && fd) return round_to(x, dst);
  if (fs) {
    if (dst == KTIR_I1) return __int_as_float(x != 0.f);
    // NaN and values int32 cannot hold convert to INT_MIN (NumPy's astype on
    // x86-64, cvttss2si): |x| < 2^31 (0x4f000000) on the magnitude bits, which
    // NaN and infinities fail, or x exactly -2^31
    const uint32_t u = __float_as_uint(x);
    int i = ((u & 0x7fffffffu) < 0x4f000000u) ? (int)x : INT_MIN;
    if (dst == KTIR_I8) i = (int8_t)i;
    if (dst == KTIR_I16) i = (int16_t)i;
    return __int_as_float(i);
  }
  int i = __float_as_int(x);
  if (fd) return round_to((float)i, dst);
  if (dst == KTIR_I1) return __int_as_float(i != 0);
  if (dst == KTIR_I8) return __int_as_float((int8_t)i);
  if (dst == KTIR_I16) return __int_as_float((int16_t)i);
  return x;
}

__device__ __forceinline__ float unop(int op, int dt, float x) {
  float r;
  switch (op) {
    case KTIR_OP_NEGF: return -x;
    case KTIR_OP_ABSF: return fabsf(x);
    case KTIR_OP_EXP: r = expf(x); break;
    case KTIR_OP_LOG: r = logf(x); break;
    case KTIR_OP_LOG2: r = log2f(x); break;
    case KTIR_OP_LOG1P: r = log1pf(x); break;
    case KTIR_OP_SQRT: r = __builtin_sqrtf(x); break;
    case KTIR_OP_RSQRT: r = (dt == KTIR_F32) ? __fdiv_rn(1.f, __builtin_sqrtf(x))
                                              : __fdiv_rn(1.f, round_to(__builtin_sqrtf(x), dt)); break;
    case KTIR_OP_TANH: r = tanhf(x); break;
    case KTIR_OP_SIN: r = sinf(x); break;
    case KTIR_OP_COS: r = cosf(x); break;
    case KTIR_OP_ERF: return erf_as(x, dt);
    case KTIR_OP_CEIL: r = ceilf(x); break;
    case KTIR_OP_FLOOR: r = floorf(x); break;
    case KTIR_OP_NOTI: return __int_as_float(__float_as_int(x) ? 0 : 1);
    case KTIR_OP_ABSI: { int i = __float_as_int(x); return __int_as_float(i < 0 ? neg_i(i) : i); }
    default: r = 0.f;
  }
  return round_to(r, dt);
}

// ---- leaf access ------------------------------------------------------------

template <int V>
__device__ __forceinline__ void leaf_load(const ktir_leaf_t& L, int nd, int64_t lane, const int64_t* idx,
                                          int64_t flat, float* out, bool bcast) {
  int64_t lo = lane_offset(L, lane);
  if (L.offsets) {
    const int64_t* off = (const int64_t*)L.offsets + lane * L.offsets_lane_stride + flat;
    int nv = bcast ? 1 : V;
    for (int v = 0; v < nv; ++v) {
      int64_t e = lo + off[v];
      out[v] = (e >= L.lo && e < L.hi) ? load_elem(L.ptr, e, L.dtype) : 0.f;
    }
    if (bcast) for (int v = 1; v < V; ++v) out[v] = out[0];
    return;
  }
  int64_t e0 = lo;
#pragma unroll
  for (int d = 0; d < KTIR_MAX_DIMS; ++d)
    if (d < nd) e0 += idx[d] * L.strides[d];
  if (bcast) {
    float x = (e0 >= L.lo && e0 < L.hi) ? load_elem(L.ptr, e0, L.dtype) : 0.f;
    for (int v = 0; v < V; ++v) out[v] = x;
    return;
  }
  if (V == 8 && (L.flags & KTIR_LEAF_VEC8) && e0 >= L.lo && e0 + V <= L.hi) {
    switch (L.dtype) {
      case KTIR_F16: {
        uint4 w = *(const uint4*)((const _Float16*)L.ptr + e0);
        const _Float16* h = (const _Float16*)&w;
        for (int v = 0; v < V; ++v) out[v] = (float)h[v];
        return;
      }
      case KTIR_BF16: {
        uint4 w = *(const uint4*)((const uint16_t*)L.ptr + e0);
        const uint32_t* u = (const uint32_t*)&w;
        for (int v = 0; v < 4; ++v) {
          out[2 * v] = __uint_as_float(u[v] << 16);
          out[2 * v + 1] = __uint_as_float(u[v] & 0xffff0000u);
        }
        return;
      }
      case KTIR_F32: case KTIR_I32: {
        float4 w0 = *(const float4*)((const float*)L.ptr + e0);
        float4 w1 = *(const float4*)((const float*)L.ptr + e0 + 4);
        out[0] = w0.x; out[1] = w0.y; out[2] = w0.z; out[3] = w0.w;
        out[4] = w1.x; out[5] = w1.y; out[6] = w1.z; out[7] = w1.w;
        return;
      }
      default: break;
    }
  }
  if (V == 4 && (L.flags & KTIR_LEAF_VEC) && e0 >= L.lo && e0 + V <= L.hi) {
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
  int64_t s = L.strides[nd - 1];
  for (int v = 0; v < V; ++v) {
    int64_t e = e0 + v * s;
    out[v] = (e >= L.lo && e < L.hi) ? load_elem(L.ptr, e, L.dtype) : 0.f;
  }
}

template <int V>
__device__ __forceinline__ void leaf_store(const ktir_leaf_t& L, int nd, int64_t lane, const int64_t* idx,
                                           int64_t flat, int64_t per_lane, const float* val, int nv) {
  int64_t lo = lane_offset(L, lane);
  if (L.offsets) {
    const int64_t* off = (const int64_t*)L.offsets + lane * L.offsets_lane_stride + flat;
    for (int v = 0; v < nv; ++v) {
      int64_t e = lo + off[v];
      if (e < L.lo || e >= L.hi) continue;
      if (L.winner && ((const int32_t*)L.winner)[e - L.winner_base] != (int32_t)(lane * per_lane + flat + v))
        continue;
      store_elem(L.ptr, e, L.dtype, val[v]);
    }
    return;
  }
  int64_t e0 = lo;
#pragma unroll
  for (int d = 0; d < KTIR_MAX_DIMS; ++d)
    if (d < nd) e0 += idx[d] * L.strides[d];
  if (V == 8 && nv == V && !L.winner && (L.flags & KTIR_LEAF_VEC8) && e0 >= L.lo && e0 + V <= L.hi) {
    switch (L.dtype) {
      case KTIR_F16: {
        _Float16 h[8];
        for (int v = 0; v < 8; ++v) h[v] = (_Float16)val[v];
        *(uint4*)((_Float16*)L.ptr + e0) = *(const uint4*)h;
        return;
      }
      case KTIR_BF16: {
        uint32_t b[8];
        for (int v = 0; v < 8; ++v) b[v] = __float_as_uint(round_bf16(val[v])) >> 16;
        *(uint4*)((uint16_t*)L.ptr + e0) =
            make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16), b[6] | (b[7] << 16));
        return;
      }
      case KTIR_F32: case KTIR_I32:
        *(float4*)((float*)L.ptr + e0) = make_float4(val[0], val[1], val[2], val[3]);
        *(float4*)((float*)L.ptr + e0 + 4) = make_float4(val[4], val[5], val[6], val[7]);
        return;
      default: break;
    }
  }
  if (V == 4 && nv == V && !L.winner && (L.flags & KTIR_LEAF_VEC) && e0 >= L.lo && e0 + V <= L.hi) {
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
  int64_t s = L.strides[nd - 1];
  for (int v = 0; v < nv; ++v) {
    int64_t e = e0 + v * s;
    if (e < L.lo || e >= L.hi) continue;
    if (L.winner && ((const int32_t*)L.winner)[e - L.winner_base] != (int32_t)(lane * per_lane + flat + v))
      continue;
    store_elem(L.ptr, e, L.dtype, val[v]);
  }
}

// ---- the interpreter ---------------------------------------------------------

#define FOR_V for (int v = 0; v < V; ++v)

// Execute one instruction for V elements.  `rowctx` marks per-row code in row
// mode: loads broadcast the element at inner index 0 and stores write once.
// The ops a "simple" program may use: arithmetic, compares, casts, selects,
// exp / sqrt / rsqrt.  Programs with anything else run the FULL variant,
// whose larger code and register footprint the common case does not pay.
__host__ __device__ __forceinline__ bool simple_op(int op) {
  switch (op) {
    case KTIR_OP_LOG: case KTIR_OP_LOG2: case KTIR_OP_LOG1P: case KTIR_OP_TANH: case KTIR_OP_SIN:
    case KTIR_OP_COS: case KTIR_OP_ERF: case KTIR_OP_REMF: case KTIR_OP_POWF: case KTIR_OP_DIVSI:
    case KTIR_OP_REMSI: case KTIR_OP_FLOORDIVSI: case KTIR_OP_FLOORREMSI: case KTIR_OP_CEILDIVSI:
    case KTIR_OP_RED: case KTIR_OP_FOLD: case KTIR_OP_ELEM: case KTIR_OP_ENDELEM:
      return false;
  }
  return true;
}

__device__ __forceinline__ float unop_simple(int op, int dt, float x) {
  float r;
  switch (op) {
    case KTIR_OP_NEGF: return -x;
    case KTIR_OP_ABSF: return fabsf(x);
    case KTIR_OP_EXP: r = expf(x); break;
    case KTIR_OP_SQRT: r = __builtin_sqrtf(x); break;
    case KTIR_OP_RSQRT: r = (dt == KTIR_F32) ? __fdiv_rn(1.f, __builtin_sqrtf(x))
                                              : __fdiv_rn(1.f, round_to(__builtin_sqrtf(x), dt)); break;
    case KTIR_OP_CEIL: r = ceilf(x); break;
    case KTIR_OP_FLOOR: r = floorf(x); break;
    case KTIR_OP_NOTI: return __int_as_float(__float_as_int(x) ? 0 : 1);
    case KTIR_OP_ABSI: { int i = __float_as_int(x); return __int_as_float(i < 0 ? neg_i(i) : i); }
    default: r = 0.f;
  }
  return round_to(r, dt);
}

__device__ __forceinline__ float binop_f_simple(int op, int dt, float x, float y) {
  float r;
  switch (op) {
    case KTIR_OP_ADDF: r = __fadd_rn(x, y); break;
    case KTIR_OP_SUBF: r = __fsub_rn(x, y); break;
    case KTIR_OP_MULF: r = mul_keep(x, y); break;
    case KTIR_OP_DIVF: r = __fdiv_rn(x, y); break;
    case KTIR_OP_MAXIMUMF: r = (x != x || y != y) ? __int_as_float(0x7fc00000) : fmaxf(x, y); break;
    case KTIR_OP_MINIMUMF: r = (x != x || y != y) ? __int_as_float(0x7fc00000) : fminf(x, y); break;
    case KTIR_OP_MAXNUMF: r = fmaxf(x, y); break;
    case KTIR_OP_MINNUMF: r = fminf(x, y); break;
    default: r = 0.f;
  }
  return round_to(r, dt);
}

__device__ __forceinline__ int binop_i_simple(int op, int x, int y) {
  switch (op) {
    case KTIR_OP_ADDI: return (int)((uint32_t)x + (uint32_t)y);
    case KTIR_OP_SUBI: return (int)((uint32_t)x - (uint32_t)y);
    case KTIR_OP_MULI: return (int)((uint32_t)x * (uint32_t)y);
    case KTIR_OP_ANDI: return x & y;
    case KTIR_OP_ORI: return x | y;
    case KTIR_OP_XORI: return x ^ y;
    case KTIR_OP_SHLI: return shl_i(x, y);
    case KTIR_OP_SHRSI: return shrs_i(x, y);
    case KTIR_OP_SHRUI: return shru_i(x, y);
    case KTIR_OP_MAXSI: return x > y ? x : y;
    case KTIR_OP_MINSI: return x < y ? x : y;
  }
  return 0;
}

template <int V, int NR, bool FULL>
__device__ __forceinline__ void exec(const ktir_prog_t& P, const ktir_instr_t in, float (&r)[NR][V],
                                     int64_t lane, const int64_t* idx, int64_t flat, int64_t per_lane,
                                     bool rowctx, bool writer, float* red, int64_t red_pos, int64_t inner) {
  const int op = in.op;
  if (op >= KTIR_OP_NEGF && op < KTIR_OP_ADDF) {
    if (FULL) {
      FOR_V r[in.dst][v] = unop(op, in.dt, r[in.a][v]);
    } else {
      FOR_V r[in.dst][v] = unop_simple(op, in.dt, r[in.a][v]);
    }
    return;
  }
  if (op >= KTIR_OP_ADDF && op < KTIR_OP_ADDI) {
    if (FULL) {
      FOR_V r[in.dst][v] = binop_f(op, in.dt, r[in.a][v], r[in.b][v]);
    } else {
      FOR_V r[in.dst][v] = binop_f_simple(op, in.dt, r[in.a][v], r[in.b][v]);
    }
    return;
  }
  if (op >= KTIR_OP_ADDI) {
    if (FULL) {
      FOR_V r[in.dst][v] = __int_as_float(binop_i(op, __float_as_int(r[in.a][v]), __float_as_int(r[in.b][v])));
    } else {
      FOR_V r[in.dst][v] = __int_as_float(binop_i_simple(op, __float_as_int(r[in.a][v]), __float_as_int(r[in.b][v])));
    }
    return;
  }
  switch (op) {
    case KTIR_OP_LD: {
      float tmp[V];
      leaf_load<V>(P.leaves[in.aux], P.ndim, lane, idx, flat, tmp, rowctx);
      FOR_V r[in.dst][v] = tmp[v];
      break;
    }
    case KTIR_OP_ST: {
      if (rowctx && !writer) break;
      float tmp[V];
      FOR_V tmp[v] = r[in.a][v];
      int nv = rowctx ? 1 : (int)((inner - idx[P.ndim - 1]) < V ? (inner - idx[P.ndim - 1]) : V);
      leaf_store<V>(P.leaves[in.aux], P.ndim, lane, idx, flat, per_lane, tmp, nv);
      break;
    }
    case KTIR_OP_CONST: FOR_V r[in.dst][v] = __int_as_float(in.imm); break;
    case KTIR_OP_LANE: {
      double d = ((const double*)P.lane_scalars)[lane * P.n_lane_scalars + in.aux];
      float x = is_float_dt(in.dt) ? round_to((float)d, in.dt) : __int_as_float((int)(long long)d);
      FOR_V r[in.dst][v] = x;
      break;
    }
    case KTIR_OP_IDX: {
      int64_t base = idx[in.aux];
      bool inner_dim = (in.aux == P.ndim - 1);
      FOR_V r[in.dst][v] = __int_as_float((int)(base + ((inner_dim && !rowctx) ? v : 0)));
      break;
    }
    case KTIR_OP_RED: {
      FOR_V if (red_pos + v < inner) red[red_pos + v] = r[in.a][v];
      break;
    }
    case KTIR_OP_CAST: FOR_V r[in.dst][v] = cast_val(r[in.a][v], in.aux, in.dt); break;
    case KTIR_OP_BITCAST: FOR_V r[in.dst][v] = r[in.a][v]; break;
    case KTIR_OP_SELECT:
      FOR_V r[in.dst][v] = __float_as_int(r[in.a][v]) ? r[in.b][v] : r[in.c][v];
      break;
    case KTIR_OP_FMA:
      FOR_V r[in.dst][v] = round_to(__fadd_rn(__fmul_rn(r[in.a][v], r[in.b][v]), r[in.c][v]), in.dt);
      break;
    case KTIR_OP_CMPF: FOR_V r[in.dst][v] = __int_as_float(cmp_f(in.aux, r[in.a][v], r[in.b][v])); break;
    case KTIR_OP_CMPI:
      FOR_V r[in.dst][v] = __int_as_float(cmp_i(in.aux, __float_as_int(r[in.a][v]), __float_as_int(r[in.b][v])));
      break;
    default: break;
  }
}

// Division by a launch-invariant divisor with one multiply-high (n < 2^31).
struct FastDiv {
  uint32_t d, m, s;
};

static inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{d, 0, 0};
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  f.s = s;
  f.m = (uint32_t)(((1ull << 32) * ((1ull << s) - d)) / d + 1);
  return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (__umulhi(n, f.m) + n) >> f.s;
}

struct FlatDivs {
  FastDiv nvi;                     // vectors per row
  FastDiv dim[KTIR_MAX_DIMS];      // extents of the outer dims
  uint32_t rows_per_lane;
};

__device__ __forceinline__ void decompose(uint32_t vid, const FlatDivs& D, int nd, int V_, int64_t inner,
                                          int64_t* idx, int64_t& lane, int64_t& flat) {
  const uint32_t row = fdiv(vid, D.nvi);
  idx[KTIR_MAX_DIMS - 1] = 0;
  uint32_t t = row;
#pragma unroll
  for (int d = KTIR_MAX_DIMS - 2; d >= 0; --d) {
    if (d < nd - 1) {
      uint32_t q = fdiv(t, D.dim[d]);
      idx[d] = t - q * D.dim[d].d;
      t = q;
    }
  }
  // the inner index lives at position nd-1
  const int64_t col = (int64_t)(vid - row * D.nvi.d) * V_;
#pragma unroll
  for (int d = 0; d < KTIR_MAX_DIMS; ++d)
    if (d == nd - 1) idx[d] = col;
  lane = t;
  flat = (int64_t)(row - t * D.rows_per_lane) * inner + col;
}

// element offset of a leaf at (lane, idx) where idx has been normalised to
// KTIR_MAX_DIMS dims with the innermost last
__device__ __forceinline__ int64_t leaf_off(const ktir_leaf_t& L, int64_t lane, const uint32_t* idx) {
  int64_t e = lane_offset(L, lane);
#pragma unroll
  for (int d = 0; d < KTIR_MAX_DIMS; ++d) e += (int64_t)idx[d] * L.strides[d];
  return e;
}


}  // namespace ktir
