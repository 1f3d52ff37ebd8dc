// Register ops of the streaming program kernels (ktir_map.hip,
// ktir_tile.hip): the semantics of the general interpreter's simple ops
// (ktir_program_impl.h), one element at a time.
#pragma once
#include "ktir_program_impl.h"

namespace ktir {

// One register op on element values a, b, c (c read only by SELECT / FMA).
__device__ __forceinline__ float exec_val(const ktir_prog_t& P, const ktir_instr_t in, float a, float b, float c,
                                          int64_t lane) {
  const int op = in.op;
  float v;
  if (op >= KTIR_OP_NEGF && op < KTIR_OP_ADDF) {
    v = unop_simple(op, in.dt, a);
  } else if (op >= KTIR_OP_ADDF && op < KTIR_OP_ADDI) {
    v = binop_f_simple(op, in.dt, a, b);
  } else if (op >= KTIR_OP_ADDI) {
    v = __int_as_float(binop_i_simple(op, __float_as_int(a), __float_as_int(b)));
  } else {
    switch (op) {
      case KTIR_OP_CONST: v = __int_as_float(in.imm); break;
      case KTIR_OP_LANE: {
        double d = ((const double*)P.lane_scalars)[lane * P.n_lane_scalars + in.aux];
        v = is_float_dt(in.dt) ? round_to((float)d, in.dt) : __int_as_float((int)(long long)d);
        break;
      }
      case KTIR_OP_CAST: v = cast_val(a, in.aux, in.dt); break;
      case KTIR_OP_BITCAST: v = a; break;
      case KTIR_OP_SELECT: v = __float_as_int(a) ? b : c; break;
      case KTIR_OP_FMA: v = round_to(__fadd_rn(__fmul_rn(a, b), c), in.dt); break;
      case KTIR_OP_CMPF: v = __int_as_float(cmp_f(in.aux, a, b)); break;
      case KTIR_OP_CMPI: v = __int_as_float(cmp_i(in.aux, __float_as_int(a), __float_as_int(b))); break;
      default: v = 0.f;
    }
  }
  return v;
}

}  // namespace ktir
