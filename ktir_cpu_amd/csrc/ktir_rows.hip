// Register-resident row kernel for row-mode programs (mode 1) whose element
// blocks are single chains: every ELEM block starts from a loaded row (or a
// row-broadcast vector), applies a chain of unary ops and binary ops against
// row scalars / loaded rows, and ends in a fold (RED + FOLD) or a store.
// Softmax, RMSNorm and LayerNorm lower to this form.
//
// A group of TPR threads owns one row of n = TPR * E elements; thread t holds
// the element pairs p = k * TPR + t (k < E/2), i.e. elements 2p and 2p + 1,
// so every load moves 2 consecutive elements per lane (coalesced across the
// wave).  The loaded rows stay in registers for all passes (each leaf is read
// from HBM once per row).  Folds reproduce the reference's pairwise-halving
// tree (dialects/linalg_ops.py:114-131) exactly: its levels pair element i
// with i + n/2, i + n/4, ...; with this layout the first log2(E/2) levels pair
// registers of one thread, the next log2(TPR) levels pair lanes t and t ^ s
// (LDS for s >= 64, wave shuffles below), the last pairs the two elements of
// a pair.  Each combine is commutative, so both partners of a butterfly hold
// the lower element's value and the result ends up in every thread.
#include "ktir_program_impl.h"

namespace ktir {

constexpr int RC_MAX_STEPS = 16;

typedef float gf2 __attribute__((ext_vector_type(2)));
typedef uint32_t gu4 __attribute__((ext_vector_type(4)));
constexpr int RC_MAX_OPS = 8;

struct RcOp {
  int8_t op, dt, aux;
  int8_t kind;      // 0 unary / cast, 1 row register operand, 2 cached row operand, 3 the chain value itself
  int8_t idx;       // register or cache slot
  int8_t swap;      // the operand is the left side
  int8_t pad[2];
};

struct RcStep {
  int8_t kind;      // 0 row instruction P.instr[pc], 1 pass, 2 row store of register P.instr[pc].a
  int8_t pc;
  int8_t src;       // pass: cache slot the chain starts from
  int8_t n_ops;
  int8_t end;       // 0 fold into register dst, 1 store to leaf st_leaf
  int8_t fold_op, fold_dt, dst, st_leaf;
  int8_t head;      // fused leading ops: 0 none, 1 SUBF(row) + EXP, 2 MULF(self)
  int8_t save;      // keep the values after the fused head for a later pass
  int8_t reuse;     // start from the values a previous pass kept (its head is the same)
  RcOp ops[RC_MAX_OPS];
};

struct RcPlan {
  int32_t n_steps, n_slots;
  int8_t slot_leaf[2];
  RcStep steps[RC_MAX_STEPS];
};

// A copy of an LDS-resident, workgroup-uniform struct in scalar registers.
template <typename T>
struct Words {
  int w[sizeof(T) / 4];
};

template <typename T>
__device__ __forceinline__ T uniform_copy(const T& x) {
  static_assert(sizeof(T) % 4 == 0, "whole words");
  const Words<T> in = __builtin_bit_cast(Words<T>, x);
  Words<T> out;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); ++i) out.w[i] = __builtin_amdgcn_readfirstlane(in.w[i]);
  return __builtin_bit_cast(T, out);
}

// Row registers of one row: uniform values in scalar registers, selected by
// the (uniform) register number.  Named members, not an array: an array
// indexed by a run-time number would live in scratch memory, and every
// scratch access waits for all of the wavefront's outstanding memory traffic.
struct RowRegs {
  float r0, r1, r2, r3, r4, r5, r6, r7;
  __device__ __forceinline__ float get(int i) const {
    switch (i) {
      case 0: return r0;
      case 1: return r1;
      case 2: return r2;
      case 3: return r3;
      case 4: return r4;
      case 5: return r5;
      case 6: return r6;
      default: return r7;
    }
  }
  __device__ __forceinline__ void set(int i, float v) {
    switch (i) {
      case 0: r0 = v; break;
      case 1: r1 = v; break;
      case 2: r2 = v; break;
      case 3: r3 = v; break;
      case 4: r4 = v; break;
      case 5: r5 = v; break;
      case 6: r6 = v; break;
      default: r7 = v; break;
    }
  }
};

// ---- host-side analysis ------------------------------------------------------

static bool rows_leaf_ok(const ktir_leaf_t& L, int nd) {
  return L.offsets == 0 && L.winner == 0 && L.strides[nd - 1] == 1 && (L.flags & KTIR_LEAF_VEC) &&
         (L.dtype == KTIR_F16 || L.dtype == KTIR_BF16 || L.dtype == KTIR_F32);
}

static bool row_op_ok(int op) {
  switch (op) {
    case KTIR_OP_LD: case KTIR_OP_ST: case KTIR_OP_IDX: case KTIR_OP_RED: case KTIR_OP_FOLD:
    case KTIR_OP_ELEM: case KTIR_OP_ENDELEM: case KTIR_OP_NOP:
      return false;
  }
  return true;
}

// operands a row instruction reads: bit 0 a, bit 1 b, bit 2 c
static int row_op_reads(int op) {
  if (op == KTIR_OP_CONST || op == KTIR_OP_LANE) return 0;
  if (op == KTIR_OP_SELECT || op == KTIR_OP_FMA) return 7;
  if (op >= KTIR_OP_ADDF || op == KTIR_OP_CMPF || op == KTIR_OP_CMPI) return 3;
  return 1;
}

// Chain ops the kernels implement (straight-line code per op keeps them
// small): float arithmetic, and f32 -> f16 / bf16 / f32 rounding casts.  An
// f16 / bf16 op is kept as its f32 op followed by a rounding cast to its
// type (the general kernels' arithmetic: f32, then rounded), except a narrow
// rsqrt, whose root is rounded before the division.
static bool chain_dt(int dt) { return dt == KTIR_F32 || dt == KTIR_F16 || dt == KTIR_BF16; }

static bool chain_unary(const ktir_instr_t& x) {
  switch (x.op) {
    case KTIR_OP_NEGF: case KTIR_OP_ABSF: case KTIR_OP_EXP: case KTIR_OP_SQRT:
      return chain_dt(x.dt);
    case KTIR_OP_RSQRT:
      return x.dt == KTIR_F32;
    case KTIR_OP_CAST:
      return x.aux == KTIR_F32 && chain_dt(x.dt);
  }
  return false;
}

static bool chain_binary(const ktir_instr_t& x) {
  switch (x.op) {
    case KTIR_OP_ADDF: case KTIR_OP_SUBF: case KTIR_OP_MULF: case KTIR_OP_DIVF: case KTIR_OP_MAXIMUMF:
    case KTIR_OP_MINIMUMF: case KTIR_OP_MAXNUMF: case KTIR_OP_MINNUMF:
      return chain_dt(x.dt);
  }
  return false;
}

// a pass plan of f32 folds combined by the arithmetic or NaN-propagating
// ops, with no NaN-ignoring min / max and no exact division among its chain
// ops.  The row-wave kernel takes the others in its FOLDX instantiations
// (folds of any op, rounded to f16 / bf16 at every level where the fold is of
// that type); of them, the fixed-form kernels take only the f16-math softmax
// and norm-scale forms.
static bool plan_plain(const RcPlan& R) {
  for (int i = 0; i < R.n_steps; ++i) {
    const RcStep& S = R.steps[i];
    if (S.kind != 1) continue;
    if (S.end == 0 && (S.fold_dt != KTIR_F32 || S.fold_op == KTIR_OP_MAXNUMF || S.fold_op == KTIR_OP_MINNUMF))
      return false;
    for (int k = 0; k < S.n_ops; ++k) {
      const RcOp& o = S.ops[k];
      if (o.op == KTIR_OP_MAXNUMF || o.op == KTIR_OP_MINNUMF || (o.op == KTIR_OP_DIVF && o.aux)) return false;
    }
  }
  return true;
}

static bool analyze_rows(const ktir_prog_t& P, RcPlan& R) {
  enum { K_NONE = 0, K_ROW = 1, K_LEAF = 2, K_ACC = 3 };
  int kind[KTIR_NREG], slot_of[KTIR_NREG];
  for (int i = 0; i < KTIR_NREG; ++i) kind[i] = K_NONE, slot_of[i] = -1;
  const int nd = P.ndim;
  R.n_steps = 0;
  R.n_slots = 0;
  auto slot_for = [&](int leaf) -> int {
    for (int s = 0; s < R.n_slots; ++s)
      if (R.slot_leaf[s] == leaf) return s;
    if (R.n_slots == 2 || !rows_leaf_ok(P.leaves[leaf], nd)) return -1;
    R.slot_leaf[R.n_slots] = (int8_t)leaf;
    return R.n_slots++;
  };
  int pc = 0;
  while (pc < P.n_instr) {
    const ktir_instr_t& in = P.instr[pc];
    if (R.n_steps == RC_MAX_STEPS) return false;
    RcStep& S = R.steps[R.n_steps];
    S = RcStep{};
    if (in.op == KTIR_OP_ST) {
      // a row-level value stored once per row (column 0 of the leaf's row)
      if (in.a < 0 || in.a >= KTIR_NREG || kind[in.a] != K_ROW || P.leaves[in.aux].offsets != 0 ||
          P.leaves[in.aux].winner != 0)
        return false;
      S.kind = 2;
      S.pc = (int8_t)pc;
      S.st_leaf = (int8_t)in.aux;
      ++R.n_steps;
      ++pc;
      continue;
    }
    if (in.op != KTIR_OP_ELEM) {
      if (!row_op_ok(in.op) || !simple_op(in.op) || in.dst < 0 || in.dst >= KTIR_NREG) return false;
      const int reads = row_op_reads(in.op);
      if (((reads & 1) && (in.a < 0 || in.a >= KTIR_NREG || kind[in.a] != K_ROW)) ||
          ((reads & 2) && (in.b < 0 || in.b >= KTIR_NREG || kind[in.b] != K_ROW)) ||
          ((reads & 4) && (in.c < 0 || in.c >= KTIR_NREG || kind[in.c] != K_ROW)))
        return false;
      S.kind = 0;
      S.pc = (int8_t)pc;
      kind[in.dst] = K_ROW;
      ++R.n_steps;
      ++pc;
      continue;
    }
    const int end = in.aux;
    if (end <= pc || end >= P.n_instr || P.instr[end].op != KTIR_OP_ENDELEM) return false;
    S.kind = 1;
    S.src = -1;
    int acc = -1;
    bool done = false;
    // start the chain from the cached row held by register r
    auto start = [&](int r) -> bool {
      if (acc >= 0 || kind[r] != K_LEAF) return false;
      S.src = (int8_t)slot_of[r];
      acc = r;
      return true;
    };
    auto add = [&](const RcOp& o) -> bool {
      if (S.n_ops == RC_MAX_OPS) return false;
      S.ops[S.n_ops++] = o;
      return true;
    };
    for (int q = pc + 1; q < end; ++q) {
      const ktir_instr_t& x = P.instr[q];
      if (done || x.dst < 0 || x.dst >= KTIR_NREG || x.a < 0 || x.a >= KTIR_NREG || x.b < 0 || x.b >= KTIR_NREG)
        return false;
      if (x.op == KTIR_OP_LD) {
        const int s = slot_for(x.aux);
        if (s < 0 || x.dst == acc) return false;
        kind[x.dst] = K_LEAF;
        slot_of[x.dst] = s;
      } else if (x.op == KTIR_OP_CAST && kind[x.a] == K_LEAF && x.dt == KTIR_F32 &&
                 x.aux == P.leaves[R.slot_leaf[slot_of[x.a]]].dtype) {
        // exact widening of a cached row: the cache holds it as f32 already
        kind[x.dst] = K_LEAF;
        slot_of[x.dst] = slot_of[x.a];
      } else if (chain_unary(x)) {
        if (kind[x.a] == K_LEAF && !start(x.a)) return false;
        if (x.a != acc) return false;
        if (x.op == KTIR_OP_CAST || x.dt == KTIR_F32) {
          if (!add(RcOp{x.op, x.dt, (int8_t)x.aux, 0, 0, 0, {0, 0}})) return false;
        } else {
          // a narrow op: its f32 op, then (unless exact, as a sign change is) the rounding
          if (!add(RcOp{x.op, KTIR_F32, 0, 0, 0, 0, {0, 0}})) return false;
          if (x.op != KTIR_OP_NEGF && x.op != KTIR_OP_ABSF &&
              !add(RcOp{KTIR_OP_CAST, x.dt, KTIR_F32, 0, 0, 0, {0, 0}}))
            return false;
        }
        acc = x.dst;
      } else if (chain_binary(x)) {
        int a = x.a, b = x.b;
        if (a != acc && b != acc) {
          if (kind[a] == K_LEAF) {
            if (!start(a)) return false;
          } else if (kind[b] == K_LEAF) {
            if (!start(b)) return false;
          } else {
            return false;
          }
        }
        // a narrow op: its f32 op (a division correctly rounded), then the rounding
        const bool narrow = x.dt != KTIR_F32;
        RcOp o{x.op, KTIR_F32, (int8_t)(narrow && x.op == KTIR_OP_DIVF), 0, 0, 0, {0, 0}};
        if (a == acc && b == acc) {
          o.kind = 3;
        } else {
          const bool left_is_acc = (a == acc);
          const int other = left_is_acc ? b : a;
          o.swap = left_is_acc ? 0 : 1;
          if (kind[other] == K_ROW) {
            o.kind = 1;
            o.idx = (int8_t)other;
          } else if (kind[other] == K_LEAF) {
            o.kind = 2;
            o.idx = (int8_t)slot_of[other];
          } else {
            return false;
          }
        }
        if (!add(o)) return false;
        // min / max give one of their operands: nothing to round
        if (narrow && x.op != KTIR_OP_MAXIMUMF && x.op != KTIR_OP_MINIMUMF && x.op != KTIR_OP_MAXNUMF &&
            x.op != KTIR_OP_MINNUMF && !add(RcOp{KTIR_OP_CAST, x.dt, KTIR_F32, 0, 0, 0, {0, 0}}))
          return false;
        acc = x.dst;
      } else if (x.op == KTIR_OP_RED || x.op == KTIR_OP_ST) {
        if (kind[x.a] == K_LEAF && acc < 0 && !start(x.a)) return false;
        if (x.a != acc) return false;
        if (x.op == KTIR_OP_RED) {
          S.end = 0;
        } else {
          if (!rows_leaf_ok(P.leaves[x.aux], nd)) return false;
          S.end = 1;
          S.st_leaf = (int8_t)x.aux;
        }
        done = true;
      } else {
        return false;
      }
      if (x.op != KTIR_OP_RED && x.op != KTIR_OP_ST && x.op != KTIR_OP_LD &&
          !(x.op == KTIR_OP_CAST && kind[x.dst] == K_LEAF))
        kind[x.dst] = K_ACC;
    }
    if (!done) return false;
    pc = end + 1;
    if (S.end == 0) {
      if (pc >= P.n_instr || P.instr[pc].op != KTIR_OP_FOLD) return false;
      const ktir_instr_t& f = P.instr[pc];
      if (f.dst < 0 || f.dst >= KTIR_NREG || f.aux >= KTIR_OP_ADDI) return false;
      if (f.aux != KTIR_OP_ADDF && f.aux != KTIR_OP_MULF && f.aux != KTIR_OP_MAXIMUMF && f.aux != KTIR_OP_MINIMUMF &&
          f.aux != KTIR_OP_MAXNUMF && f.aux != KTIR_OP_MINNUMF)
        return false;
      if (f.dt != KTIR_F32 && f.dt != KTIR_F16 && f.dt != KTIR_BF16) return false;
      S.fold_op = (int8_t)f.aux;
      S.fold_dt = f.dt;
      S.dst = f.dst;
      kind[f.dst] = K_ROW;
      ++pc;
    }
    // registers written in the block other than the cached rows are gone after it
    for (int i = 0; i < KTIR_NREG; ++i)
      if (kind[i] == K_ACC) kind[i] = K_NONE;
    ++R.n_steps;
  }
  // fused heads, and reuse of exp(x - m) between two passes that compute it
  int last_subexp = -1;
  for (int i = 0; i < R.n_steps; ++i) {
    RcStep& S = R.steps[i];
    if (S.kind == 0) {
      // a row instruction that rewrites the subtracted register ends the reuse window
      if (last_subexp >= 0 && P.instr[S.pc].dst == R.steps[last_subexp].ops[0].idx) last_subexp = -1;
      continue;
    }
    if (S.kind != 1) continue;
    const RcOp* o = S.ops;
    if (S.n_ops >= 2 && o[0].op == KTIR_OP_SUBF && o[0].kind == 1 && !o[0].swap && o[1].op == KTIR_OP_EXP &&
        o[1].kind == 0 && o[0].dt == KTIR_F32 && o[1].dt == KTIR_F32) {
      S.head = 1;
      if (last_subexp >= 0 && R.steps[last_subexp].src == S.src && R.steps[last_subexp].ops[0].idx == o[0].idx) {
        R.steps[last_subexp].save = 1;
        S.reuse = 1;
      }
      last_subexp = i;
    } else if (S.n_ops >= 1 && o[0].op == KTIR_OP_MULF && o[0].kind == 3 && o[0].dt == KTIR_F32) {
      S.head = 2;
    }
    // so does a fold into the subtracted register
    if (S.end == 0 && last_subexp >= 0 && S.dst == R.steps[last_subexp].ops[0].idx) last_subexp = -1;
  }
  return R.n_steps > 0;
}

// ---- device side ---------------------------------------------------------------

template <int DT>
__device__ __forceinline__ void load_pair(const void* ptr, int64_t e0, float& a, float& b) {
  if (DT == KTIR_F32) {
    const gf2 w = *(const KTIR_G(gf2)*)((const KTIR_G(float)*)ptr + e0);
    a = w[0];
    b = w[1];
  } else {
    const uint32_t w = *(const KTIR_G(uint32_t)*)((const KTIR_G(uint16_t)*)ptr + e0);
    if (DT == KTIR_BF16) {
      a = __uint_as_float(w << 16);
      b = __uint_as_float(w & 0xffff0000u);
    } else {
      a = (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
      b = (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
    }
  }
}

template <int DT>
__device__ __forceinline__ void store_pair(void* ptr, int64_t e0, float a, float b) {
  if (DT == KTIR_F32) {
    *(KTIR_G(gf2)*)((KTIR_G(float)*)ptr + e0) = gf2{a, b};
  } else if (DT == KTIR_BF16) {
    *(KTIR_G(uint32_t)*)((KTIR_G(uint16_t)*)ptr + e0) =
        (__float_as_uint(round_bf16(a)) >> 16) | (__float_as_uint(round_bf16(b)) & 0xffff0000u);
  } else {
    *(KTIR_G(uint32_t)*)((KTIR_G(uint16_t)*)ptr + e0) = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)a) |
                                        ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)b) << 16);
  }
}

// a row of n = tpr * E elements starting at element `base` of L: straight-line
// paired accesses when the row lies inside the allocation, else per element
// with the reference's out-of-range rules (reads 0, writes dropped)
template <int E>
__device__ __forceinline__ void load_row(const ktir_leaf_t& L, int64_t base, int t, int tpr, float (&c)[E]) {
  if (base >= L.lo && base + (int64_t)tpr * E <= L.hi) {
    switch (L.dtype) {
      case KTIR_F16:
#pragma unroll
        for (int k = 0; k < E / 2; ++k) load_pair<KTIR_F16>((const void*)L.ptr, base + 2 * (k * tpr + t), c[2 * k], c[2 * k + 1]);
        return;
      case KTIR_BF16:
#pragma unroll
        for (int k = 0; k < E / 2; ++k) load_pair<KTIR_BF16>((const void*)L.ptr, base + 2 * (k * tpr + t), c[2 * k], c[2 * k + 1]);
        return;
      default:
#pragma unroll
        for (int k = 0; k < E / 2; ++k) load_pair<KTIR_F32>((const void*)L.ptr, base + 2 * (k * tpr + t), c[2 * k], c[2 * k + 1]);
        return;
    }
  }
#pragma unroll
  for (int q = 0; q < E; ++q) {
    const int64_t e = base + 2 * ((q >> 1) * tpr + t) + (q & 1);
    c[q] = (e >= L.lo && e < L.hi) ? load_elem(L.ptr, e, L.dtype) : 0.f;
  }
}

template <int E>
__device__ __forceinline__ void store_row(const ktir_leaf_t& L, int64_t base, int t, int tpr, const float (&v)[E]) {
  if (base >= L.lo && base + (int64_t)tpr * E <= L.hi) {
    switch (L.dtype) {
      case KTIR_F16:
#pragma unroll
        for (int k = 0; k < E / 2; ++k) store_pair<KTIR_F16>((void*)L.ptr, base + 2 * (k * tpr + t), v[2 * k], v[2 * k + 1]);
        return;
      case KTIR_BF16:
#pragma unroll
        for (int k = 0; k < E / 2; ++k) store_pair<KTIR_BF16>((void*)L.ptr, base + 2 * (k * tpr + t), v[2 * k], v[2 * k + 1]);
        return;
      default:
#pragma unroll
        for (int k = 0; k < E / 2; ++k) store_pair<KTIR_F32>((void*)L.ptr, base + 2 * (k * tpr + t), v[2 * k], v[2 * k + 1]);
        return;
    }
  }
  for (int q = 0; q < E; ++q) {
    const int64_t e = base + 2 * ((q >> 1) * tpr + t) + (q & 1);
    if (e >= L.lo && e < L.hi) store_elem(L.ptr, e, L.dtype, v[q]);
  }
}

__device__ __forceinline__ float maxnan(float x, float y) {
  return (x != x || y != y) ? __int_as_float(0x7fc00000) : fmaxf(x, y);
}
__device__ __forceinline__ float minnan(float x, float y) {
  return (x != x || y != y) ? __int_as_float(0x7fc00000) : fminf(x, y);
}

// e^x on the hardware exp2: 2^(x log2 e).  The rounding of x log2 e costs
// about |x| * 6e-8 relative error (a few f32 ulps for softmax arguments).
__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// x / s for a row scalar s with r = 1/s correctly rounded: q = x r, then one
// Markstein correction q + (x - s q) r (fused); within one ulp of x / s and
// nearly always its correct rounding.  Operands near the ends of the
// exponent range take __fdiv_rn.
__device__ __forceinline__ float div_by(float x, float s, float r) {
  const float q = x * r;
  const float res = __builtin_fmaf(-s, q, x);
  return __builtin_fmaf(res, r, q);
}

// one chain op over the E chain values; the opcode and operand kind are
// uniform, so both are dispatched once outside the element loops.  Ops are
// f32: an f16 / bf16 op of the program arrives here as its f32 op and a
// rounding cast (analyze_rows), and a division marked exact (aux 1) is
// the correctly rounded one, so that the rounding to the narrow type sees
// the f32 result the general kernels compute.
template <int E>
__device__ __forceinline__ void apply_op(const RcOp o, float (&v)[E], float s, const float (&c0)[E],
                                         const float (&c1)[E]) {
#define RC_UN(expr) { _Pragma("unroll") for (int e = 0; e < E; ++e) { const float x = v[e]; v[e] = (expr); } return; }
  if (o.kind == 0) {
    switch (o.op) {
      case KTIR_OP_NEGF: RC_UN(-x)
      case KTIR_OP_ABSF: RC_UN(fabsf(x))
      case KTIR_OP_EXP: RC_UN(exp_hw(x))
      case KTIR_OP_SQRT: RC_UN(__builtin_sqrtf(x))
      case KTIR_OP_RSQRT: RC_UN(__fdiv_rn(1.f, __builtin_sqrtf(x)))
      case KTIR_OP_CAST:
        if (o.dt == KTIR_F16) RC_UN(round_f16(x))
        if (o.dt == KTIR_BF16) RC_UN(round_bf16(x))
        return;
    }
    return;
  }
#undef RC_UN
  if (o.kind == 1) {
    // row scalar operand: no per-element operand copies
#define RC_S(expr) { _Pragma("unroll") for (int e = 0; e < E; ++e) { const float x = v[e]; v[e] = (expr); } return; }
    switch (o.op) {
      case KTIR_OP_ADDF: RC_S(__fadd_rn(x, s))
      case KTIR_OP_MULF: RC_S(__fmul_rn(x, s))
      case KTIR_OP_MAXIMUMF: RC_S(maxnan(x, s))
      case KTIR_OP_MINIMUMF: RC_S(minnan(x, s))
      case KTIR_OP_MAXNUMF: RC_S(fmaxf(x, s))
      case KTIR_OP_MINNUMF: RC_S(fminf(x, s))
      case KTIR_OP_SUBF: if (o.swap) RC_S(__fsub_rn(s, x)) else RC_S(__fsub_rn(x, s))
      case KTIR_OP_DIVF:
        if (o.swap) RC_S(__fdiv_rn(s, x))
        if (o.aux) RC_S(__fdiv_rn(x, s))
        {
          const float r = __fdiv_rn(1.f, s);
          const float as = fabsf(s);
          if (as > 1e-30f && as < 1e30f && r == r) {
            // the corrected product; __fdiv_rn for huge or non-finite operands
            float mx = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) mx = fmaxf(mx, fabsf(v[e]));
            if (__all(mx < 1e30f)) {
#pragma unroll
              for (int e = 0; e < E; ++e) v[e] = div_by(v[e], s, r);
            } else {
#pragma unroll
              for (int e = 0; e < E; ++e) {
                const float x = v[e];
                v[e] = fabsf(x) < 1e30f ? div_by(x, s, r) : __fdiv_rn(x, s);
              }
            }
            return;
          }
          RC_S(__fdiv_rn(x, s))
        }
    }
    return;
#undef RC_S
  }
  // operand from the cached rows or the chain value itself
#define RC_B(expr)                                                          \
  {                                                                         \
    _Pragma("unroll") for (int e = 0; e < E; ++e) {                         \
      const float p = v[e], q = o.kind == 3 ? p : (o.idx ? c1[e] : c0[e]);  \
      const float l = o.swap ? q : p, r = o.swap ? p : q;                   \
      v[e] = (expr);                                                        \
    }                                                                       \
    return;                                                                 \
  }
  switch (o.op) {
    case KTIR_OP_ADDF: RC_B(__fadd_rn(l, r))
    case KTIR_OP_SUBF: RC_B(__fsub_rn(l, r))
    case KTIR_OP_MULF: RC_B(__fmul_rn(l, r))
    case KTIR_OP_DIVF: RC_B(__fdiv_rn(l, r))
    case KTIR_OP_MAXIMUMF: RC_B(maxnan(l, r))
    case KTIR_OP_MINIMUMF: RC_B(minnan(l, r))
    case KTIR_OP_MAXNUMF: RC_B(fmaxf(l, r))
    case KTIR_OP_MINNUMF: RC_B(fminf(l, r))
  }
#undef RC_B
}

// fold combine in the fold's dtype (f32, or rounded to f16 / bf16)
template <int OP, int DT>
__device__ __forceinline__ float fold_op(float x, float y) {
  float r;
  if (OP == KTIR_OP_ADDF) r = __fadd_rn(x, y);
  else if (OP == KTIR_OP_MULF) r = DT == KTIR_F32 ? __fmul_rn(x, y) : mul_keep(x, y);
  else if (OP == KTIR_OP_MAXIMUMF) return maxnan(x, y);
  else if (OP == KTIR_OP_MAXNUMF) return fmaxf(x, y);   // an operand's value: no rounding
  else if (OP == KTIR_OP_MINNUMF) return fminf(x, y);
  else return minnan(x, y);
  return DT == KTIR_F32 ? r : (DT == KTIR_F16 ? round_f16(r) : round_bf16(r));
}

// fold of the group's n = TPR * E values (pairwise-halving order, see top)
template <int E, int OP, int DT>
__device__ __forceinline__ float fold_group_t(float (&v)[E], int tpr, float* xch) {
#pragma unroll
  for (int h = E / 4; h >= 1; h >>= 1) {
#pragma unroll
    for (int k = 0; k < h; ++k) {
      v[2 * k] = fold_op<OP, DT>(v[2 * k], v[2 * (k + h)]);
      v[2 * k + 1] = fold_op<OP, DT>(v[2 * k + 1], v[2 * (k + h) + 1]);
    }
  }
  float a = v[0], b = v[1];
  for (int s = tpr >> 1; s >= 64; s >>= 1) {   // partners in other wavefronts: through LDS
    __syncthreads();
    xch[2 * threadIdx.x] = a;
    xch[2 * threadIdx.x + 1] = b;
    __syncthreads();
    const int p = threadIdx.x ^ s;
    a = fold_op<OP, DT>(a, xch[2 * p]);
    b = fold_op<OP, DT>(b, xch[2 * p + 1]);
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    if (s < tpr) {
      a = fold_op<OP, DT>(a, __shfl_xor(a, s));
      b = fold_op<OP, DT>(b, __shfl_xor(b, s));
    }
  }
  return fold_op<OP, DT>(a, b);
}

template <int E, int OP>
__device__ __forceinline__ float fold_group_d(float (&v)[E], int dt, int tpr, float* xch) {
  if (dt == KTIR_F32) return fold_group_t<E, OP, KTIR_F32>(v, tpr, xch);
  if (dt == KTIR_F16) return fold_group_t<E, OP, KTIR_F16>(v, tpr, xch);
  return fold_group_t<E, OP, KTIR_BF16>(v, tpr, xch);
}

template <int E>
__device__ __forceinline__ float fold_group(float (&v)[E], int op, int dt, int tpr, float* xch) {
  switch (op) {
    case KTIR_OP_ADDF: return fold_group_d<E, KTIR_OP_ADDF>(v, dt, tpr, xch);
    case KTIR_OP_MULF: return fold_group_d<E, KTIR_OP_MULF>(v, dt, tpr, xch);
    case KTIR_OP_MAXIMUMF: return fold_group_d<E, KTIR_OP_MAXIMUMF>(v, dt, tpr, xch);
    case KTIR_OP_MAXNUMF: return fold_group_d<E, KTIR_OP_MAXNUMF>(v, dt, tpr, xch);
    case KTIR_OP_MINNUMF: return fold_group_d<E, KTIR_OP_MINNUMF>(v, dt, tpr, xch);
    default: return fold_group_d<E, KTIR_OP_MINIMUMF>(v, dt, tpr, xch);
  }
}

__device__ __forceinline__ void row_exec(const ktir_prog_t& P, const ktir_instr_t in, float* rr, int64_t lane) {
  const int op = in.op;
  const float a = rr[in.a], b = rr[in.b];
  float v;
  if (op >= KTIR_OP_NEGF && op < KTIR_OP_ADDF) {
    v = unop_simple(op, in.dt, a);
  } else if (op >= KTIR_OP_ADDI) {
    v = __int_as_float(binop_i_simple(op, __float_as_int(a), __float_as_int(b)));
  } else if (op >= KTIR_OP_ADDF) {
    v = binop_f_simple(op, in.dt, a, b);
  } else {
    switch (op) {
      case KTIR_OP_CONST: v = __int_as_float(in.imm); break;
      case KTIR_OP_LANE: {
        const double d = ((const double*)P.lane_scalars)[lane * P.n_lane_scalars + in.aux];
        v = is_float_dt(in.dt) ? round_to((float)d, in.dt) : __int_as_float((int)(long long)d);
        break;
      }
      case KTIR_OP_CAST: v = cast_val(a, in.aux, in.dt); break;
      case KTIR_OP_BITCAST: v = a; break;
      case KTIR_OP_SELECT: v = __float_as_int(a) ? b : rr[in.c]; break;
      case KTIR_OP_FMA: v = round_to(__fadd_rn(__fmul_rn(a, b), rr[in.c]), in.dt); break;
      case KTIR_OP_CMPF: v = __int_as_float(cmp_f(in.aux, a, b)); break;
      case KTIR_OP_CMPI: v = __int_as_float(cmp_i(in.aux, __float_as_int(a), __float_as_int(b))); break;
      default: v = 0.f;
    }
  }
  rr[in.dst] = v;
}

template <int E>
__global__ __launch_bounds__(256) void prog_rowchain(const ktir_prog_t P, const RcPlan R, int tpr_log2,
                                                     int64_t total_rows) {
  __shared__ float xch[512];
  // row registers: one copy per wavefront (a group spans whole wavefronts) or
  // per group (several groups share a wavefront); each copy is written and
  // read by one wavefront only, in program order
  __shared__ float regs[8][KTIR_NREG];
  const int tpr = 1 << tpr_log2;
  const int grp = threadIdx.x >> tpr_log2, t = threadIdx.x & (tpr - 1);
  const int rpw = 256 >> tpr_log2;
  float* rr = regs[tpr >= 64 ? (threadIdx.x >> 6) : grp];
  const int nd = P.ndim;
  const int64_t inner = P.shape[nd - 1];
  int64_t rows_per_lane = 1;
  for (int d = 0; d < nd - 1; ++d) rows_per_lane *= P.shape[d];
  for (int64_t row0 = (int64_t)blockIdx.x * rpw; row0 < total_rows; row0 += (int64_t)gridDim.x * rpw) {
    const int64_t row = row0 + grp;
    const bool active = row < total_rows;
    const int64_t rw = active ? row : total_rows - 1;
    const int64_t lane = rw / rows_per_lane;
    int64_t rr_idx = rw - lane * rows_per_lane;
    int64_t idx[KTIR_MAX_DIMS - 1] = {0, 0, 0};
#pragma unroll
    for (int d = KTIR_MAX_DIMS - 2; d >= 0; --d) {
      if (d < nd - 1) {
        const int64_t q = rr_idx / P.shape[d];
        idx[d] = rr_idx - q * P.shape[d];
        rr_idx = q;
      }
    }
    // element offset of column 0 of this row in leaf L
    auto row_base = [&](const ktir_leaf_t& L) {
      int64_t e = lane_offset(L, lane);
#pragma unroll
      for (int d = 0; d < KTIR_MAX_DIMS - 1; ++d)
        if (d < nd - 1) e += idx[d] * L.strides[d];
      return e;
    };
    float c0[E], c1[E], kept[E];
    load_row<E>(P.leaves[R.slot_leaf[0]], row_base(P.leaves[R.slot_leaf[0]]), t, tpr, c0);
    if (R.n_slots > 1) load_row<E>(P.leaves[R.slot_leaf[1]], row_base(P.leaves[R.slot_leaf[1]]), t, tpr, c1);
    else
#pragma unroll
      for (int e = 0; e < E; ++e) c1[e] = 0.f;
    for (int si = 0; si < R.n_steps; ++si) {
      const RcStep& S = R.steps[si];
      if (S.kind == 0) {
        row_exec(P, P.instr[S.pc], rr, lane);
        continue;
      }
      if (S.kind == 2) {
        const ktir_leaf_t& L = P.leaves[S.st_leaf];
        const int64_t e = row_base(L);
        if (active && t == 0 && e >= L.lo && e < L.hi) store_elem(L.ptr, e, L.dtype, rr[P.instr[S.pc].a]);
        continue;
      }
      float v[E];
      int oi = 0;
      if (S.reuse) {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = kept[e];
        oi = 2;
      } else if (S.head == 1) {
        const float m = rr[S.ops[0].idx];
        if (S.src) {
#pragma unroll
          for (int e = 0; e < E; ++e) v[e] = exp_hw(__fsub_rn(c1[e], m));
        } else {
#pragma unroll
          for (int e = 0; e < E; ++e) v[e] = exp_hw(__fsub_rn(c0[e], m));
        }
        oi = 2;
      } else if (S.head == 2) {
        if (S.src) {
#pragma unroll
          for (int e = 0; e < E; ++e) v[e] = __fmul_rn(c1[e], c1[e]);
        } else {
#pragma unroll
          for (int e = 0; e < E; ++e) v[e] = __fmul_rn(c0[e], c0[e]);
        }
        oi = 1;
      } else if (S.src) {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = c1[e];
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = c0[e];
      }
      if (S.save) {
#pragma unroll
        for (int e = 0; e < E; ++e) kept[e] = v[e];
      }
      for (; oi < S.n_ops; ++oi) {
        const RcOp o = S.ops[oi];
        apply_op<E>(o, v, o.kind == 1 ? rr[o.idx] : 0.f, c0, c1);
      }
      if (S.end == 0) {
        const float f = fold_group<E>(v, S.fold_op, S.fold_dt, tpr, xch);
        rr[S.dst] = f;
      } else if (active) {
        store_row<E>(P.leaves[S.st_leaf], row_base(P.leaves[S.st_leaf]), t, tpr, v);
      }
    }
    (void)inner;
    __syncthreads();    // the next row's folds reuse xch
  }
}

// ---- one wavefront per row, rows staged in LDS -----------------------------------
//
// For rows of n = 128 K elements whose cached leaves fill whole 1 KB blocks: a
// wavefront owns a row, the row's cached leaves move HBM -> registers -> LDS
// (the next row's loads are in flight while this one is computed; leaves that
// are the same for every row are staged once), and lane l handles the element
// pairs 128 k + 2 l + {0, 1}, k < K.  Folds: the lane's pairs go through the
// in-thread levels of the halving tree (the bits of k), then lanes
// l ^ 32 .. l ^ 1, then the two elements of the pair.

// Self-contained plan of the row-wave kernel (copied to LDS by each
// workgroup, so the kernel's control reads are LDS reads that never wait
// behind the row loads in flight).
struct RwLeaf {
  uint64_t ptr, lane_base;
  int64_t base, lane_stride, lo, hi;
  int64_t strides[KTIR_MAX_DIMS - 1];   // outer dims
  int32_t dtype, esize;
};

struct RwHead {
  int8_t kind, src, n_ops, end, fold_op, fold_dt, dst, out;   // out: store leaf (index into RwPlan.leaf)
  int8_t head, pad[3];
  ktir_instr_t ins;                     // kind 0: the row instruction; kind 2: the row-level store
};

struct RwStep : RwHead {
  RcOp ops[RC_MAX_OPS];
};

struct RwPlan {
  int32_t n_steps, n_slots, nd, n_leaves;
  int64_t shape[KTIR_MAX_DIMS];
  uint64_t lane_scalars;
  int64_t n_lane_scalars;
  int32_t off[2], bytes[2], inv[2];
  RwLeaf leaf[4];                       // 0, 1: cached slots; then store leaves
  RwStep steps[RC_MAX_STEPS];
};

struct RwOut {          // the store leaf of a pass, by value (no pointer into the kernel arguments)
  uint64_t ptr;
  int64_t lo, hi, base;
  int dt;
};

__device__ __forceinline__ void global_pair_store(const RwOut& L, int64_t e0, float a, float b) {
  if (e0 >= L.lo && e0 + 2 <= L.hi) {
    switch (L.dt) {
      case KTIR_F32: store_pair<KTIR_F32>((void*)L.ptr, e0, a, b); return;
      case KTIR_BF16: store_pair<KTIR_BF16>((void*)L.ptr, e0, a, b); return;
      default: store_pair<KTIR_F16>((void*)L.ptr, e0, a, b); return;
    }
  }
  if (e0 >= L.lo && e0 < L.hi) store_elem(L.ptr, e0, L.dt, a);
  if (e0 + 1 >= L.lo && e0 + 1 < L.hi) store_elem(L.ptr, e0 + 1, L.dt, b);
}

__device__ __forceinline__ float fold_rt(int op, float x, float y) {
  switch (op) {
    case KTIR_OP_ADDF: return __fadd_rn(x, y);
    case KTIR_OP_MULF: return __fmul_rn(x, y);
    case KTIR_OP_MAXIMUMF: return maxnan(x, y);
    default: return minnan(x, y);
  }
}

// a fold combine of any fold op in the fold's dtype (sums and products
// rounded to f16 / bf16 at every level, as the reference's tree fold on a
// narrow tile does; a min / max is one of its operands)
__device__ __forceinline__ float fold_any(int op, int dt, float x, float y) {
  switch (op) {
    case KTIR_OP_ADDF: return round_to(__fadd_rn(x, y), dt);
    case KTIR_OP_MULF: return round_to(mul_keep(x, y), dt);
    case KTIR_OP_MAXIMUMF: return maxnan(x, y);
    case KTIR_OP_MINIMUMF: return minnan(x, y);
    case KTIR_OP_MAXNUMF: return fmaxf(x, y);
    default: return fminf(x, y);
  }
}

// Pairs k = c NB + q (c < B) of a cached row in LDS: v[2c], v[2c + 1] are the
// elements 128 k + 2 l + {0, 1}.
template <int B, int NB>
__device__ __forceinline__ void rw_lds_row(const uint8_t* sp, int dp, int q, int l, float (&v)[2 * B]) {
  if (dp == KTIR_F32) {
#pragma unroll
    for (int c = 0; c < B; ++c) {
      const gf2 w = *(const gf2*)(sp + 4 * (128 * (c * NB + q) + 2 * l));
      v[2 * c] = w[0];
      v[2 * c + 1] = w[1];
    }
  } else if (dp == KTIR_BF16) {
#pragma unroll
    for (int c = 0; c < B; ++c) {
      const uint32_t w = *(const uint32_t*)(sp + 2 * (128 * (c * NB + q) + 2 * l));
      v[2 * c] = __uint_as_float(w << 16);
      v[2 * c + 1] = __uint_as_float(w & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int c = 0; c < B; ++c) {
      const uint32_t w = *(const uint32_t*)(sp + 2 * (128 * (c * NB + q) + 2 * l));
      v[2 * c] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
      v[2 * c + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
    }
  }
}

// v <- v op c (or c op v when swapped), element by element
template <int E>
__device__ __forceinline__ void rw_binary(int op, bool swap, float (&v)[E], const float (&c)[E]) {
#define RW_B(expr)                                           \
  {                                                          \
    if (swap) {                                              \
      _Pragma("unroll") for (int e = 0; e < E; ++e) {        \
        const float x = c[e], y = v[e];                      \
        v[e] = (expr);                                       \
      }                                                      \
    } else {                                                 \
      _Pragma("unroll") for (int e = 0; e < E; ++e) {        \
        const float x = v[e], y = c[e];                      \
        v[e] = (expr);                                       \
      }                                                      \
    }                                                        \
    return;                                                  \
  }
  switch (op) {
    case KTIR_OP_ADDF: RW_B(__fadd_rn(x, y))
    case KTIR_OP_SUBF: RW_B(__fsub_rn(x, y))
    case KTIR_OP_MULF: RW_B(__fmul_rn(x, y))
    case KTIR_OP_DIVF: RW_B(__fdiv_rn(x, y))
    case KTIR_OP_MAXIMUMF: RW_B(maxnan(x, y))
    case KTIR_OP_MINIMUMF: RW_B(minnan(x, y))
    case KTIR_OP_MAXNUMF: RW_B(fmaxf(x, y))
    case KTIR_OP_MINNUMF: RW_B(fminf(x, y))
  }
#undef RW_B
}

// fold of the step's B pairs to one pair: the halving tree over c (c with
// c + B/2, then c + B/4, ...), the left operand the lower index
template <int B, int OP>
__device__ __forceinline__ void rw_fold_step(float (&v)[2 * B]) {
#pragma unroll
  for (int h = B / 2; h >= 1; h >>= 1) {
#pragma unroll
    for (int c = 0; c < h; ++c) {
      v[2 * c] = fold_op<OP, KTIR_F32>(v[2 * c], v[2 * (c + h)]);
      v[2 * c + 1] = fold_op<OP, KTIR_F32>(v[2 * c + 1], v[2 * (c + h) + 1]);
    }
  }
}

// the same halving tree for any fold op and dtype (op and dtype dispatched
// once; a min / max needs no rounding, so its dtype does not matter)
template <int B, int OP, int DT>
__device__ __forceinline__ void rw_fold_step_t(float (&v)[2 * B]) {
#pragma unroll
  for (int h = B / 2; h >= 1; h >>= 1) {
#pragma unroll
    for (int c = 0; c < h; ++c) {
      v[2 * c] = fold_op<OP, DT>(v[2 * c], v[2 * (c + h)]);
      v[2 * c + 1] = fold_op<OP, DT>(v[2 * c + 1], v[2 * (c + h) + 1]);
    }
  }
}

template <int B, int OP>
__device__ __forceinline__ void rw_fold_step_dt(float (&v)[2 * B], int dt) {
  if (dt == KTIR_F16) rw_fold_step_t<B, OP, KTIR_F16>(v);
  else if (dt == KTIR_BF16) rw_fold_step_t<B, OP, KTIR_BF16>(v);
  else rw_fold_step_t<B, OP, KTIR_F32>(v);
}

template <int B>
__device__ __forceinline__ void rw_fold_exact(float (&v)[2 * B], int op, int dt) {
  switch (op) {
    case KTIR_OP_ADDF: rw_fold_step_dt<B, KTIR_OP_ADDF>(v, dt); return;
    case KTIR_OP_MULF: rw_fold_step_dt<B, KTIR_OP_MULF>(v, dt); return;
    case KTIR_OP_MAXIMUMF: rw_fold_step_t<B, KTIR_OP_MAXIMUMF, KTIR_F32>(v); return;
    case KTIR_OP_MINIMUMF: rw_fold_step_t<B, KTIR_OP_MINIMUMF, KTIR_F32>(v); return;
    case KTIR_OP_MAXNUMF: rw_fold_step_t<B, KTIR_OP_MAXNUMF, KTIR_F32>(v); return;
    default: rw_fold_step_t<B, KTIR_OP_MINNUMF, KTIR_F32>(v); return;
  }
}

// One pass of a row.  Lane l holds the K pairs k of its row (elements
// 128 k + 2 l + {0, 1}) as NB steps of B pairs, step q holding k = c NB + q:
// the whole step's values are in registers, so every op of the pass is
// dispatched once per step.  A fold pass reduces each step by the halving
// tree over c (the tree's levels over the high bits of k), the NB <= 4 step
// roots by its levels over the low bits of k (the bits of q), then lanes
// l ^ 32 .. l ^ 1, then the two elements of the pair.  A store pass writes every pair.
template <int K, bool FOLDX>
__device__ __forceinline__ float rw_pass(const RwHead& S, const RcOp* ops, const uint8_t* s0, int d0,
                                         const uint8_t* s1, int d1, const RowRegs& rr, const RwOut& SL,
                                         bool out_in_range, int l) {
  constexpr int B = K < 16 ? K : 16;
  constexpr int NB = K / B;
  static_assert(NB <= 4, "at most four steps per row");
  const bool fold = S.end == 0;
  const int fop = S.fold_op;
  const int fdt = S.fold_dt;
  const int n_ops = S.n_ops;
  const uint8_t* sp = S.src ? s1 : s0;
  const int dp = S.src ? d1 : d0;
  float ra[NB], rb[NB];
#pragma unroll
  for (int q = 0; q < NB; ++q) {
    float v[2 * B];
    rw_lds_row<B, NB>(sp, dp, q, l, v);
    int oi = 0;
    if (S.head == 1) {
      const float m = rr.get(uniform_copy(ops[0]).idx);
#pragma unroll
      for (int e = 0; e < 2 * B; ++e) v[e] = exp_hw(__fsub_rn(v[e], m));
      oi = 2;
    } else if (S.head == 2) {
#pragma unroll
      for (int e = 0; e < 2 * B; ++e) v[e] = __fmul_rn(v[e], v[e]);
      oi = 1;
    }
    for (; oi < n_ops; ++oi) {
      const RcOp o = uniform_copy(ops[oi]);
      if (o.kind == 2) {
        float c[2 * B];
        rw_lds_row<B, NB>(o.idx ? s1 : s0, o.idx ? d1 : d0, q, l, c);
        rw_binary<2 * B>(o.op, o.swap, v, c);
      } else if (o.kind == 3) {
        float c[2 * B];
#pragma unroll
        for (int e = 0; e < 2 * B; ++e) c[e] = v[e];
        rw_binary<2 * B>(o.op, false, v, c);
      } else {
        apply_op<2 * B>(o, v, o.kind == 1 ? rr.get(o.idx) : 0.f, v, v);
      }
    }
    if (!fold) {
      if (out_in_range) {
        switch (SL.dt) {
          case KTIR_F32:
#pragma unroll
            for (int c = 0; c < B; ++c)
              store_pair<KTIR_F32>((void*)SL.ptr, SL.base + 128 * (c * NB + q) + 2 * l, v[2 * c], v[2 * c + 1]);
            break;
          case KTIR_BF16:
#pragma unroll
            for (int c = 0; c < B; ++c)
              store_pair<KTIR_BF16>((void*)SL.ptr, SL.base + 128 * (c * NB + q) + 2 * l, v[2 * c], v[2 * c + 1]);
            break;
          default:
#pragma unroll
            for (int c = 0; c < B; ++c)
              store_pair<KTIR_F16>((void*)SL.ptr, SL.base + 128 * (c * NB + q) + 2 * l, v[2 * c], v[2 * c + 1]);
        }
      } else {
#pragma unroll
        for (int c = 0; c < B; ++c) global_pair_store(SL, SL.base + 128 * (c * NB + q) + 2 * l, v[2 * c], v[2 * c + 1]);
      }
      continue;
    }
    if constexpr (FOLDX) {
      rw_fold_exact<B>(v, fop, fdt);
    } else {
      switch (fop) {
        case KTIR_OP_ADDF: rw_fold_step<B, KTIR_OP_ADDF>(v); break;
        case KTIR_OP_MULF: rw_fold_step<B, KTIR_OP_MULF>(v); break;
        case KTIR_OP_MAXIMUMF: rw_fold_step<B, KTIR_OP_MAXIMUMF>(v); break;
        default: rw_fold_step<B, KTIR_OP_MINIMUMF>(v); break;
      }
    }
    ra[q] = v[0];
    rb[q] = v[1];
  }
  if (!fold) return 0.f;
  // the tree's levels over the bits of q
#pragma unroll
  for (int h = NB / 2; h >= 1; h >>= 1) {
#pragma unroll
    for (int q = 0; q < h; ++q) {
      ra[q] = FOLDX ? fold_any(fop, fdt, ra[q], ra[q + h]) : fold_rt(fop, ra[q], ra[q + h]);
      rb[q] = FOLDX ? fold_any(fop, fdt, rb[q], rb[q + h]) : fold_rt(fop, rb[q], rb[q + h]);
    }
  }
  float a = ra[0], b = rb[0];
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) {
    a = FOLDX ? fold_any(fop, fdt, a, __shfl_xor(a, s)) : fold_rt(fop, a, __shfl_xor(a, s));
    b = FOLDX ? fold_any(fop, fdt, b, __shfl_xor(b, s)) : fold_rt(fop, b, __shfl_xor(b, s));
  }
  return FOLDX ? fold_any(fop, fdt, a, b) : fold_rt(fop, a, b);
}

// Position of row r: its lane (core) and its index in each outer dim.  Rows,
// lanes and dims are below 2^31 (checked at launch): 32-bit division.
struct RwPos {
  int32_t lane;
  int32_t idx[KTIR_MAX_DIMS - 1];
};

template <typename PL>
__device__ __forceinline__ RwPos rw_pos(const PL& SP, int64_t r, int32_t rows_per_lane) {
  RwPos p;
  const uint32_t ru = (uint32_t)r, rpl = (uint32_t)rows_per_lane;
  const uint32_t lane = ru / rpl;
  uint32_t t = ru - lane * rpl;
  p.lane = (int32_t)lane;
  const int nd = __builtin_amdgcn_readfirstlane(SP.nd);
#pragma unroll
  for (int d = KTIR_MAX_DIMS - 2; d >= 0; --d) {
    p.idx[d] = 0;
    if (d < nd - 1) {
      const uint32_t ext = (uint32_t)__builtin_amdgcn_readfirstlane((int)SP.shape[d]);
      const uint32_t q = t / ext;
      p.idx[d] = (int32_t)(t - q * ext);
      t = q;
    }
  }
  return p;
}

// element offset of column 0 of the row at p in leaf L
__device__ __forceinline__ int64_t rw_row_base(const RwLeaf& L, const RwPos& p) {
  int64_t e = L.lane_base ? uni(((const KTIR_G(int64_t)*)L.lane_base)[p.lane]) : L.base + (int64_t)p.lane * L.lane_stride;
#pragma unroll
  for (int d = 0; d < KTIR_MAX_DIMS - 1; ++d) e += (int64_t)p.idx[d] * L.strides[d];
  return e;
}

// registers <- row r of the non-invariant slots; false (nothing read) when a
// row is not wholly inside its allocation
template <int NQ>
__device__ __forceinline__ bool rw_load_regs(const RwPlan& SP, uint4 (&st)[NQ], const RwPos& p, int64_t inner, int l) {
  const int n_slots = __builtin_amdgcn_readfirstlane(SP.n_slots);
  int q0 = 0;
  for (int s = 0; s < n_slots; ++s) {
    if (__builtin_amdgcn_readfirstlane(SP.inv[s])) continue;
    const RwLeaf L = uniform_copy(SP.leaf[s]);
    const int64_t x = rw_row_base(L, p);
    if (x < L.lo || x + inner > L.hi) return false;
  }
  for (int s = 0; s < n_slots; ++s) {
    if (__builtin_amdgcn_readfirstlane(SP.inv[s])) continue;
    const RwLeaf L = uniform_copy(SP.leaf[s]);
    const int64_t x = rw_row_base(L, p);
    const int nq = __builtin_amdgcn_readfirstlane(SP.bytes[s]) >> 10;
    const KTIR_G(uint8_t)* src = (const KTIR_G(uint8_t)*)L.ptr + x * L.esize + 16 * l;
#pragma unroll
    for (int i = 0; i < NQ; ++i)
      if (i >= q0 && i < q0 + nq) st[i] = __builtin_bit_cast(uint4, *(const KTIR_G(gu4)*)(src + 1024 * (i - q0)));
    q0 += nq;
  }
  return true;
}

template <int NQ>
__device__ __forceinline__ void rw_store_regs(const RwPlan& SP, const uint4 (&st)[NQ], uint8_t* lds, int l) {
  const int n_slots = __builtin_amdgcn_readfirstlane(SP.n_slots);
  int q0 = 0;
  for (int s = 0; s < n_slots; ++s) {
    if (__builtin_amdgcn_readfirstlane(SP.inv[s])) continue;
    const int nq = __builtin_amdgcn_readfirstlane(SP.bytes[s]) >> 10;
    uint8_t* dst = lds + __builtin_amdgcn_readfirstlane(SP.off[s]) + 16 * l;
#pragma unroll
    for (int i = 0; i < NQ; ++i)
      if (i >= q0 && i < q0 + nq) *(uint4*)(dst + 1024 * (i - q0)) = st[i];
    q0 += nq;
  }
}

// element by element into LDS with the reference's out-of-range read rule (0)
__device__ __forceinline__ void rw_stage_slow(const RwPlan& SP, int s, const RwPos& p,
                                              int64_t inner, uint8_t* lds, int l) {
  const RwLeaf L = uniform_copy(SP.leaf[s]);
  const int64_t e = rw_row_base(L, p);
  uint8_t* dst = lds + __builtin_amdgcn_readfirstlane(SP.off[s]);
  for (int64_t i = l; i < inner; i += 64) {
    const int64_t x = e + i;
    const float v = (x >= L.lo && x < L.hi) ? load_elem(L.ptr, x, L.dtype) : 0.f;
    if (L.dtype == KTIR_F32) ((float*)dst)[i] = v;
    else if (L.dtype == KTIR_BF16) ((uint16_t*)dst)[i] = (uint16_t)(__float_as_uint(v) >> 16);
    else ((_Float16*)dst)[i] = (_Float16)v;
  }
}

template <typename PL, typename RR>
__device__ __forceinline__ void rw_row_exec(const PL& SP, const ktir_instr_t in, RR& rr, int64_t lane) {
  const int op = in.op;
  const float a = rr.get(in.a), b = rr.get(in.b);
  float v;
  if (op >= KTIR_OP_NEGF && op < KTIR_OP_ADDF) {
    v = unop_simple(op, in.dt, a);
  } else if (op >= KTIR_OP_ADDI) {
    v = __int_as_float(binop_i_simple(op, __float_as_int(a), __float_as_int(b)));
  } else if (op >= KTIR_OP_ADDF) {
    v = binop_f_simple(op, in.dt, a, b);
  } else {
    switch (op) {
      case KTIR_OP_CONST: v = __int_as_float(in.imm); break;
      case KTIR_OP_LANE: {
        const double d = ((const KTIR_G(double)*)uni((int64_t)SP.lane_scalars))[lane * uni(SP.n_lane_scalars) + in.aux];
        v = is_float_dt(in.dt) ? round_to((float)d, in.dt) : __int_as_float((int)(long long)d);
        break;
      }
      case KTIR_OP_CAST: v = cast_val(a, in.aux, in.dt); break;
      case KTIR_OP_BITCAST: v = a; break;
      case KTIR_OP_SELECT: v = __float_as_int(a) ? b : rr.get(in.c); break;
      case KTIR_OP_FMA: v = round_to(__fadd_rn(__fmul_rn(a, b), rr.get(in.c)), in.dt); break;
      case KTIR_OP_CMPF: v = __int_as_float(cmp_f(in.aux, a, b)); break;
      case KTIR_OP_CMPI: v = __int_as_float(cmp_i(in.aux, __float_as_int(a), __float_as_int(b))); break;
      default: v = 0.f;
    }
  }
  rr.set(in.dst, __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v))));
}

// Row staging: the next row's cached leaves are read into registers (NQ
// 16-byte chunks per lane: chunk i of lane l is bytes 1024 i + 16 l of the
// slots' rows laid end to end) while the current row is computed from LDS,
// then written to LDS.  Plain loads and LDS stores: the compiler waits for
// the loaded registers only where they are stored.
// three wavefronts per SIMD where the registers fit without spilling
template <int K, int NQ>
constexpr int rw_waves() { return (K == 32 && NQ == 8) || (K == 16 && NQ == 4) || K <= 8 ? 3 : 2; }

template <int K, int NQ, bool FOLDX = false>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(rw_waves<K, NQ>()))) void prog_rowwave(const RwPlan Pk, int64_t total_rows) {
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ RwPlan SP;
  RowRegs rr{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int l = threadIdx.x;
  {
    const int* src = (const int*)&Pk;
    int* dst = (int*)&SP;
    for (int i = l; i < (int)(sizeof(RwPlan) / 4); i += 64) dst[i] = src[i];
  }
  __syncthreads();
  const int n_steps = __builtin_amdgcn_readfirstlane(SP.n_steps);
  const int n_slots = __builtin_amdgcn_readfirstlane(SP.n_slots);
  const int nd = __builtin_amdgcn_readfirstlane(SP.nd);
  int64_t shape[KTIR_MAX_DIMS];
#pragma unroll
  for (int d = 0; d < KTIR_MAX_DIMS; ++d) shape[d] = uni(SP.shape[d]);
  const int64_t inner = nd == 1 ? shape[0] : (nd == 2 ? shape[1] : (nd == 3 ? shape[2] : shape[3]));
  int64_t rows_per_lane = 1;
#pragma unroll
  for (int d = 0; d < KTIR_MAX_DIMS - 1; ++d)
    if (d < nd - 1) rows_per_lane *= shape[d];
  const int32_t rpl = (int32_t)rows_per_lane;
  uint4 st[NQ];
  int64_t r = blockIdx.x;
  RwPos pos = rw_pos(SP, r, rpl);
  if (r < total_rows) {
    for (int s = 0; s < n_slots; ++s)
      if (__builtin_amdgcn_readfirstlane(SP.inv[s])) rw_stage_slow(SP, s, pos, inner, lds, l);
    if (rw_load_regs<NQ>(SP, st, pos, inner, l)) {
      rw_store_regs<NQ>(SP, st, lds, l);
    } else {
      for (int s = 0; s < n_slots; ++s)
        if (!__builtin_amdgcn_readfirstlane(SP.inv[s])) rw_stage_slow(SP, s, pos, inner, lds, l);
    }
  }
  for (; r < total_rows; r += gridDim.x) {
    const int64_t rn = r + gridDim.x;
    const bool more = rn < total_rows;
    const RwPos pn = rw_pos(SP, more ? rn : r, rpl);
    const bool fast = more && rw_load_regs<NQ>(SP, st, pn, inner, l);
    const uint8_t* s0 = lds + __builtin_amdgcn_readfirstlane(SP.off[0]);
    const uint8_t* s1 = n_slots > 1 ? lds + __builtin_amdgcn_readfirstlane(SP.off[1]) : nullptr;
    const int d0 = __builtin_amdgcn_readfirstlane(SP.leaf[0].dtype);
    const int d1 = n_slots > 1 ? __builtin_amdgcn_readfirstlane(SP.leaf[1].dtype) : KTIR_F32;
    for (int si = 0; si < n_steps; ++si) {
      const RwHead S = uniform_copy(*(const RwHead*)&SP.steps[si]);
      if (S.kind == 0) {
        rw_row_exec(SP, S.ins, rr, pos.lane);
        continue;
      }
      if (S.kind == 2) {
        const RwLeaf L = uniform_copy(SP.leaf[S.out]);
        const int64_t e = rw_row_base(L, pos);
        if (l == 0 && e >= L.lo && e < L.hi) store_elem(L.ptr, e, L.dtype, rr.get(S.ins.a));
        continue;
      }
      RwOut SL{0, 0, 0, 0, KTIR_F32};
      bool in_range = false;
      if (S.end) {
        const RwLeaf L = uniform_copy(SP.leaf[S.out]);
        SL = RwOut{L.ptr, L.lo, L.hi, rw_row_base(L, pos), L.dtype};
        in_range = SL.base >= SL.lo && SL.base + inner <= SL.hi;
      }
      const float f = rw_pass<K, FOLDX>(S, SP.steps[si].ops, s0, d0, s1, d1, rr, SL, in_range, l);
      if (S.end == 0) rr.set(S.dst, __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(f))));
    }
    // the row's LDS reads are done (LDS operations of a wavefront complete in order)
    if (fast) {
      rw_store_regs<NQ>(SP, st, lds, l);
    } else if (more) {
      for (int s = 0; s < n_slots; ++s)
        if (!__builtin_amdgcn_readfirstlane(SP.inv[s])) rw_stage_slow(SP, s, pn, inner, lds, l);
    }
    pos = pn;
  }
}

// Upper bound on the workgroups of a row-kernel launch (0: none).  Every row
// kernel strides its workgroups over the rows, so any bound gives the same
// results; a small one makes each workgroup run many rows.
static int64_t g_row_grid_limit = 0;

int64_t row_grid_limit(int64_t blocks) {
  return g_row_grid_limit > 0 && blocks > g_row_grid_limit ? g_row_grid_limit : blocks;
}

// One resident wavefront per row stream: as many workgroups as the device
// holds at once (so no second, partial round of workgroups), each taking an
// equal share of the rows.
template <int K, int NQ, bool FOLDX = false>
static void launch_rowwave(const RwPlan& W, int lds_bytes, int64_t rows) {
  static int cached_lds = -1, cached_resident = 0;
  if (cached_lds != lds_bytes) {
    int per_cu = 0, cus = 0, dev = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, prog_rowwave<K, NQ, FOLDX>, 64, lds_bytes) != hipSuccess ||
        hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu < 1 || cus < 1) {
      per_cu = 1;
      cus = 256;
    }
    cached_resident = per_cu * cus;
    cached_lds = lds_bytes;
  }
  const int64_t per_block = (rows + cached_resident - 1) / cached_resident;
  const int64_t blocks = row_grid_limit((rows + per_block - 1) / per_block);
  hipLaunchKernelGGL((prog_rowwave<K, NQ, FOLDX>), dim3((unsigned)blocks), dim3(64), lds_bytes, stream(), W, rows);
}

template <int K>
static bool pick_nq(int nq, const RwPlan& W, int lds_bytes, int64_t rows, bool foldx) {
  // K/4 chunks: one 16-bit slot; K/2: one f32 slot or two 16-bit slots; K: more (at most 16 chunks)
  constexpr int A = K / 4 > 0 ? K / 4 : 1, B = K / 2, C = K;
  if (foldx) {
    // plans with f16 / bf16 or NaN-ignoring folds: one or two row slots
    if (nq <= A) { launch_rowwave<K, A, true>(W, lds_bytes, rows); return true; }
    if constexpr (B <= 16) {
      if (nq <= B) { launch_rowwave<K, B, true>(W, lds_bytes, rows); return true; }
    }
    return false;
  }
  if (nq <= A) { launch_rowwave<K, A>(W, lds_bytes, rows); return true; }
  if constexpr (B <= 16) {
    if (nq <= B) { launch_rowwave<K, B>(W, lds_bytes, rows); return true; }
  }
  if constexpr (C <= 16) {
    if (nq <= C) { launch_rowwave<K, C>(W, lds_bytes, rows); return true; }
  }
  return false;
}

static RwLeaf rw_leaf(const ktir_prog_t& P, int leaf) {
  const ktir_leaf_t& L = P.leaves[leaf];
  RwLeaf o{};
  o.ptr = L.ptr;
  o.lane_base = L.lane_base;
  o.base = L.base;
  o.lane_stride = L.lane_stride;
  o.lo = L.lo;
  o.hi = L.hi;
  for (int d = 0; d < KTIR_MAX_DIMS - 1; ++d) o.strides[d] = d < P.ndim - 1 ? L.strides[d] : 0;
  o.dtype = L.dtype;
  o.esize = L.dtype == KTIR_F32 ? 4 : 2;
  return o;
}

static bool try_launch_rowwave(const ktir_prog_t& P, const RcPlan& R, int64_t rows, int64_t inner, bool foldx) {
  if (inner % 128 || inner / 128 < 4 || inner / 128 > 64) return false;
  if (rows > INT32_MAX) return false;   // row positions use 32-bit arithmetic
  for (int d = 0; d < P.ndim; ++d)
    if (P.shape[d] > INT32_MAX) return false;
  RwPlan W{};
  W.n_steps = R.n_steps;
  W.n_slots = R.n_slots;
  W.nd = P.ndim;
  for (int d = 0; d < KTIR_MAX_DIMS; ++d) W.shape[d] = d < P.ndim ? P.shape[d] : 1;
  W.lane_scalars = P.lane_scalars;
  W.n_lane_scalars = P.n_lane_scalars;
  const int nd = P.ndim;
  int32_t off = 0, nq = 0;
  for (int s = 0; s < R.n_slots; ++s) {
    const ktir_leaf_t& L = P.leaves[R.slot_leaf[s]];
    W.leaf[s] = rw_leaf(P, R.slot_leaf[s]);
    W.bytes[s] = (int32_t)(inner * W.leaf[s].esize);
    if (W.bytes[s] % 1024) return false;
    if (!(L.flags & (W.leaf[s].esize == 4 ? KTIR_LEAF_VEC : KTIR_LEAF_VEC8))) return false;   // 16-byte aligned rows
    bool inv = L.lane_base == 0 && L.lane_stride == 0;
    for (int d = 0; d < nd - 1; ++d) inv = inv && (L.strides[d] == 0 || P.shape[d] == 1);
    W.inv[s] = inv;
    W.off[s] = off;
    off += W.bytes[s];
    if (!inv) nq += W.bytes[s] >> 10;
  }
  int n_leaves = R.n_slots;
  for (int i = 0; i < R.n_steps; ++i) {
    const RcStep& S = R.steps[i];
    RwStep& D = W.steps[i];
    D.kind = S.kind;
    if (S.kind == 1 && S.end == 0 && S.fold_dt != KTIR_F32 && !foldx) return false;
    if (S.kind == 0 || S.kind == 2) D.ins = P.instr[S.pc];
    if (S.kind == 2 || (S.kind == 1 && S.end == 1)) {
      if (n_leaves == 4) return false;
      W.leaf[n_leaves] = rw_leaf(P, S.st_leaf);
      D.out = (int8_t)n_leaves++;
    }
    D.src = S.src;
    D.n_ops = S.n_ops;
    D.end = S.end;
    D.fold_op = S.fold_op;
    D.fold_dt = S.fold_dt;
    D.dst = S.dst;
    D.head = S.head;
    for (int o = 0; o < RC_MAX_OPS; ++o) D.ops[o] = S.ops[o];
  }
  W.n_leaves = n_leaves;
  if (off > 64 * 1024 || nq > 16) return false;
  switch (inner / 128) {
    case 4: return pick_nq<4>(nq, W, off, rows, foldx);
    case 8: return pick_nq<8>(nq, W, off, rows, foldx);
    case 16: return pick_nq<16>(nq, W, off, rows, foldx);
    case 32: return pick_nq<32>(nq, W, off, rows, foldx);
    case 64: return pick_nq<64>(nq, W, off, rows, foldx);
  }
  return false;
}

// ---- fixed-form row kernels -----------------------------------------------------
//
// Two row programs get kernels whose passes are straight-line code; the pass
// plan only supplies their registers, rows and the row instructions between
// the folds:
//   softmax:    m <- max fold of x; [row instructions]; s <- add fold of
//               exp(x - m'); [row instructions]; y <- exp(x - m') / s'
//               (exp(x - m') computed once and kept);
//   norm-scale: a <- add fold of x * x; [row instructions];
//               y <- (x * r) * w, (x * w) * r or x * r   (RMSNorm).
// A wavefront owns a row of n = 512 NQ 16-bit elements.  Lane l holds chunk i
// (i < NQ) as the elements 512 i + 8 l + j, j < 8, read and written as 16
// bytes; the next row's chunks are in flight while the current row is
// computed.  No LDS: the row's values, exp(x - m') and the weights stay in
// registers.  The add fold follows the reference's halving tree over this
// layout: the chunk bits in registers, the lane bits by shuffles (lanes
// l ^ 32 .. l ^ 1), the bits of j in registers.  The max fold's result does
// not depend on the order: the largest element, or NaN if any element is NaN.
//
// The same two forms computed in f16, as the reference's own row loops
// write them (every op on an f16 tile, so every step rounded to f16):
//   softmax16: m <- max fold (maxnumf or maximumf) of x; d = f16(x - m');
//              e = f16(exp d); s <- f16 add fold of e; y = f16(e / s');
//   norm16:    a <- f16 add fold of f16(x * x); y = f16(f16(x * r) * w) (or
//              w first, or no w).
// NumPy's f16 add, sub and mul round the f32 result of two f16 values, which
// is the correctly rounded f16 result (f32 has at least 2 * 11 + 2 bits), so
// packed f16 instructions give the same bits; exp is the hardware exp2
// rounded to f16 (within one f16 ulp of NumPy's, as the general kernels'
// exp), and the division a quotient within one f32 ulp rounded to f16.
constexpr int RF_MAX_ROW = 8;
enum { RF_SOFTMAX = 1, RF_NORM = 2, RF_SOFTMAX16 = 3, RF_NORM16 = 4 };

struct RfPlan {
  int32_t nd, has_w, w_first, n_row0, n_row1, numf;   // numf: softmax16's max ignores NaN
  int64_t shape[KTIR_MAX_DIMS];
  uint64_t lane_scalars;
  int64_t n_lane_scalars;
  RwLeaf x, w, y;
  int8_t fold0, fold1;        // registers the folds write
  int8_t m, s;                // softmax: the subtracted register and the divisor; norm-scale: s the multiplier
  int32_t pad1;
  ktir_instr_t row0[RF_MAX_ROW], row1[RF_MAX_ROW];   // after the first and the second fold
};

template <int DT>
__device__ __forceinline__ void rf_unpack(const gu4 c, float (&v)[8]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t u = c[k];
    if (DT == KTIR_BF16) {
      v[2 * k] = __uint_as_float(u << 16);
      v[2 * k + 1] = __uint_as_float(u & 0xffff0000u);
    } else {
      v[2 * k] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u & 0xffffu));
      v[2 * k + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(u >> 16));
    }
  }
}

// eight values rounded to nearest-even in DT, packed
template <int DT>
__device__ __forceinline__ gu4 rf_pack(const float (&v)[8]) {
  gu4 c;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (DT == KTIR_BF16)
      c[k] = (__float_as_uint(round_bf16(v[2 * k])) >> 16) | (__float_as_uint(round_bf16(v[2 * k + 1])) & 0xffff0000u);
    else
      c[k] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * k]) |
             ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * k + 1]) << 16);
  }
  return c;
}

// as rf_pack, f16 pairs converted by one instruction (v_cvt_pk_f16_f32, round
// to nearest even); the row kernels whose register count it does not raise
template <int DT>
__device__ __forceinline__ gu4 rf_pack2(const float (&v)[8]) {
  if (DT == KTIR_BF16) return rf_pack<DT>(v);
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  gu4 c;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const f2 x = {v[2 * k], v[2 * k + 1]};
    c[k] = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, h2));
  }
  return c;
}

// the chunks of the 16-bit row at element e0 of L: 16-byte loads when the row
// lies inside [lo, hi), else element by element (out-of-range elements read 0)
template <int NQ>
__device__ __forceinline__ void rf_load(const RwLeaf& L, int64_t e0, int l, gu4 (&c)[NQ]) {
  if (e0 >= L.lo && e0 + 512 * NQ <= L.hi) {
    const KTIR_G(uint8_t)* p = (const KTIR_G(uint8_t)*)L.ptr + 2 * e0 + 16 * l;
#pragma unroll
    for (int i = 0; i < NQ; ++i) c[i] = *(const KTIR_G(gu4)*)(p + 1024 * i);
    return;
  }
  const KTIR_G(uint16_t)* p = (const KTIR_G(uint16_t)*)L.ptr;
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int64_t e = e0 + 512 * i + 8 * l + 2 * k;
      const uint32_t a = (e >= L.lo && e < L.hi) ? p[e] : 0u;
      const uint32_t b = (e + 1 >= L.lo && e + 1 < L.hi) ? p[e + 1] : 0u;
      c[i][k] = a | (b << 16);
    }
  }
}

// chunk i of the row at element e0 of L: a streaming 16-byte store when the
// row lies inside [lo, hi) (`in`), else the in-range elements only
__device__ __forceinline__ void rf_store(const RwLeaf& L, int64_t e0, bool in, int i, int l, const gu4 c) {
  const int64_t e = e0 + 512 * i + 8 * l;
  if (in) {
    __builtin_nontemporal_store(c, (KTIR_G(gu4)*)((KTIR_G(uint16_t)*)L.ptr + e));
    return;
  }
  KTIR_G(uint16_t)* p = (KTIR_G(uint16_t)*)L.ptr;
#pragma unroll
  for (int k = 0; k < 8; ++k)
    if (e + k >= L.lo && e + k < L.hi) p[e + k] = (uint16_t)(c[k >> 1] >> (16 * (k & 1)));
}

// add fold in the reference's halving order of the row's values, which
// get(i, v) produces for chunk i
template <int NQ, typename G>
__device__ __forceinline__ float rf_sum(G get) {
  constexpr int H = NQ > 1 ? NQ / 2 : 1;
  float t[H][8];
#pragma unroll
  for (int i = 0; i < H; ++i) {
    float a[8];
    get(i, a);
    if (NQ > 1) {
      float b[8];
      get(i + H, b);
#pragma unroll
      for (int j = 0; j < 8; ++j) t[i][j] = __fadd_rn(a[j], b[j]);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) t[i][j] = a[j];
    }
    // one chunk pair at a time: the values of all chunks at once would
    // take more registers than the row itself
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int h = H / 2; h >= 1; h >>= 1)
#pragma unroll
    for (int i = 0; i < h; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) t[i][j] = __fadd_rn(t[i][j], t[i + h][j]);
  float a[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) a[j] = t[0][j];
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1)
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = __fadd_rn(a[j], __shfl_xor(a[j], s));
#pragma unroll
  for (int h = 4; h >= 1; h >>= 1)
#pragma unroll
    for (int j = 0; j < h; ++j) a[j] = __fadd_rn(a[j], a[j + h]);
  return a[0];
}

// Row registers in lanes 0..7 of one vector register: a read is one lane
// access and a write one lane select, with no selection over the register
// number.
struct RowLanes {
  int v, lane;
  __device__ __forceinline__ float get(int i) const { return __int_as_float(__builtin_amdgcn_readlane(v, i)); }
  __device__ __forceinline__ void set(int i, float x) {
    const int u = __builtin_amdgcn_readfirstlane(__float_as_int(x));
    v = lane == i ? u : v;
  }
};

// An empty statement that the compiler must assume rewrites the chunks: the
// row is unpacked again in each pass from its 16-bit chunks instead of being
// kept as f32 values (twice the registers) between the passes.
template <int NQ>
__device__ __forceinline__ void rf_fence(gu4 (&c)[NQ]) {
#pragma unroll
  for (int i = 0; i < NQ; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t u = c[i][k];
      asm volatile("" : "+v"(u));
      c[i][k] = u;
    }
}

template <int NQ, int DT>
__device__ __forceinline__ void rf_softmax(const RfPlan& F, gu4 (&c)[NQ], const RwPos& p, RowLanes& rr, int l) {
  // row max, NaN-propagating as arith.maximumf (exact on the 16-bit values:
  // f16 rows two at a time with v_pk_maximum3_f16)
  float mx;
  if (DT == KTIR_F16) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 a = {-__builtin_inff16(), -__builtin_inff16()}, b = a;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      // the words through scalars: this clang lowers __builtin_bit_cast of a
      // vector element (c[i][k]) as a read of element 0
      const uint32_t w0 = c[i][0], w1 = c[i][1], w2 = c[i][2], w3 = c[i][3];
      a = __builtin_elementwise_maximum(a, __builtin_bit_cast(h2, w0));
      b = __builtin_elementwise_maximum(b, __builtin_bit_cast(h2, w1));
      a = __builtin_elementwise_maximum(a, __builtin_bit_cast(h2, w2));
      b = __builtin_elementwise_maximum(b, __builtin_bit_cast(h2, w3));
    }
    a = __builtin_elementwise_maximum(a, b);
    mx = __builtin_elementwise_maximum((float)a.x, (float)a.y);
  } else {
    float a = -__builtin_inff(), b = a;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      float v[8];
      rf_unpack<DT>(c[i], v);
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        a = __builtin_elementwise_maximum(a, v[j]);
        b = __builtin_elementwise_maximum(b, v[j + 1]);
      }
    }
    mx = __builtin_elementwise_maximum(a, b);
  }
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) mx = __builtin_elementwise_maximum(mx, __shfl_xor(mx, s));
  rr.set(F.fold0, mx);
  for (int k = 0; k < F.n_row0; ++k) rw_row_exec(F, F.row0[k], rr, p.lane);
  const float m = rr.get(F.m);
  rf_fence<NQ>(c);
  // exp(x - m') (at most 1: x <= m').  An f16 row keeps the exponentials
  // rounded to f16 and packed for the store pass (half the registers of f32
  // values), and the row sum adds those f16 values two per dot2: an
  // exponential below f16's normal range (x - m' < -9.7) loses relative
  // precision, but the output e / s (s >= 1) is then below f16's normal range
  // too, so the error stays under one f16 ulp of the output (2^-11 of it in
  // the normal range).  A bf16 row keeps f32 exponentials: bf16 outputs hold
  // their relative precision far below f16's range.
  // While |m'| < 2048 the exponent is one FMA into exp2 (the rounding of
  // m' log2 e is then below 2^-12 of it); else the difference first.
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  typedef float f2 __attribute__((ext_vector_type(2)));
  constexpr bool PACK = DT == KTIR_F16;
  constexpr int NE = PACK ? NQ * 4 : NQ * 8;
  uint32_t ep[NE];                 // f16 pairs (PACK) or f32 bit patterns
  const bool near = fabsf(m) < 2048.f;
  const float c0 = -__fmul_rn(m, 1.44269504088896341f);
  const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
  float s0 = 0.f, s1 = 0.f;
  {
    // one loop for both forms: near, x - 0 (exact) into the FMA with c0;
    // far, x - m' first and no addend (the same roundings as either form alone)
    const float msub = near ? 0.f : m, c0u = near ? c0 : 0.f;
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      float v[8];
      rf_unpack<DT>(c[i], v);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const f2 x = {__builtin_amdgcn_exp2f(__builtin_fmaf(__fsub_rn(v[2 * k], msub), 1.44269504088896341f, c0u)),
                      __builtin_amdgcn_exp2f(__builtin_fmaf(__fsub_rn(v[2 * k + 1], msub), 1.44269504088896341f, c0u))};
        if constexpr (PACK) {
          ep[4 * i + k] = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, h2));
        } else {
          ep[8 * i + 2 * k] = __float_as_uint(x.x);
          ep[8 * i + 2 * k + 1] = __float_as_uint(x.y);
        }
      }
    }
  }
  if constexpr (PACK) {
#pragma unroll
    for (int q = 0; q < NE; q += 2) {
      s0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, ep[q]), one, s0, false);
      s1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, ep[q + 1]), one, s1, false);
    }
  } else {
#pragma unroll
    for (int q = 0; q < NE; q += 2) {
      s0 = __fadd_rn(s0, __uint_as_float(ep[q]));
      s1 = __fadd_rn(s1, __uint_as_float(ep[q + 1]));
    }
  }
  float sum = __fadd_rn(s0, s1);
  // v_dot2_f32_f16 does not carry a NaN operand into its sum as an f32 add
  // would.  An exponential is NaN only if the row max is NaN or m' is not
  // finite (x - m' is NaN only for x NaN or x = m' = +-inf), so only then are
  // the f16 values checked; a NaN among them makes the lane's part NaN, and
  // the adds below carry it into the row sum.
  if constexpr (PACK) {
    if (mx != mx || !(fabsf(m) <= 3.40282347e38f)) {
      bool nan_e = false;
#pragma unroll
      for (int q = 0; q < NE; ++q) {
        const h2 w = __builtin_bit_cast(h2, ep[q]);
        nan_e = nan_e || w.x != w.x || w.y != w.y;
      }
      if (nan_e) sum = __builtin_nanf("");
    }
  }
#pragma unroll
  for (int sh = 32; sh >= 1; sh >>= 1) sum = __fadd_rn(sum, __shfl_xor(sum, sh));
  rr.set(F.fold1, sum);
  for (int k = 0; k < F.n_row1; ++k) rw_row_exec(F, F.row1[k], rr, p.lane);
  const float s = rr.get(F.s);
  // e / s as e times the correctly rounded 1 / s (within 1.5 f32 ulps of the
  // quotient, before the 16-bit rounding of the store); the plain quotient
  // for a sum that is tiny, huge or not finite
  const float r = __fdiv_rn(1.f, s);
  const float as = fabsf(s);
  const bool fast = as > 1e-30f && as < 1e30f && r == r;
  const int64_t e0 = rw_row_base(F.y, p);
  const bool in = e0 >= F.y.lo && e0 + 512 * NQ <= F.y.hi;
  // the two divisions on separate (uniform) branches
  auto out = [&](auto div) {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      float y[8];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        f2 e;
        if constexpr (PACK) {
          e = __builtin_convertvector(__builtin_bit_cast(h2, ep[4 * i + k]), f2);
        } else {
          e = f2{__uint_as_float(ep[8 * i + 2 * k]), __uint_as_float(ep[8 * i + 2 * k + 1])};
        }
        y[2 * k] = div(e.x);
        y[2 * k + 1] = div(e.y);
      }
      rf_store(F.y, e0, in, i, l, rf_pack2<DT>(y));
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  if (fast) {
    out([&](float e) { return __fmul_rn(e, r); });
  } else {
    // rare (huge or non-finite operands): one quotient at a time, so that
    // this branch does not set the kernel's register count
    out([&](float e) {
      const float q = __fdiv_rn(e, s);
      __builtin_amdgcn_sched_barrier(0);
      return q;
    });
  }
}

// w: the weight row in LDS (lane l's own 16-byte pieces, at 1024 i + 16 l)
template <int NQ, int DT>
__device__ __forceinline__ void rf_norm(const RfPlan& F, gu4 (&c)[NQ], const gu4* w, const RwPos& p, RowLanes& rr,
                                        int l) {
  rr.set(F.fold0, rf_sum<NQ>([&](int i, float (&v)[8]) {
    rf_unpack<DT>(c[i], v);
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __fmul_rn(v[j], v[j]);
  }));
  for (int k = 0; k < F.n_row0; ++k) rw_row_exec(F, F.row0[k], rr, p.lane);
  const float s = rr.get(F.s);
  const int64_t e0 = rw_row_base(F.y, p);
  const bool in = e0 >= F.y.lo && e0 + 512 * NQ <= F.y.hi;
  rf_fence<NQ>(c);
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    float y[8];
    rf_unpack<DT>(c[i], y);
    if (F.has_w) {
      float wv[8];
      rf_unpack<DT>(w[64 * i + l], wv);
      if (F.w_first) {
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = __fmul_rn(__fmul_rn(y[j], wv[j]), s);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) y[j] = __fmul_rn(__fmul_rn(y[j], s), wv[j]);
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) y[j] = __fmul_rn(y[j], s);
    }
    rf_store(F.y, e0, in, i, l, rf_pack<DT>(y));
    __builtin_amdgcn_sched_barrier(0);
  }
}

typedef _Float16 rf_h2 __attribute__((ext_vector_type(2)));
typedef float rf_f2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ rf_h2 rf_word(uint32_t u) { return __builtin_bit_cast(rf_h2, u); }
__device__ __forceinline__ uint32_t rf_bits(rf_h2 h) { return __builtin_bit_cast(uint32_t, h); }

// f16 add fold in the reference's halving order of the row's values, which
// get(i, k) produces as word k (elements 2k, 2k + 1) of chunk i; every add
// rounded to f16 (packed adds on the pairs)
template <int NQ, typename G>
__device__ __forceinline__ float rf_sum16(G get) {
  constexpr int H = NQ > 1 ? NQ / 2 : 1;
  rf_h2 t[H][4];
#pragma unroll
  for (int i = 0; i < H; ++i)
#pragma unroll
    for (int k = 0; k < 4; ++k) t[i][k] = NQ > 1 ? get(i, k) + get(i + H, k) : get(i, k);
#pragma unroll
  for (int h = H / 2; h >= 1; h >>= 1)
#pragma unroll
    for (int i = 0; i < h; ++i)
#pragma unroll
      for (int k = 0; k < 4; ++k) t[i][k] = t[i][k] + t[i + h][k];
  rf_h2 a[4] = {t[0][0], t[0][1], t[0][2], t[0][3]};
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1)
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] = a[k] + rf_word((uint32_t)__shfl_xor((int)rf_bits(a[k]), s));
  // the bits of j: j with j + 4 (word k with word k + 2), j + 2 (word 0 with 1), j + 1
  a[0] = a[0] + a[2];
  a[1] = a[1] + a[3];
  a[0] = a[0] + a[1];
  return (float)(_Float16)(a[0].x + a[0].y);
}

template <int NQ>
__device__ __forceinline__ void rf_softmax16(const RfPlan& F, gu4 (&c)[NQ], const RwPos& p, RowLanes& rr, int l) {
  // row max of the f16 values: the order does not change a max
  rf_h2 a = {-__builtin_inff16(), -__builtin_inff16()}, b = a;
  float mx;
  if (__builtin_amdgcn_readfirstlane(F.numf)) {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const uint32_t w0 = c[i][0], w1 = c[i][1], w2 = c[i][2], w3 = c[i][3];
      a = __builtin_elementwise_max(a, rf_word(w0));
      b = __builtin_elementwise_max(b, rf_word(w1));
      a = __builtin_elementwise_max(a, rf_word(w2));
      b = __builtin_elementwise_max(b, rf_word(w3));
    }
    a = __builtin_elementwise_max(a, b);
    mx = fmaxf((float)a.x, (float)a.y);
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) mx = fmaxf(mx, __shfl_xor(mx, s));
  } else {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const uint32_t w0 = c[i][0], w1 = c[i][1], w2 = c[i][2], w3 = c[i][3];
      a = __builtin_elementwise_maximum(a, rf_word(w0));
      b = __builtin_elementwise_maximum(b, rf_word(w1));
      a = __builtin_elementwise_maximum(a, rf_word(w2));
      b = __builtin_elementwise_maximum(b, rf_word(w3));
    }
    a = __builtin_elementwise_maximum(a, b);
    mx = __builtin_elementwise_maximum((float)a.x, (float)a.y);
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) mx = __builtin_elementwise_maximum(mx, __shfl_xor(mx, s));
  }
  rr.set(F.fold0, mx);
  for (int k = 0; k < F.n_row0; ++k) rw_row_exec(F, F.row0[k], rr, p.lane);
  const float m = rr.get(F.m);
  // e = f16(exp(f16(x - m'))), kept packed for the store pass.  With m' an
  // f16 value, f16(x - m') is one packed f16 subtraction (NumPy's f16
  // subtraction rounds the f32 difference of two f16 values, the correctly
  // rounded f16 difference); else the f32 difference, rounded.
  uint32_t ep[NQ * 4];
  const _Float16 mh = (_Float16)m;
  const bool m16 = (float)mh == m || m != m;
  const rf_h2 m2 = {mh, mh};
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      rf_f2 dr;
      if (m16) {
        dr = __builtin_convertvector(rf_word(c[i][k]) - m2, rf_f2);
      } else {
        const rf_f2 x = __builtin_convertvector(rf_word(c[i][k]), rf_f2);
        const rf_f2 d = {__fsub_rn(x.x, m), __fsub_rn(x.y, m)};
        dr = __builtin_convertvector(__builtin_convertvector(d, rf_h2), rf_f2);
      }
      const rf_f2 e = {exp_hw(dr.x), exp_hw(dr.y)};
      ep[4 * i + k] = rf_bits(__builtin_convertvector(e, rf_h2));
    }
  }
  const float sum = rf_sum16<NQ>([&](int i, int k) { return rf_word(ep[4 * i + k]); });
  rr.set(F.fold1, sum);
  for (int k = 0; k < F.n_row1; ++k) rw_row_exec(F, F.row1[k], rr, p.lane);
  const float s = rr.get(F.s);
  const int64_t e0 = rw_row_base(F.y, p);
  const bool in = e0 >= F.y.lo && e0 + 512 * NQ <= F.y.hi;
  // f16(e / s'): the quotient within one f32 ulp (div_by: the correctly
  // rounded 1 / s' and one fused correction) before the f16 rounding, which it
  // changes only next to an f16 rounding midpoint; the plain quotient for a
  // sum that is tiny, huge or not finite
  const float r = __fdiv_rn(1.f, s);
  const float as = fabsf(s);
  const bool fast = as > 1e-30f && as < 1e30f && r == r;
  auto out = [&](auto div) {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      gu4 y;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const rf_f2 e = __builtin_convertvector(rf_word(ep[4 * i + k]), rf_f2);
        const rf_f2 q = {div(e.x), div(e.y)};
        y[k] = rf_bits(__builtin_convertvector(q, rf_h2));
      }
      rf_store(F.y, e0, in, i, l, y);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  if (fast) {
    out([&](float e) { return div_by(e, s, r); });
  } else {
    out([&](float e) {
      const float q = __fdiv_rn(e, s);
      __builtin_amdgcn_sched_barrier(0);
      return q;
    });
  }
}

// w: the weight row in LDS (lane l's own 16-byte pieces, at 1024 i + 16 l)
template <int NQ>
__device__ __forceinline__ void rf_norm16(const RfPlan& F, gu4 (&c)[NQ], const gu4* w, const RwPos& p, RowLanes& rr,
                                          int l) {
  rr.set(F.fold0, rf_sum16<NQ>([&](int i, int k) {
    const rf_h2 x = rf_word(c[i][k]);
    return x * x;
  }));
  for (int k = 0; k < F.n_row0; ++k) rw_row_exec(F, F.row0[k], rr, p.lane);
  const float s = rr.get(F.s);
  const int64_t e0 = rw_row_base(F.y, p);
  const bool in = e0 >= F.y.lo && e0 + 512 * NQ <= F.y.hi;
  // f16(x * s) as one packed f16 product when s is an f16 value (the f32
  // product of two f16 values rounded once); else in f32, then rounded
  const _Float16 sh = (_Float16)s;
  const bool s16 = (float)sh == s || s != s;
  const rf_h2 s2 = {sh, sh};
  auto scale = [&](rf_h2 x) -> rf_h2 {
    if (s16) return x * s2;
    const rf_f2 xf = __builtin_convertvector(x, rf_f2);
    return __builtin_convertvector(rf_f2{__fmul_rn(xf.x, s), __fmul_rn(xf.y, s)}, rf_h2);
  };
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    gu4 y;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      rf_h2 x = rf_word(c[i][k]);
      if (F.has_w) {
        const rf_h2 wk = rf_word(w[64 * i + l][k]);
        x = F.w_first ? scale(x * wk) : scale(x) * wk;
      } else {
        x = scale(x);
      }
      y[k] = rf_bits(x);
    }
    rf_store(F.y, e0, in, i, l, y);
  }
}

template <int NQ, int RECIPE, int DT>
__device__ __forceinline__ void rf_row(const RfPlan& F, gu4 (&c)[NQ], const gu4* w, const RwPos& p, RowLanes& rr,
                                       int l) {
  if (RECIPE == RF_SOFTMAX) rf_softmax<NQ, DT>(F, c, p, rr, l);
  else if (RECIPE == RF_NORM) rf_norm<NQ, DT>(F, c, w, p, rr, l);
  else if (RECIPE == RF_SOFTMAX16) rf_softmax16<NQ>(F, c, p, rr, l);
  else rf_norm16<NQ>(F, c, w, p, rr, l);
}

// Rows r = blockIdx.x + k gridDim.x, two row buffers in turn (no copy between
// them, so the next row's loads stay in flight across the current row).
template <int NQ, int RECIPE, int DT>
__global__ __launch_bounds__(64) void prog_rowfix(const RfPlan F, int64_t total_rows) {
  __shared__ gu4 w[RECIPE == RF_NORM || RECIPE == RF_NORM16 ? 64 * NQ : 1];
  const int l = threadIdx.x;
  int64_t rows_per_lane = 1;
#pragma unroll
  for (int d = 0; d < KTIR_MAX_DIMS - 1; ++d)
    if (d < F.nd - 1) rows_per_lane *= F.shape[d];
  const int32_t rpl = (int32_t)rows_per_lane;
  RowLanes rr{0, l};
  int64_t r = blockIdx.x;
  if (r >= total_rows) return;
  gu4 ca[NQ], cb[NQ];
  RwPos pa = rw_pos(F, r, rpl);
  if ((RECIPE == RF_NORM || RECIPE == RF_NORM16) && F.has_w) {
    // the same row for every row; each lane reads back only what it wrote
    rf_load<NQ>(F.w, rw_row_base(F.w, pa), l, ca);
#pragma unroll
    for (int i = 0; i < NQ; ++i) w[64 * i + l] = ca[i];
  }
  rf_load<NQ>(F.x, rw_row_base(F.x, pa), l, ca);
  for (;;) {
    const int64_t rb = r + gridDim.x;
    const RwPos pb = rw_pos(F, rb < total_rows ? rb : r, rpl);
    if (rb < total_rows) rf_load<NQ>(F.x, rw_row_base(F.x, pb), l, cb);
    rf_row<NQ, RECIPE, DT>(F, ca, w, pa, rr, l);
    if (rb >= total_rows) break;
    r = rb + gridDim.x;
    pa = rw_pos(F, r < total_rows ? r : rb, rpl);
    if (r < total_rows) rf_load<NQ>(F.x, rw_row_base(F.x, pa), l, ca);
    rf_row<NQ, RECIPE, DT>(F, cb, w, pb, rr, l);
    if (r >= total_rows) break;
  }
}

template <int NQ, int RECIPE, int DT>
static void launch_rowfix(const RfPlan& F, int64_t rows) {
  static int resident = 0;
  if (!resident) {
    int per_cu = 0, cus = 0, dev = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, prog_rowfix<NQ, RECIPE, DT>, 64, 0) != hipSuccess ||
        hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu < 1 || cus < 1) {
      per_cu = 1;
      cus = 256;
    }
    resident = per_cu * cus;
  }
  const int64_t per_block = (rows + resident - 1) / resident;
  const int64_t blocks = row_grid_limit((rows + per_block - 1) / per_block);
  hipLaunchKernelGGL((prog_rowfix<NQ, RECIPE, DT>), dim3((unsigned)blocks), dim3(64), 0, stream(), F, rows);
}

template <int NQ>
static void rowfix_dt(const RfPlan& F, int recipe, int dt, int64_t rows) {
  if (recipe == RF_SOFTMAX16) {
    launch_rowfix<NQ, RF_SOFTMAX16, KTIR_F16>(F, rows);
  } else if (recipe == RF_NORM16) {
    launch_rowfix<NQ, RF_NORM16, KTIR_F16>(F, rows);
  } else if (recipe == RF_SOFTMAX) {
    if (dt == KTIR_F16) launch_rowfix<NQ, RF_SOFTMAX, KTIR_F16>(F, rows);
    else launch_rowfix<NQ, RF_SOFTMAX, KTIR_BF16>(F, rows);
  } else {
    if (dt == KTIR_F16) launch_rowfix<NQ, RF_NORM, KTIR_F16>(F, rows);
    else launch_rowfix<NQ, RF_NORM, KTIR_BF16>(F, rows);
  }
}

static bool rf_leaf_ok(const ktir_leaf_t& L, int nd, int dt) {
  return rows_leaf_ok(L, nd) && L.dtype == dt && (L.flags & KTIR_LEAF_VEC8);
}

static bool rf_invariant(const ktir_prog_t& P, const ktir_leaf_t& L) {
  bool inv = L.lane_base == 0 && L.lane_stride == 0;
  for (int d = 0; d < P.ndim - 1; ++d) inv = inv && (L.strides[d] == 0 || P.shape[d] == 1);
  return inv;
}

static bool rf_op(const RcOp& o, int op, int kind) {
  return o.op == op && o.dt == KTIR_F32 && o.kind == kind && (op != KTIR_OP_DIVF || o.aux == 0);
}

// Match the pass plan against the two fixed forms and launch; false leaves
// the program to the general row kernels.
static bool try_launch_rowfix(const ktir_prog_t& P, const RcPlan& R, int64_t rows, int64_t inner) {
  if (inner != 512 && inner != 1024 && inner != 2048 && inner != 4096) return false;
  if (rows > INT32_MAX) return false;
  for (int d = 0; d < P.ndim; ++d)
    if (P.shape[d] > INT32_MAX) return false;
  int pass[3], n_pass = 0, gap[3] = {0, 0, 0};
  for (int i = 0; i < R.n_steps; ++i) {
    const RcStep& S = R.steps[i];
    if (S.kind == 1) {
      if (n_pass == 3) return false;
      pass[n_pass++] = i;
    } else if (S.kind == 0) {
      if (n_pass == 0 || gap[n_pass - 1] == RF_MAX_ROW) return false;
      ++gap[n_pass - 1];
    } else {
      return false;
    }
  }
  RfPlan F{};
  F.nd = P.ndim;
  for (int d = 0; d < KTIR_MAX_DIMS; ++d) F.shape[d] = d < P.ndim ? P.shape[d] : 1;
  F.lane_scalars = P.lane_scalars;
  F.n_lane_scalars = P.n_lane_scalars;
  auto rows_of = [&](int g, ktir_instr_t* dst) {
    int k = 0;
    for (int i = pass[g] + 1; i < R.n_steps && R.steps[i].kind == 0; ++i) dst[k++] = P.instr[R.steps[i].pc];
    return k;
  };
  const RcStep& A = R.steps[pass[0]];
  // f16 folds: the f16-math forms (f16 rows only)
  const bool m16 = A.fold_dt == KTIR_F16;
  if (A.end != 0 || (A.fold_dt != KTIR_F32 && !m16)) return false;
  const int sx = A.src;
  const ktir_leaf_t& X = P.leaves[R.slot_leaf[sx]];
  const int dt = X.dtype;
  if ((dt != KTIR_F16 && dt != KTIR_BF16) || (m16 && dt != KTIR_F16) || !rf_leaf_ok(X, P.ndim, dt)) return false;
  F.x = rw_leaf(P, R.slot_leaf[sx]);
  const RcStep& Z = R.steps[pass[n_pass - 1]];   // the storing pass
  if (Z.end != 1 || Z.src != sx || !rf_leaf_ok(P.leaves[Z.st_leaf], P.ndim, dt) || gap[n_pass - 1] != 0) return false;
  F.y = rw_leaf(P, Z.st_leaf);
  // an optional last rounding to the stored dtype (the store rounds the same way)
  auto tail = [&](const RcStep& S, int n) {
    return S.n_ops == n || (S.n_ops == n + 1 && S.ops[n].op == KTIR_OP_CAST && S.ops[n].kind == 0 &&
                            S.ops[n].aux == KTIR_F32 && S.ops[n].dt == dt);
  };
  // an f16 op as analyze_rows keeps it: its f32 op, then the rounding to f16;
  // the storing pass's last rounding may be left to the (f16) store
  auto nop = [&](const RcStep& S, int i, int op, int kind) {
    return i + 1 < S.n_ops && S.ops[i].op == op && S.ops[i].dt == KTIR_F32 && S.ops[i].kind == kind &&
           S.ops[i + 1].op == KTIR_OP_CAST && S.ops[i + 1].kind == 0 && S.ops[i + 1].aux == KTIR_F32 &&
           S.ops[i + 1].dt == KTIR_F16;
  };
  auto nlast = [&](const RcStep& S, int i, int op, int kind) {
    return (S.n_ops == i + 2 && nop(S, i, op, kind)) ||
           (S.n_ops == i + 1 && S.ops[i].op == op && S.ops[i].dt == KTIR_F32 && S.ops[i].kind == kind);
  };
  int recipe;
  if (n_pass == 3 && m16) {
    const RcStep& B = R.steps[pass[1]];
    if (R.n_slots != 1 || A.n_ops != 0 || (A.fold_op != KTIR_OP_MAXNUMF && A.fold_op != KTIR_OP_MAXIMUMF)) return false;
    if (B.src != sx || B.end != 0 || B.n_ops != 4 || B.fold_op != KTIR_OP_ADDF || B.fold_dt != KTIR_F16) return false;
    if (!nop(B, 0, KTIR_OP_SUBF, 1) || B.ops[0].swap || !nop(B, 2, KTIR_OP_EXP, 0)) return false;
    if (!nop(Z, 0, KTIR_OP_SUBF, 1) || Z.ops[0].swap || Z.ops[0].idx != B.ops[0].idx || !nop(Z, 2, KTIR_OP_EXP, 0) ||
        !nlast(Z, 4, KTIR_OP_DIVF, 1) || Z.ops[4].swap)
      return false;
    // e is computed once: m' must hold the same value in both passes
    const int m = B.ops[0].idx;
    if (B.dst == m) return false;
    F.n_row1 = rows_of(1, F.row1);
    for (int k = 0; k < F.n_row1; ++k)
      if (F.row1[k].dst == m) return false;
    F.fold1 = B.dst;
    F.m = (int8_t)m;
    F.s = Z.ops[4].idx;
    F.numf = A.fold_op == KTIR_OP_MAXNUMF;
    recipe = RF_SOFTMAX16;
  } else if (n_pass == 2 && m16) {
    if (A.n_ops != 2 || !nop(A, 0, KTIR_OP_MULF, 3) || A.fold_op != KTIR_OP_ADDF) return false;
    const RcOp* o = Z.ops;
    if (nlast(Z, 0, KTIR_OP_MULF, 1)) {
      F.s = o[0].idx;
    } else if (nop(Z, 0, KTIR_OP_MULF, 1) && nlast(Z, 2, KTIR_OP_MULF, 2) && o[2].idx != sx) {
      F.s = o[0].idx;
      F.has_w = 1;
    } else if (nop(Z, 0, KTIR_OP_MULF, 2) && nlast(Z, 2, KTIR_OP_MULF, 1) && o[0].idx != sx) {
      F.s = o[2].idx;
      F.has_w = 1;
      F.w_first = 1;
    } else {
      return false;
    }
    if (R.n_slots != 1 + F.has_w) return false;
    if (F.has_w) {
      const ktir_leaf_t& W = P.leaves[R.slot_leaf[1 - sx]];
      if (!rf_leaf_ok(W, P.ndim, dt) || !rf_invariant(P, W)) return false;
      F.w = rw_leaf(P, R.slot_leaf[1 - sx]);
    }
    recipe = RF_NORM16;
  } else if (m16) {
    return false;
  } else if (n_pass == 3) {
    const RcStep& B = R.steps[pass[1]];
    if (R.n_slots != 1 || A.n_ops != 0 || A.fold_op != KTIR_OP_MAXIMUMF) return false;
    if (B.src != sx || B.end != 0 || B.n_ops != 2 || B.fold_op != KTIR_OP_ADDF || B.fold_dt != KTIR_F32) return false;
    if (!rf_op(B.ops[0], KTIR_OP_SUBF, 1) || B.ops[0].swap || !rf_op(B.ops[1], KTIR_OP_EXP, 0)) return false;
    if (!tail(Z, 3) || !rf_op(Z.ops[0], KTIR_OP_SUBF, 1) || Z.ops[0].swap || Z.ops[0].idx != B.ops[0].idx ||
        !rf_op(Z.ops[1], KTIR_OP_EXP, 0) || !rf_op(Z.ops[2], KTIR_OP_DIVF, 1) || Z.ops[2].swap)
      return false;
    // exp(x - m') is computed once: m' must hold the same value in both passes
    const int m = B.ops[0].idx;
    if (B.dst == m) return false;
    F.n_row1 = rows_of(1, F.row1);
    for (int k = 0; k < F.n_row1; ++k)
      if (F.row1[k].dst == m) return false;
    F.fold1 = B.dst;
    F.m = (int8_t)m;
    F.s = Z.ops[2].idx;
    recipe = RF_SOFTMAX;
  } else if (n_pass == 2) {
    if (A.n_ops != 1 || !rf_op(A.ops[0], KTIR_OP_MULF, 3) || A.fold_op != KTIR_OP_ADDF) return false;
    const RcOp* o = Z.ops;
    if (tail(Z, 1) && rf_op(o[0], KTIR_OP_MULF, 1)) {
      F.s = o[0].idx;
    } else if (tail(Z, 2) && rf_op(o[0], KTIR_OP_MULF, 1) && rf_op(o[1], KTIR_OP_MULF, 2) && o[1].idx != sx) {
      F.s = o[0].idx;
      F.has_w = 1;
    } else if (tail(Z, 2) && rf_op(o[0], KTIR_OP_MULF, 2) && rf_op(o[1], KTIR_OP_MULF, 1) && o[0].idx != sx) {
      F.s = o[1].idx;
      F.has_w = 1;
      F.w_first = 1;
    } else {
      return false;
    }
    if (R.n_slots != 1 + F.has_w) return false;
    if (F.has_w) {
      const ktir_leaf_t& W = P.leaves[R.slot_leaf[1 - sx]];
      if (!rf_leaf_ok(W, P.ndim, dt) || !rf_invariant(P, W)) return false;
      F.w = rw_leaf(P, R.slot_leaf[1 - sx]);
    }
    recipe = RF_NORM;
  } else {
    return false;
  }
  F.fold0 = A.dst;
  F.n_row0 = rows_of(0, F.row0);
  switch (inner / 512) {
    case 1: rowfix_dt<1>(F, recipe, dt, rows); break;
    case 2: rowfix_dt<2>(F, recipe, dt, rows); break;
    case 4: rowfix_dt<4>(F, recipe, dt, rows); break;
    default: rowfix_dt<8>(F, recipe, dt, rows); break;
  }
  return true;
}

// Launch `P` (mode 1) through the row-chain kernel if it has the supported form.
bool try_launch_rows(const ktir_prog_t& P, int64_t rows, int64_t inner) {
  if (P.mode != 1 || inner < 64 || inner > 8192 || (inner & (inner - 1))) return false;
  if (P.lanes > 0 && P.lane_scalars == 0) {
    for (int i = 0; i < P.n_instr; ++i)
      if (P.instr[i].op == KTIR_OP_LANE) return false;
  }
  RcPlan R;
  if (!analyze_rows(P, R)) return false;
  const bool plain = plan_plain(R);
  // the fixed forms: the f32-math ones take plain plans, the f16-math ones
  // f16 folds (try_launch_rowfix checks which)
  if (try_launch_rowfix(P, R, rows, inner)) return true;
  if (try_launch_rowwave(P, R, rows, inner, !plain)) return true;
  // threads per row and elements per thread: n = tpr * E, E in {2..32}, tpr in {32..256}
  int tpr = (int)(inner / 16);
  if (tpr > 256) tpr = 256;
  if (tpr < 32) tpr = 32;
  const int E = (int)(inner / tpr);
  if (E < 2 || E > 32) return false;
  int tpr_log2 = 0;
  while ((1 << tpr_log2) < tpr) ++tpr_log2;
  const int rpw = 256 / tpr;
  int64_t blocks = (rows + rpw - 1) / rpw;
  if (blocks > 65536) blocks = 65536;
  blocks = row_grid_limit(blocks);
  switch (E) {
    case 2: hipLaunchKernelGGL(prog_rowchain<2>, dim3((unsigned)blocks), dim3(256), 0, stream(), P, R, tpr_log2, rows); break;
    case 4: hipLaunchKernelGGL(prog_rowchain<4>, dim3((unsigned)blocks), dim3(256), 0, stream(), P, R, tpr_log2, rows); break;
    case 8: hipLaunchKernelGGL(prog_rowchain<8>, dim3((unsigned)blocks), dim3(256), 0, stream(), P, R, tpr_log2, rows); break;
    case 16: hipLaunchKernelGGL(prog_rowchain<16>, dim3((unsigned)blocks), dim3(256), 0, stream(), P, R, tpr_log2, rows); break;
    case 32: hipLaunchKernelGGL(prog_rowchain<32>, dim3((unsigned)blocks), dim3(256), 0, stream(), P, R, tpr_log2, rows); break;
    default: return false;
  }
  return true;
}

}  // namespace ktir

extern "C" int ktir_set_row_grid_limit(int64_t max_workgroups) {
  if (max_workgroups < 0) return ktir::set_error(KTIR_E_ARG, "ktir_set_row_grid_limit: negative limit");
  ktir::g_row_grid_limit = max_workgroups;
  return KTIR_OK;
}
