/*
 * ktir_hip.h — C ABI of the MI355X (gfx950) execution backend for KTIR.
 *
 * This is the drop-in boundary under the Python `KTIRInterpreter`
 * (reference `ktir_cpu/interpreter.py:40-395`).  The reference executes each
 * simulated Spyre core one after another and every tile op as NumPy calls on
 * a simulated HBM (`ktir_cpu/memory.py:311-398`).  Here the simulated HBM is one
 * device arena, tile values are device buffers, and tile ops run as the gfx950
 * kernels below.  Only plain integers, doubles and device addresses cross this
 * boundary; every entry point returns 0 on success or a negative KTIR_E_* code,
 * with a message available from ktir_last_error().
 *
 * Terminology (from the reference): a *lane* is one instance of the KTIR
 * function body executing in lockstep with others: one simulated grid core
 * (`ktir_cpu/grid.py:434-469`), or one (core, loop-iteration) pair when the
 * host runs independent `scf.for` iterations side by side.  A *leaf* is one
 * strided or offset-list view of device memory read or written by a kernel.
 */
#ifndef KTIR_HIP_H
#define KTIR_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (mapped to Python exceptions by the host runtime) ---- */
#define KTIR_OK 0
#define KTIR_E_HIP -1        /* HIP runtime error                  -> RuntimeError */
#define KTIR_E_ARG -2        /* invalid descriptor / argument       -> ValueError   */
#define KTIR_E_INDEX -3      /* negative indirect index (reference ops/memory_ops.py:378-382) -> IndexError */
#define KTIR_E_UNSUPPORTED -4 /* shape / dtype not handled          -> NotImplementedError */

/* ---- element types (reference dtypes.py:24-39; bf16 is an extension) ---- */
#define KTIR_F16 0
#define KTIR_BF16 1
#define KTIR_F32 2
#define KTIR_I1 3   /* stored as one byte, like numpy bool */
#define KTIR_I32 4  /* also `index` (reference maps index to int32) */
#define KTIR_I64 5
#define KTIR_I8 6
#define KTIR_I16 7

/* ---- fused-program opcodes ----
 * A program is a straight-line list of instructions over 8 virtual registers
 * of 32-bit values (f32 for f16/bf16/f32 data, int32 for integer data).
 * Each float op rounds its result to the instruction's dtype, which reproduces
 * NumPy's f16 arithmetic (compute in f32, round to nearest even). */
#define KTIR_OP_NOP 0
#define KTIR_OP_LD 1          /* dst <- leaf[aux] at the current element */
#define KTIR_OP_ST 2          /* leaf[aux] <- a (converted to the leaf dtype) */
#define KTIR_OP_CONST 3       /* dst <- imm (as dt) */
#define KTIR_OP_LANE 4        /* dst <- lane_scalars[lane * n_lane_scalars + aux] (as dt) */
#define KTIR_OP_IDX 5         /* dst <- iteration index along dim aux (int) */
#define KTIR_OP_RED 6         /* row mode: deposit a into the row reduction buffer */
#define KTIR_OP_FOLD 7        /* row mode: dst <- pairwise-halving fold of the buffer with binop aux */
#define KTIR_OP_ELEM 8        /* row mode: begin element loop; i = pc of matching KTIR_OP_ENDELEM */
#define KTIR_OP_ENDELEM 9
#define KTIR_OP_CAST 10       /* dst(dt) <- a(aux = source dtype) : ext/trunc/sitofp/fptosi/... */
#define KTIR_OP_BITCAST 11    /* dst <- a reinterpreted (32-bit) */
#define KTIR_OP_SELECT 12     /* dst <- a ? b : c */
#define KTIR_OP_FMA 13        /* dst <- a * b + c (f32 then round to dt) */
#define KTIR_OP_CMPF 14       /* dst(i1) <- pred aux (a, b) over floats */
#define KTIR_OP_CMPI 15       /* dst(i1) <- pred aux (a, b) over ints */
/* unary float 20..39 */
#define KTIR_OP_NEGF 20
#define KTIR_OP_ABSF 21
#define KTIR_OP_EXP 22
#define KTIR_OP_LOG 23
#define KTIR_OP_LOG2 24
#define KTIR_OP_LOG1P 25
#define KTIR_OP_SQRT 26
#define KTIR_OP_RSQRT 27
#define KTIR_OP_TANH 28
#define KTIR_OP_SIN 29
#define KTIR_OP_COS 30
#define KTIR_OP_ERF 31
#define KTIR_OP_CEIL 32
#define KTIR_OP_FLOOR 33
#define KTIR_OP_NOTI 34       /* i1 logical not */
#define KTIR_OP_ABSI 35
/* binary float 40..59 */
#define KTIR_OP_ADDF 40
#define KTIR_OP_SUBF 41
#define KTIR_OP_MULF 42
#define KTIR_OP_DIVF 43
#define KTIR_OP_REMF 44       /* Python/NumPy modulo: sign of the divisor */
#define KTIR_OP_MAXIMUMF 45   /* NaN-propagating max (np.maximum) */
#define KTIR_OP_MINIMUMF 46
#define KTIR_OP_MAXNUMF 47    /* NaN-ignoring max (np.fmax) */
#define KTIR_OP_MINNUMF 48
#define KTIR_OP_POWF 49
/* binary int 60..89 */
#define KTIR_OP_ADDI 60
#define KTIR_OP_SUBI 61
#define KTIR_OP_MULI 62
#define KTIR_OP_DIVSI 63      /* truncating */
#define KTIR_OP_REMSI 64      /* truncating remainder */
#define KTIR_OP_FLOORDIVSI 65
#define KTIR_OP_FLOORREMSI 66 /* Python modulo */
#define KTIR_OP_CEILDIVSI 67
#define KTIR_OP_ANDI 68
#define KTIR_OP_ORI 69
#define KTIR_OP_XORI 70
#define KTIR_OP_SHLI 71
#define KTIR_OP_SHRSI 72
#define KTIR_OP_SHRUI 73
#define KTIR_OP_MAXSI 74
#define KTIR_OP_MINSI 75

/* comparison predicates (arith.cmpf / arith.cmpi) */
#define KTIR_CMP_FALSE 0
#define KTIR_CMP_OEQ 1
#define KTIR_CMP_OGT 2
#define KTIR_CMP_OGE 3
#define KTIR_CMP_OLT 4
#define KTIR_CMP_OLE 5
#define KTIR_CMP_ONE 6
#define KTIR_CMP_ORD 7
#define KTIR_CMP_UEQ 8
#define KTIR_CMP_UGT 9
#define KTIR_CMP_UGE 10
#define KTIR_CMP_ULT 11
#define KTIR_CMP_ULE 12
#define KTIR_CMP_UNE 13
#define KTIR_CMP_UNO 14
#define KTIR_CMP_TRUE 15
#define KTIR_CMP_EQ 16
#define KTIR_CMP_NE 17
#define KTIR_CMP_SLT 18
#define KTIR_CMP_SLE 19
#define KTIR_CMP_SGT 20
#define KTIR_CMP_SGE 21
#define KTIR_CMP_ULTI 22
#define KTIR_CMP_ULEI 23
#define KTIR_CMP_UGTI 24
#define KTIR_CMP_UGEI 25

#define KTIR_MAX_DIMS 4
#define KTIR_MAX_LEAVES 10
#define KTIR_MAX_INSTR 112
#define KTIR_NREG 8
#define KTIR_MAX_ROW 16384   /* longest row a row-mode program can fold in LDS */

/* leaf flags */
#define KTIR_LEAF_VEC 1      /* inner stride 1, every 4-element vector start aligned: wide accesses */
#define KTIR_LEAF_VEC8 2     /* same for 8-element vectors */
#define KTIR_LEAF_CHECKED 4  /* matmul operand: the host verified that every lane's reads stay inside
                                [lo, hi) and that every lane offset is a multiple of 8 elements */

/* One strided (or offset-list) view of device memory.
 * Element address for lane l at iteration index (i0..i3):
 *   ptr + bpe * (lane_off(l) + sum_d i_d * strides[d])               (strided)
 *   ptr + bpe * (lane_off(l) + offsets[l * offsets_lane_stride + flat]) (offset list)
 * with lane_off(l) = lane_base ? lane_base[l] : base + l * lane_stride.
 * Element offsets outside [lo, hi) read as zero and are not written: the
 * reference's zero-pad-on-over-read and truncate-on-over-write for an
 * allocation (memory.py:243-259, :281-305). */
typedef struct ktir_leaf {
  uint64_t ptr;
  int64_t base;
  int64_t lane_stride;
  uint64_t lane_base;            /* const int64_t* [lanes] or 0 */
  uint64_t offsets;              /* const int64_t* or 0 */
  int64_t offsets_lane_stride;
  int64_t strides[KTIR_MAX_DIMS];
  int64_t lo, hi;
  uint64_t winner;               /* const int32_t*: last-writer-wins table for scatters, or 0 */
  int64_t winner_base;           /* element offset of winner[0] */
  int32_t dtype;
  int32_t flags;
} ktir_leaf_t;

typedef struct ktir_instr {
  int8_t op, dst, a, b, c, dt;
  int16_t aux;       /* leaf / dim / predicate / source dtype / lane-scalar slot / pc of ENDELEM */
  int32_t imm;       /* CONST bits: float32 bits for float dtypes, int32 otherwise */
} ktir_instr_t;

/* A fused tile program over the iteration space [lanes, shape[0..ndim-1]].
 * mode 0 (flat): every element independently (elementwise chains, copies,
 *   broadcasts, transposes, casts, gathers, scatters).
 * mode 1 (rows): one workgroup per row (all dims but the last); ELEM blocks
 *   loop over the row, RED/FOLD implement the reference's pairwise-halving
 *   reduction (dialects/linalg_ops.py:86-133) in LDS; instructions outside
 *   ELEM blocks compute per-row values. */
typedef struct ktir_prog {
  int32_t mode, ndim, n_instr, n_leaves;
  /* flat mode: registers 0..n_pf-1 are preloaded from leaves pf_leaf[0..n_pf-1]
   * before the instructions run, so all of a vector's loads are in flight at once */
  int32_t n_pf;
  int8_t pf_leaf[4];
  int64_t lanes;
  int64_t shape[KTIR_MAX_DIMS];
  uint64_t lane_scalars;          /* const double* [lanes * n_lane_scalars] or 0 */
  int64_t n_lane_scalars;
  ktir_leaf_t leaves[KTIR_MAX_LEAVES];
  ktir_instr_t instr[KTIR_MAX_INSTR];
} ktir_prog_t;

/* ---- runtime (reference: interpreter.py:95-120 builds the simulated HBM) ---- */
const char* ktir_last_error(void);
int ktir_init(int device);
/* Waits for the library stream, then releases what ktir_init and later calls
 * created (stream, device error flag); device buffers from ktir_malloc stay
 * the caller's.  A later ktir_init starts over.  The reference has no teardown
 * (its HBM is garbage collected); this is the C side's end of a session. */
int ktir_shutdown(void);
int ktir_device_info(int* cu_count, int* clock_khz, int64_t* hbm_bytes, char* name, int name_len);
int ktir_malloc(uint64_t bytes, uint64_t* dptr);
int ktir_free(uint64_t dptr);
int ktir_memcpy_h2d(uint64_t dst, const void* src, uint64_t bytes);
int ktir_memcpy_d2h(void* dst, uint64_t src, uint64_t bytes);
int ktir_memcpy_d2d(uint64_t dst, uint64_t src, uint64_t bytes);
int ktir_memset(uint64_t dst, int value, uint64_t bytes);
int ktir_sync(void);
int ktir_check_error_flag(void);  /* device-side errors (negative indices) raised since the last call */
/* HIP events on the library's stream, for timing launches (created without the
   system-scope fence at record time: timestamps only, not synchronisation) */
int ktir_event_create(uint64_t* ev);
int ktir_event_record(uint64_t ev);
int ktir_event_elapsed_ms(uint64_t start, uint64_t stop, float* ms);
int ktir_event_destroy(uint64_t ev);

/* ---- fused tile programs ----
 * Replaces the per-op NumPy tile kernels of the reference: MemoryOps.load /
 * store (ops/memory_ops.py:724-865), the arith/math elementwise handlers
 * (dialects/_helpers.py:39-54, ops/arith_ops.py, ops/math_ops.py:27-138),
 * linalg.broadcast/transpose/fill/generic (dialects/linalg_ops.py:272-614),
 * linalg.reduce (:137-246) and the tensor reshapes (dialects/tensor_ops.py).
 * The descriptor travels by value in the kernel arguments (no host-device
 * copy per launch), so launches stay asynchronous on the library stream. */
int ktir_launch_program(const ktir_prog_t* prog);
/* Upper bound on the workgroups of one row-program launch (0, the default:
 * as many as the device holds at once, or one per row).  The row kernels
 * stride their workgroups over the rows, so results do not depend on it; a
 * small bound makes every workgroup run many rows (used by tests to cover
 * that path at small sizes).  No reference counterpart: a launch-shape knob. */
int ktir_set_row_grid_limit(int64_t max_workgroups);

/* ---- last-writer-wins scatter support ----
 * Reference memory.py:281-291 writes duplicates in enumeration order, so the
 * last position wins.  ktir_scatter_winners fills winner[off - winner_base]
 * with the largest flat position (lane * n + i) that writes each offset; a
 * following program whose store leaf carries `winner` writes only winners. */
int ktir_scatter_winners(const ktir_leaf_t* leaf, int64_t lanes, int64_t n, uint64_t winner);

/* ---- indirect access tiles (reference ops/memory_ops.py:224-576, 868-964) ----
 * out[l * n + p] = dir[l * dir_ls + p] + sum_k idx_k(l, p) * stride_k where
 * idx_k(l, p) = index value read from index view k at element
 * pos_k[l * pos_ls_k + p] (+ pos_lane_k[l]).  A negative index raises
 * KTIR_E_INDEX on the next ktir_check_error_flag().  Up to 4 indirect dims. */
typedef struct ktir_iat {
  int64_t lanes, n;
  uint64_t dir;          /* const int64_t* direct part */
  int64_t dir_ls;
  int32_t n_ind, pad;
  uint64_t idx_ptr[4];   /* device address of each index view's element 0 */
  int32_t idx_dtype[4];
  int64_t idx_hi[4];     /* valid element window of the index allocation */
  int64_t idx_lo[4];
  uint64_t pos[4];       /* const int64_t* */
  int64_t pos_ls[4];
  uint64_t pos_lane[4];  /* const int64_t* [lanes] or 0 */
  int64_t stride[4];
  uint64_t out;          /* int64_t* [lanes * n] */
} ktir_iat_t;
int ktir_iat_offsets(const ktir_iat_t* d);

/* ---- matmul tiles (reference dialects/linalg_ops.py:307-369, ops/arith_ops.py:324-340) ----
 * For every lane: C = A @ B (+ C0 when accumulate), A [M,K], B [K,N].
 * The K loop may be a fused `scf.for` reduction loop: `ksteps` steps, each
 * advancing A and B by a_kstep / b_kstep elements (the K-loop GEMM of
 * examples/triton-ktir/matmul_fwd_ktir.mlir:33-57).  f16 / bf16 operands use
 * gfx950 MFMA with f32 accumulation; f32 operands use f32 FMA. */
typedef struct ktir_mm {
  int64_t lanes, M, N, K, ksteps;
  ktir_leaf_t a, b;       /* strides[0] = row stride, strides[1] = column stride */
  int64_t a_kstep, b_kstep;
  ktir_leaf_t c;          /* result (f32 / f16 / bf16), strides[0..1] */
  ktir_leaf_t c0;         /* accumulator input when accumulate == 1 */
  int32_t accumulate;     /* 0: C = A@B; 1: C = C0 + A@B; 2: C = 0.0 + A@B (outs is a zero splat) */
  int32_t round_dt;       /* dtype the product is rounded to before accumulating (the KTIR operand dtype) */
  /* Optional: lanes grouped 2 x 2 into 256 x 256 blocks (M = N = 128 only):
   * const int32_t* [4 * n_quads] {top-left, top-right, bottom-left,
   * bottom-right}; the right lane's B starts N columns after the left's with
   * the same A, the bottom lane's A M rows below the top's with the same B.
   * 0 / 0: not grouped. */
  uint64_t quads;
  int64_t n_quads;
} ktir_mm_t;
int ktir_launch_matmul(const ktir_mm_t* d);

/* ---- ordered indirect read-modify-write of rows ----
 * Replaces, for a whole `scf.for` over index chunks, the reference's sequence
 *   g = ktdp.load src[ind(idx[p + k]), c]     (ops/memory_ops.py:868-915)
 *   o = ktdp.load dst[ind(idx[q + k]), c]
 *   ktdp.store f(o, g), dst[ind(idx[q + k]), c] (ops/memory_ops.py:918-964, memory.py:281-291)
 * run instance after instance (instances = (core, iteration) in the
 * reference's order, grid.py:595-616).  Results are bit-exact: inside one
 * instance a repeated destination row keeps only its last position; across
 * instances the updates of one row are applied one after another in order.
 * f is  dst = round_dt(op(dst, src))  (order 0) or  round_dt(op(src, dst))  (order 1). */
typedef struct ktir_rmw {
  int64_t n_inst, K, D;
  uint64_t dst_pos;        /* const int64_t* [n_inst]: index-tensor element of row 0's dst index */
  uint64_t src_pos;        /* const int64_t* [n_inst]: index-tensor element of row 0's src index */
  uint64_t dst_idx_ptr, src_idx_ptr;   /* index tensors (element 0) */
  int32_t dst_idx_dtype, src_idx_dtype;
  int64_t dst_idx_hi, src_idx_hi;      /* valid element window [0, hi) of the index tensors */
  uint64_t dst_ptr, src_ptr;           /* dst / src allocations (element 0) */
  int32_t dst_dtype, src_dtype;
  int64_t dst_base, dst_row, dst_col, dst_hi;  /* view origin, row and column strides, allocation size (elements) */
  int64_t src_base, src_row, src_col, src_hi;
  int32_t op, order, dt, pad;
  int64_t n_rows;          /* destination rows covered by the head table */
  uint64_t head;           /* int32_t [n_rows] scratch: -1 in every entry on entry, and so left on return */
  uint64_t link;           /* int32_t [2 * n_inst * K] scratch (a successor slot per entry):
                              -1 in every word on entry, and so left on return */
  uint64_t rows;           /* int32_t [2 * n_inst * K] scratch: the record of each entry */
  uint64_t srcs;           /* unused (0) */
} ktir_rmw_t;
int ktir_launch_row_rmw(const ktir_rmw_t* d);
/* Which apply kernel ktir_launch_row_rmw takes for `d` (host-only, launches
 * nothing): KTIR_RMW_ROWS, the destination-row-order kernel (f32 rows, f16 or
 * f32 sources, unit column stride, 16-byte aligned rows of a multiple of 128
 * columns), or KTIR_RMW_GENERIC; a negative KTIR_E_* code for a bad descriptor. */
#define KTIR_RMW_GENERIC 0
#define KTIR_RMW_ROWS 1
int ktir_rmw_variant(const ktir_rmw_t* d);
/* ktir_launch_row_rmw without caller scratch: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc).  head, link,
 * rows and srcs of `d` are ignored; the library's own 24 MiB device array
 * (one per device, set up by ktir_init, kept until the process ends) holds
 * them.  Limits: n_rows <= 2^21 and n_inst * K <= 2^20, else
 * KTIR_E_UNSUPPORTED.  Allocates nothing.  All calls on one device share the
 * array: calls that overlap on one device (other streams, other threads)
 * race and must not be issued. */
int ktir_launch_row_rmw_noalloc(const ktir_rmw_t* d);

/* ---- fused online-softmax attention loop ----
 * Replaces a whole KV `scf.for` of the flash-attention form (the reference's
 * examples/triton-ktir/paged_attention.mlir:191-396 and
 * notebooks/demo_gen_mlir.py:471-567 build the same loop from these ops):
 *   S = scale * (Q @ K_j^T), optional causal select(pred(kpos, qpos), S, neg),
 *   m' = max(m, rowmax S), P = exp(S - m'), alpha = exp(m - m'),
 *   acc' = acc * alpha + P @ V_j,  l' = l * alpha + rowsum P
 * with loop-carried f32 m, l (per row) and acc.  One lane = one query block
 * of M rows; lane l runs trips[l] iterations, the K tile of iteration j
 * starts at k_base[l] + j * k_step (V: v_base[l] + j * v_step).  M = N = D = 128, bf16 or f16
 * Q/K/V, MFMA with f32 accumulation; P enters the P @ V product as a
 * hi + lo pair of operand-type values (about 16 significant bits). */
typedef struct ktir_attn {
  int64_t lanes, M, N, D;
  uint64_t q_ptr, k_ptr, v_ptr;        /* element 0 of each tensor */
  uint64_t q_base, k_base, v_base;     /* const int64_t* [lanes] element offsets (iteration 0 for k, v) */
  int64_t q_row, k_row, v_row;         /* row strides in elements (column stride 1) */
  int64_t k_step, v_step;              /* element offset per iteration */
  uint64_t trips;                      /* const int32_t* [lanes] */
  uint64_t order;                      /* const int32_t* [lanes]: workgroup -> lane, or 0 */
  uint64_t qpos0;                      /* const int64_t* [lanes]: position of query row 0 */
  uint64_t kpos0;                      /* const int64_t* [lanes]: position of key 0 at iteration 0 */
  int64_t kpos_step;                   /* key position increment per iteration */
  float scale, neg;                    /* S multiplier; value of masked scores */
  int32_t causal, pred;                /* mask on (KTIR_CMP_* predicate keep = pred(kpos, qpos)) */
  int32_t dtype;                       /* KTIR_BF16 or KTIR_F16 */
  int32_t pad;
  uint64_t m_out, l_out, acc_out;      /* f32 [lanes, M], [lanes, M], [lanes, M, D] final state
                                          (acc_out 0: not written) */
  /* optional fused epilogue O = acc / l (the division of the reference's
   * examples/triton-ktir/paged_attention.mlir:400-420 and its store), rounded
   * to o_dtype and written at o_ptr + o_base[l] + row * o_row + d */
  uint64_t o_ptr, o_base;              /* 0: no epilogue; o_base: const int64_t* [lanes] */
  int64_t o_row;
  int32_t o_dtype;
  /* nonzero: v16_ptr and v16_flag still hold the copy and verdict of this V
   * range from an earlier launch, and V has not changed since (the caller
   * vouches for it), so the conversion is skipped */
  int32_t v16_ready;
  /* optional f16 copy of V for bf16 operands (0: not used): the launch first
   * converts elements [v16_lo, v16_lo + v16_n) of V into v16_ptr (f16, same
   * order; v16_lo and v16_n multiples of 8) and sets the device int32 at
   * v16_flag if any value is not finite or has |v| >= 65536.  If none is,
   * P @ V runs in f16 with P rounded once to f16 (11 significant bits; V
   * values below 2^-14 become f16 subnormals, off by at most 2^-25);
   * otherwise it runs in bf16 with P as hi + lo as without the copy.  Used
   * only when O = acc / l is the launch's one result (o_ptr set, acc_out 0);
   * f16 operands take the single-rounding f16 product under the same rule. */
  uint64_t v16_ptr, v16_flag;
  int64_t v16_lo, v16_n;
  /* optional (0 / 0: not used): const int32_t* [2 * n_pairs] lanes run two
   * per workgroup ({lane, lane or -1}; paired lanes have equal k_base, v_base
   * and kpos0; every lane appears once).  Used in the cases that run P @ V
   * in f16 with scale > 0 and (under a mask) neg = -inf: one group of four
   * wavefronts per lane, the two groups taking turns between MFMA work and
   * softmax.  Other launches ignore the pairs and run one lane per workgroup. */
  uint64_t pairs;
  int64_t n_pairs;
} ktir_attn_t;
int ktir_launch_attention(const ktir_attn_t* d);

/* ---- paged attention (reference examples/triton-ktir/paged_attention.mlir:194-392,
 * executed op by op per core and iteration by dialects/linalg_ops.py:307-596) ----
 * For every lane l, `trips[l]` iterations j of the online-softmax loop over
 * pages of a K / V cache, starting from m = m0, l = l0, acc = 0:
 *   page  = tbl[tbl_pos[l] + j * tbl_step]  (an index outside [tbl_lo, tbl_hi)
 *           reads 0; a negative one sets the device error flag and reads 0)
 *   K[c][x] = k[k_base[l] + page * k_page + c * k_row + x]   (c < N, x < D;
 *           outside [k_lo, k_hi) reads 0), V likewise
 *   s[r][c] = scale * sum_x Q[r][x] K[c][x], Q[r][x] = q[q_base[l] + r * q_row + x]
 *   causal: s = neg unless pred(kpos0[l] + j * kpos_step + c, qpos0[l] + r / row_div)
 *   m' = maximumf(m, max_c s); p = exp(s - m'); alpha = exp(m - m')
 *   acc' = acc * alpha + p V; l' = l * alpha + sum_c p; m = m'
 * all in f32.  Final m, l -> m_out / l_out [lanes, M], acc -> acc_out
 * [lanes, M, D].  Limits: D a multiple of 4, M * D <= 8192; LDS 4 * (M (D+8)
 * + N (D+8) + N D + M N + 3 M) bytes <= 160 KiB.  N = 16, M <= 16, D in
 * {32, 64, 128, 256} and one 16-bit type for q, k and v run on MFMA: exact
 * products, f32 sums in the MFMA's order, p rounded once to f16 (f16
 * operands) or as bf16 hi + lo (within rtol 1e-2 / atol 1e-3 of the f32
 * loop, not bit-exact). */
typedef struct ktir_pattn {
  int64_t lanes, M, N, D;
  uint64_t q_ptr, q_base;              /* q_base: const int64_t* [lanes] */
  int64_t q_row, q_lo, q_hi;
  int32_t q_dtype, kv_dtype;           /* KTIR_F16, KTIR_BF16 or KTIR_F32 */
  uint64_t k_ptr, v_ptr, k_base, v_base;
  int64_t k_row, v_row, k_page, v_page, k_lo, k_hi, v_lo, v_hi;
  uint64_t tbl_ptr, tbl_pos;           /* tbl_pos: const int64_t* [lanes] */
  int64_t tbl_step, tbl_lo, tbl_hi;
  int32_t tbl_dtype, pred;             /* KTIR_I8 / I16 / I32 / I64; KTIR_CMP_* keep predicate */
  uint64_t trips;                      /* const int32_t* [lanes] */
  uint64_t order;                      /* const int32_t* [lanes]: workgroup -> lane, or 0 */
  uint64_t qpos0, kpos0;               /* const int64_t* [lanes] */
  int64_t kpos_step, row_div;
  int32_t causal, pad;
  float scale, neg, m0, l0;
  uint64_t m_out, l_out, acc_out;
  /* optional finalisation (out_ptr != 0), the division and cast that follow
   * the reference's loop: out[o(r, x)] = (out_dtype)(acc[r][x] / l[r]) with
   * o(r, x) = out_base[l] + (r / out_grp) * out_gstride + (r % out_grp) *
   * out_row + x, elements outside [out_lo, out_hi) not written; m, l and acc
   * are written as well */
  uint64_t out_ptr, out_base;          /* out_base: const int64_t* [lanes] */
  int64_t out_grp, out_gstride, out_row, out_lo, out_hi;
  int32_t out_dtype, out_pad;
} ktir_pattn_t;
int ktir_launch_paged_attention(const ktir_pattn_t* d);

#ifdef __cplusplus
}
#endif
#endif /* KTIR_HIP_H */
