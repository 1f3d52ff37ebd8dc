// Fused online-softmax attention loop (flash attention) on gfx950 MFMA.
//
// One workgroup per lane (a block of 128 query rows); wavefront w owns query
// rows 32w .. 32w+31.  Per KV tile j (128 keys):
//   S^T = K_j Q^T   v_mfma_f32_32x32x16 with A = K rows from LDS and
//                   B = Q^T fragments kept in registers, so the D layout puts
//                   one query row per lane (lanes l and l^32 share a row):
//                   lane l holds row l%32, keys 8g + 4h + t (h = l/32).
//   row max / row sum: 64 values in the lane + one v_permlane32_swap.
//   O^T += V_j^T P^T  with A = V^T fragments read from the row-major V tile
//                   by ds_read_b64_tr_b16 (gfx950 LDS transpose read) and
//                   B = P^T fragments: the 8 consecutive keys a lane needs
//                   are 4 of its own values and 4 of lane l^32's, which one
//                   v_permlane32_swap per packed word delivers.
// so O rows also live in lanes and the per-row rescale by alpha needs no
// communication.  K and V tiles move HBM -> LDS with global_load_lds_dwordx4
// (no registers): the next K tile streams in while P @ V runs, the next V
// tile while the next scores are computed.  In LDS a tile row is 256 bytes
// with its 16-byte chunk c stored at slot c ^ swz16(row % 16) (an XOR of row
// bits), so every ds_read_b128 and ds_read_b64_tr_b16 phase hits distinct
// banks (with 32 or 64 LDS banks alike).
// Semantics follow the KTIR loop body (see ktir_hip.h):
// m' = max(m, rowmax S) (NaN-propagating like arith.maximumf),
// P = exp(S - m'), alpha = exp(m - m'), acc' = acc*alpha + P@V,
// l' = l*alpha + rowsum P, all in f32.  The kernel keeps P, acc and l
// relative to a base mr <= m that is moved up to m only when m passes it by
// more than 8 (and once at the end): the same values up to rounding, with
// the per-tile rescale of acc mostly gone.
#include <climits>

#include "ktir_common.h"

namespace ktir {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int AT = 128;            // M = N = D
constexpr float LOG2E = 1.44269504088896341f;

template <bool BF16>
__device__ __forceinline__ f32x16_t mfma_at(const uint4& a, const uint4& b, f32x16_t c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c,
                                                  0, 0, 0);
}

// (a, b) rounded to nearest-even in the operand type, packed low/high
template <bool BF16>
__device__ __forceinline__ uint32_t cvt2(float a, float b) {
  const f32x2_t v = {a, b};
  if constexpr (BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
  else return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
}

// the two operand-type values of a packed word, back in f32
template <bool BF16>
__device__ __forceinline__ f32x2_t uncvt2(uint32_t w) {
  if constexpr (BF16) return f32x2_t{__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u)};
  else return __builtin_convertvector(__builtin_bit_cast(f16x2_t, w), f32x2_t);
}

// P is carried into the P @ V product as hi + lo, both in the operand type
// (hi = P rounded, lo = the rounded remainder), so the product keeps about
// 16 significant bits of P instead of the operand type's 8 (bf16) / 11 (f16).
template <bool BF16>
__device__ __forceinline__ void split4(const float* p, uint32_t& h0, uint32_t& h1, uint32_t& l0, uint32_t& l1) {
  h0 = cvt2<BF16>(p[0], p[1]);
  h1 = cvt2<BF16>(p[2], p[3]);
  const f32x2_t a = uncvt2<BF16>(h0), b = uncvt2<BF16>(h1);
  l0 = cvt2<BF16>(__fsub_rn(p[0], a.x), __fsub_rn(p[1], a.y));
  l1 = cvt2<BF16>(__fsub_rn(p[2], b.x), __fsub_rn(p[3], b.y));
}

// v_permlane32_swap: lanes 32-63 of a trade places with lanes 0-31 of b, so
// afterwards lanes 0-31 hold a of both half-waves (own in a, the other
// half's in b) and lanes 32-63 hold b of both (the other half's in a)
__device__ __forceinline__ void swap32(uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  a = r[0];
  b = r[1];
}

// value of the other half-wave's lane l ^ 32
__device__ __forceinline__ float other_half(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// max / sum of x over the lane pair (l, l ^ 32): after v_permlane32_swap the
// two results hold the pair's two values in either order, so one maximum or
// add of them gives both lanes the same result (IEEE add commutes)
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __builtin_elementwise_maximum(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __fadd_rn(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// arith.maximumf: NaN-propagating maximum (v_maximum3_f32 on gfx950)
__device__ __forceinline__ float fmax_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float fmax3_nan(float a, float b, float c) { return fmax_nan(fmax_nan(a, b), c); }

// x = -inf in the lanes of mask, in place (v_cndmask_b32 on x's own
// register: the caller's S values keep the registers the MFMAs wrote)
// -inf where `kill` holds: a plain select, so the compiler inserts the wait
// states between an MFMA result and this VALU read itself
__device__ __forceinline__ float mask_ninf(float x, bool kill) { return kill ? -__builtin_inff() : x; }

// e^x as 2^(x log2 e) on the hardware exp2 (v_exp_f32)
__device__ __forceinline__ float exp_f(float x) { return __builtin_amdgcn_exp2f(__fmul_rn(x, LOG2E)); }

// ds_read_b64_tr_b16: in each 16-lane group, member t receives element t % 4
// of the 4-element chunks addressed by members 4s + t / 4, s = 0..3
__device__ __forceinline__ uint2 ds_tr16(const uint16_t* p) {
  const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t*)p);
  return __builtin_bit_cast(uint2, v);
}

// slot permutation of the 16 chunks of a 256-byte LDS row r
__device__ __forceinline__ int swz16(int r) {
  return ((r & 1) ? 4 : 0) ^ ((r & 2) ? 10 : 0) ^ ((r & 4) ? 1 : 0) ^ ((r & 8) ? 8 : 0);
}

// byte offset of lane l's chunk in a 4-row block whose rows have
// row % 16 = 4 q + l / 16 (row l / 16 of the block)
__device__ __forceinline__ uint32_t tile_lane_off(int l, int64_t row_stride, int q) {
  const int r = l >> 4, c = (l & 15) ^ swz16(4 * q + r);
  return (uint32_t)((r * row_stride + 8 * c) * 2);
}

// Wave w (uniform) copies rows 32w .. 32w+31 of a 128 x 128 tile into LDS: 8
// blocks of 4 rows (1 KB), lane l filling slot l % 16 of row 4b + l / 16 of
// block b.  buffer_load ... lds: a scalar buffer base per wave, a scalar
// offset per block and a 32-bit lane offset that depends on b % 4 (computed
// here: a few VALU instructions instead of registers held across the loop).
__device__ __forceinline__ void tile_to_lds(const uint16_t* src, int64_t row_stride, uint16_t* lds, int wu, int l) {
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(src + (int64_t)(32 * wu) * row_stride), (short)0, (int)((31 * row_stride + AT) * 2), 0x00020000);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(lds + 512 * (8 * wu + i)),
                                             16, tile_lane_off(l, row_stride, i & 3), (int)(i * 8 * row_stride), 0, 0);
}

#define AT_S_LOOP(BODY)                                      \
  _Pragma("unroll") for (int kt = 0; kt < 4; ++kt) {         \
    _Pragma("unroll") for (int i = 0; i < 16; ++i) { BODY; } }

// The position mask keeps score (row, key) iff ((lo <= kpos - qpos <= hi) != inv).
// PV16: the P @ V product in f16 (V f16: the f16 operands, or the f16 copy of
// bf16 V), P rounded once to f16; else in the operand type with P as hi + lo.
// one query block (lane order[blk], or blk) of the launch
template <bool BF16, bool PV16>
__device__ __forceinline__ void attn_block(const ktir_attn_t& d, int mlo, int mhi, int minv, int64_t blk) {
  __shared__ __align__(16) uint16_t Ks[AT * AT];    // K tile, [key][d] (chunk-swizzled rows)
  __shared__ __align__(16) uint16_t Vs[AT * AT];    // V tile, [key][d] (chunk-swizzled rows)
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, h = l >> 5, r32 = l & 31;
  const int64_t lane = uni(d.order ? ((const int32_t*)d.order)[blk] : blk);
  const int T = uni(((const int32_t*)d.trips)[lane]);
  const uint16_t* Q = (const uint16_t*)d.q_ptr;
  const uint16_t* K = (const uint16_t*)d.k_ptr;
  const uint16_t* V = BF16 && PV16 ? (const uint16_t*)d.v16_ptr - d.v16_lo : (const uint16_t*)d.v_ptr;
  const int row = w * 32 + r32;                      // this lane's query row
  const int64_t kb0 = uni(((const int64_t*)d.k_base)[lane]), vb0 = uni(((const int64_t*)d.v_base)[lane]);
  uint4 qf[8];                                       // Q^T fragments: Q[row][16 s + 8 h .. + 8]
  const int wu = __builtin_amdgcn_readfirstlane(w);
  if (T > 0) {
    const uint16_t* qr = Q + uni(((const int64_t*)d.q_base)[lane]) + (int64_t)row * d.q_row + 8 * h;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = *(const uint4*)(qr + 16 * s);
    tile_to_lds(K + kb0, d.k_row, Ks, wu, l);
    tile_to_lds(V + vb0, d.v_row, Vs, wu, l);
    __builtin_amdgcn_s_waitcnt(0);
  }
  __syncthreads();
  const int64_t qpos = uni(((const int64_t*)d.qpos0)[lane]) + row;
  const int64_t kpos00 = uni(((const int64_t*)d.kpos0)[lane]);
  const bool pos_scale = d.scale > 0.f;
  const float c1 = __fmul_rn(d.scale, LOG2E);
  const f32x16_t z16 = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  f32x16_t o0 = z16, o1 = z16, o2 = z16, o3 = z16;   // O^T tiles: d = 32 dt + 8g + 4h + t, row r32
  // m: running row max (the reference's m).  P, lsum and O are kept relative
  // to mr <= m, moved up to m only when m passes mr by more than AT_REBASE
  // (P <= e^8 meanwhile), and brought to m once after the loop: the same
  // quantities as rescaling every tile, with far fewer rescales.
  float m = -__builtin_inff(), mr = -__builtin_inff(), lsum = 0.f;
#define AT_REBASE(MN)                                                    \
  do {                                                                   \
    const bool up = (MN) > __fadd_rn(mr, 8.0f);                          \
    if (__any(up)) {                                                     \
      const float al = up ? exp_f(__fsub_rn(mr, (MN))) : 1.f;            \
      _Pragma("unroll") for (int i = 0; i < 16; ++i) {                   \
        o0[i] = __fmul_rn(o0[i], al);                                    \
        o1[i] = __fmul_rn(o1[i], al);                                    \
        o2[i] = __fmul_rn(o2[i], al);                                    \
        o3[i] = __fmul_rn(o3[i], al);                                    \
      }                                                                  \
      lsum = __fmul_rn(lsum, al);                                        \
      mr = up ? (MN) : mr;                                               \
    }                                                                    \
  } while (0)
  // K A-fragments: row 32 kt + r32, chunk 2 s + h at slot (2 s + h) ^ swz16(r32 % 16)
  const int k_off = r32 * AT;
  const int k_x = swz16(r32 & 15);
  // V^T fragment rows d = 32 dt + l % 32, keys 16 ks + 8 h + [0..8): member tj of
  // 16-lane group tg addresses key 8 (tg / 2) + tj / 4 (+4), d 16 (tg % 2) + 4 (tj % 4)
  const int tg = l >> 4, tj = l & 15;
  const int v_row0 = 8 * (tg >> 1) + (tj >> 2);
  const int v_c = 2 * (tg & 1) + ((tj >> 1) & 1), v_in = 4 * (tj & 1);
  // chunk index bases (4 dt + v_c) ^ swz16(row) = 4 dt ^ (v_c ^ swz16(row)): two per lane
  const int v_b0 = v_row0 * AT + v_in, v_x0 = v_c ^ swz16(v_row0), v_x1 = v_c ^ swz16(v_row0 + 4);
  for (int j = 0; j < T; ++j) {
    const bool more = j + 1 < T;
    // fragment addresses are recomputed in the loop from opaque bases (a few
    // VALU instructions) instead of 16 registers held across it
    int kx = k_x, vfb = v_b0, vx0 = v_x0, vx1 = v_x1;
    asm volatile("" : "+v"(kx), "+v"(vfb), "+v"(vx0), "+v"(vx1));
    // S^T = K Q^T: 4 key tiles x 8 d-steps
    f32x16_t s0 = z16, s1 = z16, s2 = z16, s3 = z16;
    // MFMA blocks run at raised wave priority: of the two waves sharing a
    // SIMD, the one with matrix work issues first, which moves the other's
    // softmax under its MFMAs instead of in step with them
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const uint16_t* kp = &Ks[k_off + 8 * ((2 * s + h) ^ kx)];
      s0 = mfma_at<BF16>(*(const uint4*)(kp + 0 * 32 * AT), qf[s], s0);
      s1 = mfma_at<BF16>(*(const uint4*)(kp + 1 * 32 * AT), qf[s], s1);
      s2 = mfma_at<BF16>(*(const uint4*)(kp + 2 * 32 * AT), qf[s], s2);
      s3 = mfma_at<BF16>(*(const uint4*)(kp + 3 * 32 * AT), qf[s], s3);
    }
    __builtin_amdgcn_s_setprio(0);
    // lane value (kt, i) is key kt*32 + 8(i/4) + 4h + i%4 of row `row`
    float sv[4][16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      sv[0][i] = s0[i];
      sv[1][i] = s1[i];
      sv[2][i] = s2[i];
      sv[3][i] = s3[i];
    }
    const int64_t kpos_j = kpos00 + (int64_t)j * d.kpos_step;
    const int dbase = (int)(kpos_j - qpos);          // kpos - qpos of this lane's key 0; keys add 0 .. 127
    const bool all_keep = !d.causal ||
        (minv ? (dbase + 127 < mlo || dbase > mhi) : (dbase >= mlo && dbase + 127 <= mhi));
    float mn, ls;
    // no masked score in the wave and scale > 0: rowmax S = scale * rowmax(QK)
    // (rounding is monotonic for scale > 0) and P = 2^(QK * scale log2e - mr log2e)
    const bool fast = pos_scale && __all(all_keep);
    if (fast) {
      float x0 = fmax_nan(sv[0][0], sv[0][1]), x1 = fmax_nan(sv[1][0], sv[1][1]);
      float x2 = fmax_nan(sv[2][0], sv[2][1]), x3 = fmax_nan(sv[3][0], sv[3][1]);
#pragma unroll
      for (int i = 2; i < 16; i += 2) {
        x0 = fmax_nan(x0, fmax_nan(sv[0][i], sv[0][i + 1]));
        x1 = fmax_nan(x1, fmax_nan(sv[1][i], sv[1][i + 1]));
        x2 = fmax_nan(x2, fmax_nan(sv[2][i], sv[2][i + 1]));
        x3 = fmax_nan(x3, fmax_nan(sv[3][i], sv[3][i + 1]));
      }
      float xm = fmax_nan(fmax_nan(x0, x1), fmax_nan(x2, x3));
      xm = fmax_nan(xm, other_half(xm));
      mn = fmax_nan(m, __fmul_rn(d.scale, xm));
    } else {
      AT_S_LOOP(sv[kt][i] = __fmul_rn(d.scale, sv[kt][i]))
      if (d.causal) {
        AT_S_LOOP({
          const int df = dbase + kt * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
          if ((df >= mlo && df <= mhi) == (bool)minv) sv[kt][i] = d.neg;
        })
      }
      float xm = -__builtin_inff();
      AT_S_LOOP(xm = fmax_nan(xm, sv[kt][i]))
      xm = fmax_nan(xm, other_half(xm));
      mn = fmax_nan(m, xm);
    }
    AT_REBASE(mn);
    if (fast) {
      const float c0 = -__fmul_rn(mr, LOG2E);
      AT_S_LOOP(sv[kt][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[kt][i], c1, c0)))
    } else {
      AT_S_LOOP(sv[kt][i] = exp_f(__fsub_rn(sv[kt][i], mr)))
    }
    {
      float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        a0 = __fadd_rn(a0, sv[0][i]);
        a1 = __fadd_rn(a1, sv[1][i]);
        a2 = __fadd_rn(a2, sv[2][i]);
        a3 = __fadd_rn(a3, sv[3][i]);
      }
      ls = __fadd_rn(__fadd_rn(a0, a1), __fadd_rn(a2, a3));
      ls = __fadd_rn(ls, other_half(ls));
    }
    lsum = __fadd_rn(lsum, ls);
    m = mn;
    __builtin_amdgcn_s_waitcnt(0);                    // this wave's part of V_j has landed
    __syncthreads();                                  // every wave: done with Ks, V_j in LDS
    if (more) tile_to_lds(K + kb0 + (int64_t)(j + 1) * d.k_step, d.k_row, Ks, wu, l);
    // O^T += V^T P^T over 8 key-steps of 16 keys
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      // lane half h holds key groups g0 (a*) and g0 + 1 (b*) of key tile ks / 2;
      // after the swaps both halves hold keys 16 ks + 8 h + [0..8) in order
      const int kt = ks >> 1, g0 = 2 * (ks & 1);
      const uint16_t* vt = &Vs[16 * ks * AT];
      uint4 a[4];
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const uint2 lo = ds_tr16(vt + vfb + 8 * ((4 * dt) ^ vx0)), hi = ds_tr16(vt + vfb + 4 * AT + 8 * ((4 * dt) ^ vx1));
        a[dt] = make_uint4(lo.x, lo.y, hi.x, hi.y);
      }
      if constexpr (PV16) {
        uint32_t ah0 = cvt2<false>(sv[kt][4 * g0], sv[kt][4 * g0 + 1]);
        uint32_t ah1 = cvt2<false>(sv[kt][4 * g0 + 2], sv[kt][4 * g0 + 3]);
        uint32_t bh0 = cvt2<false>(sv[kt][4 * g0 + 4], sv[kt][4 * g0 + 5]);
        uint32_t bh1 = cvt2<false>(sv[kt][4 * g0 + 6], sv[kt][4 * g0 + 7]);
        swap32(ah0, bh0);
        swap32(ah1, bh1);
        const uint4 ph = make_uint4(ah0, ah1, bh0, bh1);
        o0 = mfma_at<false>(a[0], ph, o0);
        o1 = mfma_at<false>(a[1], ph, o1);
        o2 = mfma_at<false>(a[2], ph, o2);
        o3 = mfma_at<false>(a[3], ph, o3);
      } else {
        uint32_t ah0, ah1, al0, al1, bh0, bh1, bl0, bl1;
        split4<BF16>(&sv[kt][4 * g0], ah0, ah1, al0, al1);
        split4<BF16>(&sv[kt][4 * g0 + 4], bh0, bh1, bl0, bl1);
        swap32(ah0, bh0);
        swap32(ah1, bh1);
        swap32(al0, bl0);
        swap32(al1, bl1);
        const uint4 ph = make_uint4(ah0, ah1, bh0, bh1), pl = make_uint4(al0, al1, bl0, bl1);
        o0 = mfma_at<BF16>(a[0], ph, o0);
        o1 = mfma_at<BF16>(a[1], ph, o1);
        o2 = mfma_at<BF16>(a[2], ph, o2);
        o3 = mfma_at<BF16>(a[3], ph, o3);
        o0 = mfma_at<BF16>(a[0], pl, o0);
        o1 = mfma_at<BF16>(a[1], pl, o1);
        o2 = mfma_at<BF16>(a[2], pl, o2);
        o3 = mfma_at<BF16>(a[3], pl, o3);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_s_waitcnt(0);                    // this wave's part of K_{j+1} has landed
    __syncthreads();                                  // every wave: done with Vs, K_{j+1} in LDS
    if (more) tile_to_lds(V + vb0 + (int64_t)(j + 1) * d.v_step, d.v_row, Vs, wu, l);
  }
  // final state, relative to m
  if (T > 0) {
    const float fin = exp_f(__fsub_rn(mr, m));
    if (!__all(fin == 1.f)) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        o0[i] = __fmul_rn(o0[i], fin);
        o1[i] = __fmul_rn(o1[i], fin);
        o2[i] = __fmul_rn(o2[i], fin);
        o3[i] = __fmul_rn(o3[i], fin);
      }
      lsum = __fmul_rn(lsum, fin);
    }
  }
#undef AT_REBASE
  if (h == 0) {
    ((float*)d.m_out)[lane * AT + row] = m;
    ((float*)d.l_out)[lane * AT + row] = lsum;
  }
  if (d.acc_out) {
    float* orow = (float*)d.acc_out + (lane * AT + row) * AT + 4 * h;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      *(float4*)(orow + 0 * 32 + 8 * g) = make_float4(o0[4 * g], o0[4 * g + 1], o0[4 * g + 2], o0[4 * g + 3]);
      *(float4*)(orow + 1 * 32 + 8 * g) = make_float4(o1[4 * g], o1[4 * g + 1], o1[4 * g + 2], o1[4 * g + 3]);
      *(float4*)(orow + 2 * 32 + 8 * g) = make_float4(o2[4 * g], o2[4 * g + 1], o2[4 * g + 2], o2[4 * g + 3]);
      *(float4*)(orow + 3 * 32 + 8 * g) = make_float4(o3[4 * g], o3[4 * g + 1], o3[4 * g + 2], o3[4 * g + 3]);
    }
  }
  if (d.o_ptr) {
    // O = acc / l (f32, correctly rounded), then rounded to the output type
    const int64_t ob = uni(((const int64_t*)d.o_base)[lane]) + (int64_t)row * d.o_row + 4 * h;
#define AT_EPI(o, dt)                                                                            \
    _Pragma("unroll") for (int g = 0; g < 4; ++g) {                                              \
      const float q0 = __fdiv_rn(o[4 * g], lsum), q1 = __fdiv_rn(o[4 * g + 1], lsum);            \
      const float q2 = __fdiv_rn(o[4 * g + 2], lsum), q3 = __fdiv_rn(o[4 * g + 3], lsum);        \
      const int64_t e = ob + 32 * dt + 8 * g;                                                    \
      if (d.o_dtype == KTIR_F32)                                                                 \
        *(float4*)((float*)d.o_ptr + e) = make_float4(q0, q1, q2, q3);                           \
      else if (d.o_dtype == KTIR_BF16)                                                           \
        *(uint2*)((uint16_t*)d.o_ptr + e) = make_uint2(cvt2<true>(q0, q1), cvt2<true>(q2, q3));   \
      else                                                                                       \
        *(uint2*)((uint16_t*)d.o_ptr + e) = make_uint2(cvt2<false>(q0, q1), cvt2<false>(q2, q3)); \
    }
    AT_EPI(o0, 0)
    AT_EPI(o1, 1)
    AT_EPI(o2, 2)
    AT_EPI(o3, 3)
#undef AT_EPI
  }
}

template <bool BF16, bool PV16>
__global__ __launch_bounds__(256, 2) void attn_kernel(const ktir_attn_t d, int mlo, int mhi, int minv) {
  if (BF16 && d.v16_ptr && d.o_ptr && !d.acc_out) {
    // the conversion before this launch decided which of the two kernels runs
    if ((*(const int*)d.v16_flag != 0) == PV16) return;
  }
  attn_block<BF16, PV16>(d, mlo, mhi, minv, blockIdx.x);
}

// The hi + lo bf16 variant behind the f16 form: it runs only when the V
// conversion found a value f16 cannot hold, and otherwise every workgroup
// exits at once, so it takes a small grid whose workgroups loop over the
// query blocks.
__global__ __launch_bounds__(256, 2) void attn_kernel_gated(const ktir_attn_t d, int mlo, int mhi, int minv) {
  if (*(const int*)d.v16_flag == 0) return;
  for (int64_t blk = blockIdx.x; blk < d.lanes; blk += gridDim.x) {
    if (blk != (int64_t)blockIdx.x) __syncthreads();   // the previous block's LDS reads are done
    attn_block<true, false>(d, mlo, mhi, minv, blk);
  }
}

// ---- two query blocks per workgroup, alternating matrix and vector work ----
//
// Workgroup of 8 wavefronts: group g = w / 4 runs query block pairs[2 b + g]
// exactly as attn_kernel runs one (wave w % 4 owns 32 rows), and both groups
// read the same K/V tile stream (the host pairs lanes with equal K/V bases
// and key positions).  Per KV tile j a group has a matrix phase M_j
// (O += P_{j-1} V_{j-1}, then S_j = K_j Q^T: 64 MFMAs) and a vector phase
// V_j (softmax of S_j into P_j: max, exp, row sum, about 300 VALU
// instructions).  Group 1 runs one phase behind group 0 and every phase ends
// at a workgroup barrier, so on each SIMD one wavefront's MFMAs always run
// beside the other's softmax.  P @ V in f16 (P rounded once), as the PV16
// form of attn_kernel.  K and V tiles are double-buffered: at even phase 2i
// every wave streams its 16 rows of K_{i+1} and V_i into the buffers tiles
// i - 1 and i - 2 have left; they are waited for at the end of phase 2i + 1.

// Wave w8 (uniform, 0..7) copies rows 16 w8 .. 16 w8 + 15 of a 128 x 128 tile
// into LDS: 4 blocks of 4 rows, as tile_to_lds.
__device__ __forceinline__ void tile16_to_lds(const uint16_t* src, int64_t row_stride, uint16_t* lds, int w8, int l) {
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(src + (int64_t)(16 * w8) * row_stride), (short)0, (int)((15 * row_stride + AT) * 2), 0x00020000);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(lds + 512 * (4 * w8 + i)),
                                             16, tile_lane_off(l, row_stride, i), (int)(i * 8 * row_stride), 0, 0);
}

// c + the two f16 values of w (v_dot2_f32_f16 against (1, 1): exact
// products, one f32 sum)
__device__ __forceinline__ float dot2_one(uint32_t w, float c) {
  const f16x2_t one = {(_Float16)1.0f, (_Float16)1.0f};
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w), one, c, false);
}

// row sum of P: this lane's 64 values plus the other half-wave's
__device__ __forceinline__ float pp_rowsum(const f32x16_t (&p)[4]) {
  float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    a0 = __fadd_rn(a0, p[0][i]);
    a1 = __fadd_rn(a1, p[1][i]);
    a2 = __fadd_rn(a2, p[2][i]);
    a3 = __fadd_rn(a3, p[3][i]);
  }
  const float ls = __fadd_rn(__fadd_rn(a0, a1), __fadd_rn(a2, a3));
  return __fadd_rn(ls, other_half(ls));
}

template <bool BF16>
__global__ __launch_bounds__(512, 1) void attn_pp(const ktir_attn_t d, int mlo, int mhi, int minv) {
  if (BF16 && *(const int*)d.v16_flag != 0) return;   // V not exact in f16: attn_kernel<true, false> runs
  __shared__ __align__(16) uint16_t K0s[AT * AT];     // K tiles of even / odd j
  __shared__ __align__(16) uint16_t K1s[AT * AT];
  __shared__ __align__(16) uint16_t V0s[AT * AT];     // V tiles of even / odd j
  __shared__ __align__(16) uint16_t V1s[AT * AT];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, h = l >> 5, r32 = l & 31;
  const int g = __builtin_amdgcn_readfirstlane(w >> 2), w8 = __builtin_amdgcn_readfirstlane(w);
  const int32_t* pairs = (const int32_t*)d.pairs;
  const int la = uni(pairs[2 * blockIdx.x]), lb = uni(pairs[2 * blockIdx.x + 1]);
  const int32_t* trips = (const int32_t*)d.trips;
  const int ta = la >= 0 ? uni(trips[la]) : 0, tb = lb >= 0 ? uni(trips[lb]) : 0;
  const int lane = g ? lb : la, T = g ? tb : ta, Tmax = ta > tb ? ta : tb;
  const int lk = la >= 0 ? la : lb;                   // whose K/V stream (both share it)
  const uint16_t* K = (const uint16_t*)d.k_ptr;
  const uint16_t* V = BF16 ? (const uint16_t*)d.v16_ptr - d.v16_lo : (const uint16_t*)d.v_ptr;
  const int64_t kbase = lk >= 0 ? uni(((const int64_t*)d.k_base)[lk]) : 0;
  const int64_t vbase = lk >= 0 ? uni(((const int64_t*)d.v_base)[lk]) : 0;
  const int row = (w & 3) * 32 + r32;
  uint4 qf[8];
  int64_t qpos = 0;
  if (T > 0) {
    const uint16_t* qr = (const uint16_t*)d.q_ptr + uni(((const int64_t*)d.q_base)[lane]) + (int64_t)row * d.q_row + 8 * h;
#pragma unroll
    for (int st = 0; st < 8; ++st) qf[st] = *(const uint4*)(qr + 16 * st);
    qpos = uni(((const int64_t*)d.qpos0)[lane]) + row;
  }
  const int64_t kpos00 = lk >= 0 ? uni(((const int64_t*)d.kpos0)[lk]) : 0;
  if (Tmax > 0) tile16_to_lds(K + kbase, d.k_row, K0s, w8, l);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const float c1 = __fmul_rn(d.scale, LOG2E);
  const f32x16_t z16 = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  f32x16_t o0 = z16, o1 = z16, o2 = z16, o3 = z16;
  f32x16_t sc[4] = {z16, z16, z16, z16};             // S_j between M_j and V_j
  uint4 ph[8];                                        // P_j (f16, in MFMA operand order) between V_j and M_{j+1}
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) ph[ks] = make_uint4(0, 0, 0, 0);
  float m = -__builtin_inff(), mr = -__builtin_inff(), lsum = 0.f;
  const int k_off = r32 * AT, k_x = swz16(r32 & 15);
  const int tg = l >> 4, tj = l & 15;
  // P@V runs over the keys in the order that puts every lane's own S values
  // in its P fragment: MFMA k = 8h + j is key 4h + j (j < 4) or 8 + 4h + j - 4
  // of the 16-key step, so the V fragment of half h reads rows 4h .. 4h+3
  // and 8 + 4h .. 8 + 4h + 3 of the step (no exchange between half-waves)
  const int v_row0 = 4 * (tg >> 1) + (tj >> 2);
  const int v_c = 2 * (tg & 1) + ((tj >> 1) & 1), v_in = 4 * (tj & 1);
  const int v_b0 = v_row0 * AT + v_in, v_x0 = v_c ^ swz16(v_row0), v_x1 = v_c ^ swz16(v_row0 + 8);

  // matrix phase M_j: O += P_{j-1} V_{j-1} (V tile in VB), then S_j = K_j Q^T (K tile in KB)
#define PP_M(J, KB, VB)                                                                              \
  do {                                                                                               \
    int kx = k_x, vfb = v_b0, vx0 = v_x0, vx1 = v_x1;                                                \
    asm volatile("" : "+v"(kx), "+v"(vfb), "+v"(vx0), "+v"(vx1));                                    \
    __builtin_amdgcn_s_setprio(1);                                                                   \
    if ((J) >= 1 && (J) <= T) {                                                                      \
      _Pragma("unroll") for (int ks = 0; ks < 8; ++ks) {                                             \
        const uint16_t* vt = &(VB)[16 * ks * AT];                                                    \
        uint4 a[4];                                                                                  \
        _Pragma("unroll") for (int dt = 0; dt < 4; ++dt) {                                           \
          const uint2 lo = ds_tr16(vt + vfb + 8 * ((4 * dt) ^ vx0));                                 \
          const uint2 hi = ds_tr16(vt + vfb + 8 * AT + 8 * ((4 * dt) ^ vx1));                        \
          a[dt] = make_uint4(lo.x, lo.y, hi.x, hi.y);                                                \
        }                                                                                            \
        o0 = mfma_at<false>(a[0], ph[ks], o0);                                                       \
        o1 = mfma_at<false>(a[1], ph[ks], o1);                                                       \
        o2 = mfma_at<false>(a[2], ph[ks], o2);                                                       \
        o3 = mfma_at<false>(a[3], ph[ks], o3);                                                       \
      }                                                                                              \
      /* the 8 fragment reads of key step ks + 1 between the 4 MFMAs of ks */                       \
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);                                             \
      _Pragma("unroll") for (int x = 0; x < 28; ++x) {                                               \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                           \
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);                                           \
      }                                                                                              \
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);                                             \
    }                                                                                                \
    if ((J) < T) {                                                                                   \
      _Pragma("unroll") for (int kt = 0; kt < 4; ++kt) sc[kt] = z16;                                 \
      _Pragma("unroll") for (int st = 0; st < 8; ++st) {                                             \
        const uint16_t* kp = &(KB)[k_off + 8 * ((2 * st + h) ^ kx)];                                 \
        _Pragma("unroll") for (int kt = 0; kt < 4; ++kt)                                             \
          sc[kt] = mfma_at<BF16>(*(const uint4*)(kp + kt * 32 * AT), qf[st], sc[kt]);                \
      }                                                                                              \
      /* the 4 K-fragment reads of d-step st + 1 between the 4 MFMAs of st */                      \
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);                                             \
      _Pragma("unroll") for (int x = 0; x < 28; ++x) {                                               \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                           \
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                           \
      }                                                                                              \
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);                                             \
    }                                                                                                \
    __builtin_amdgcn_s_setprio(0);                                                                   \
  } while (0)

  // vector phase V_j: softmax of S_j (online, base mr as in attn_kernel) into
  // ph.  The launch runs this kernel only for scale > 0 and, under a position
  // mask, the fill value -inf: a score outside the kept positions becomes
  // -inf in place, after which one form serves every tile (the maximum
  // ignores -inf unless the whole row is masked, and 2^(-inf c1 + c0) = 0,
  // exactly what exp(-inf - m) gives).
#define PP_V(J)                                                                                      \
  do {                                                                                               \
    if ((J) >= 0 && (J) < T) {                                                                       \
      const int dbase = (int)(kpos00 + (int64_t)(J) * d.kpos_step - qpos);                           \
      const bool all_keep = !d.causal ||                                                             \
          (minv ? (dbase + 127 < mlo || dbase > mhi) : (dbase >= mlo && dbase + 127 <= mhi));        \
      if (!__all(all_keep)) {                                                                        \
        _Pragma("unroll") for (int kt = 0; kt < 4; ++kt) {                                           \
          _Pragma("unroll") for (int i = 0; i < 16; ++i) {                                           \
            const int df = dbase + kt * 32 + 8 * (i >> 2) + 4 * h + (i & 3);                         \
            sc[kt][i] = mask_ninf(sc[kt][i], (df >= mlo && df <= mhi) == (bool)minv);                \
          }                                                                                          \
        }                                                                                            \
      }                                                                                              \
      /* four chains of v_maximum3 (15 scores each), then the 4 left and the chains */               \
      float x[4];                                                                                    \
      _Pragma("unroll") for (int kt = 0; kt < 4; ++kt) {                                             \
        x[kt] = fmax3_nan(sc[kt][0], sc[kt][1], sc[kt][2]);                                          \
        _Pragma("unroll") for (int i = 3; i < 15; i += 2) x[kt] = fmax3_nan(x[kt], sc[kt][i], sc[kt][i + 1]); \
      }                                                                                              \
      const float y0 = fmax3_nan(x[0], sc[0][15], sc[1][15]);                                        \
      const float y1 = fmax3_nan(x[1], sc[2][15], sc[3][15]);                                        \
      const float xm = pair_max(fmax_nan(fmax3_nan(y0, y1, x[2]), x[3]));                            \
      const float mn = fmax_nan(m, __fmul_rn(d.scale, xm));                                          \
      const bool up = mn > __fadd_rn(mr, 8.0f);                                                      \
      if (__any(up)) {                                                                               \
        const float al = up ? exp_f(__fsub_rn(mr, mn)) : 1.f;                                        \
        _Pragma("unroll") for (int i = 0; i < 16; ++i) {                                             \
          o0[i] = __fmul_rn(o0[i], al);                                                              \
          o1[i] = __fmul_rn(o1[i], al);                                                              \
          o2[i] = __fmul_rn(o2[i], al);                                                              \
          o3[i] = __fmul_rn(o3[i], al);                                                              \
        }                                                                                            \
        lsum = __fmul_rn(lsum, al);                                                                  \
        mr = up ? mn : mr;                                                                           \
      }                                                                                              \
      const float c0 = -__fmul_rn(mr, LOG2E);                                                        \
      AT_S_LOOP(sc[kt][i] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kt][i], c1, c0)))               \
      m = mn;                                                                                        \
      /* the row sum from the f16 P the product uses: two values per dot2 */                        \
      float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;                                                  \
      _Pragma("unroll") for (int ks = 0; ks < 8; ++ks) {                                             \
        const int kt = ks >> 1, g0 = 2 * (ks & 1);                                                   \
        uint32_t ah0 = cvt2<false>(sc[kt][4 * g0], sc[kt][4 * g0 + 1]);                              \
        uint32_t ah1 = cvt2<false>(sc[kt][4 * g0 + 2], sc[kt][4 * g0 + 3]);                          \
        uint32_t bh0 = cvt2<false>(sc[kt][4 * g0 + 4], sc[kt][4 * g0 + 5]);                          \
        uint32_t bh1 = cvt2<false>(sc[kt][4 * g0 + 6], sc[kt][4 * g0 + 7]);                          \
        s0 = dot2_one(ah0, s0);                                                                      \
        s1 = dot2_one(ah1, s1);                                                                      \
        s2 = dot2_one(bh0, s2);                                                                      \
        s3 = dot2_one(bh1, s3);                                                                      \
        ph[ks] = make_uint4(ah0, ah1, bh0, bh1);                                                     \
      }                                                                                              \
      lsum = __fadd_rn(lsum, pair_sum(__fadd_rn(__fadd_rn(s0, s1), __fadd_rn(s2, s3))));             \
    }                                                                                                \
  } while (0)

  // at even phase 2i: K_{i+1} and V_i start streaming (into the buffers of
  // tiles i - 1 and i - 2, which the last phase finished with)
#define PP_DMA(I, KN, VN)                                                                            \
  do {                                                                                               \
    if ((I) + 1 < Tmax) tile16_to_lds(K + kbase + (int64_t)((I) + 1) * d.k_step, d.k_row, KN, w8, l); \
    if ((I) < Tmax) tile16_to_lds(V + vbase + (int64_t)(I) * d.v_step, d.v_row, VN, w8, l);          \
  } while (0)
  // group 0 finishes at phase 2 ta, group 1 at 2 tb + 1; four phases per trip
  const int nph = 2 * Tmax + 2;
  // phase ends: a plain barrier after an even phase (nothing in LDS changes
  // hands there), a full one after an odd phase, when the tiles streamed at
  // the even phase must have landed
#define PP_SYNC_EVEN()                   \
  do {                                   \
    __builtin_amdgcn_sched_barrier(0);   \
    __builtin_amdgcn_s_barrier();        \
    __builtin_amdgcn_sched_barrier(0);   \
  } while (0)
#define PP_SYNC_ODD()                    \
  do {                                   \
    __builtin_amdgcn_sched_barrier(0);   \
    __builtin_amdgcn_s_waitcnt(0);       \
    __syncthreads();                     \
    __builtin_amdgcn_sched_barrier(0);   \
  } while (0)
  // each group's own phase sequence (a static M, V order, so S and P live in
  // registers only between their two phases); both run the same barriers
  if (g == 0) {
    for (int p = 0; p < nph; p += 4) {
      const int i = p >> 1;                           // tiles i (even) and i + 1
      PP_DMA(i, K1s, V0s);
      PP_M(i, K0s, V1s);
      PP_SYNC_EVEN();
      PP_V(i);
      PP_SYNC_ODD();
      PP_DMA(i + 1, K0s, V1s);
      PP_M(i + 1, K1s, V0s);
      PP_SYNC_EVEN();
      PP_V(i + 1);
      PP_SYNC_ODD();
    }
  } else {
    for (int p = 0; p < nph; p += 4) {
      const int i = p >> 1;
      PP_DMA(i, K1s, V0s);
      PP_V(i - 1);
      PP_SYNC_EVEN();
      PP_M(i, K0s, V1s);
      PP_SYNC_ODD();
      PP_DMA(i + 1, K0s, V1s);
      PP_V(i);
      PP_SYNC_EVEN();
      PP_M(i + 1, K1s, V0s);
      PP_SYNC_ODD();
    }
  }
#undef PP_SYNC_EVEN
#undef PP_SYNC_ODD
#undef PP_DMA
#undef PP_V
#undef PP_M
  if (lane < 0) return;
  if (T > 0) {
    const float fin = exp_f(__fsub_rn(mr, m));
    if (!__all(fin == 1.f)) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        o0[i] = __fmul_rn(o0[i], fin);
        o1[i] = __fmul_rn(o1[i], fin);
        o2[i] = __fmul_rn(o2[i], fin);
        o3[i] = __fmul_rn(o3[i], fin);
      }
      lsum = __fmul_rn(lsum, fin);
    }
  }
  if (h == 0) {
    ((float*)d.m_out)[lane * AT + row] = m;
    ((float*)d.l_out)[lane * AT + row] = lsum;
  }
  const int64_t ob = uni(((const int64_t*)d.o_base)[lane]) + (int64_t)row * d.o_row + 4 * h;
  // O = acc / l as acc * (1 / l): one correctly rounded reciprocal per row
  // instead of 64 IEEE divisions per lane (within 1.5 ulp of the quotient,
  // before the result's own rounding; l = 0, inf or NaN give the quotient's
  // inf / 0 / NaN as well)
  const float rl = __frcp_rn(lsum);
#define PP_EPI(o, dt)                                                                            \
  _Pragma("unroll") for (int gg = 0; gg < 4; ++gg) {                                             \
    const float q0 = __fmul_rn(o[4 * gg], rl), q1 = __fmul_rn(o[4 * gg + 1], rl);                \
    const float q2 = __fmul_rn(o[4 * gg + 2], rl), q3 = __fmul_rn(o[4 * gg + 3], rl);            \
    const int64_t e = ob + 32 * dt + 8 * gg;                                                     \
    if (d.o_dtype == KTIR_F32)                                                                   \
      *(float4*)((float*)d.o_ptr + e) = make_float4(q0, q1, q2, q3);                             \
    else if (d.o_dtype == KTIR_BF16)                                                             \
      *(uint2*)((uint16_t*)d.o_ptr + e) = make_uint2(cvt2<true>(q0, q1), cvt2<true>(q2, q3));     \
    else                                                                                         \
      *(uint2*)((uint16_t*)d.o_ptr + e) = make_uint2(cvt2<false>(q0, q1), cvt2<false>(q2, q3));   \
  }
  PP_EPI(o0, 0)
  PP_EPI(o1, 1)
  PP_EPI(o2, 2)
  PP_EPI(o3, 3)
#undef PP_EPI
}

// f16 copy of bf16 V: 8 elements per thread and step; *bad |= any value that
// is not finite or has |v| >= 65536 (bf16 magnitude bits >= 0x4780)
__global__ __launch_bounds__(256) void attn_v16(const uint16_t* src, uint16_t* dst, int64_t n8, int* bad) {
  int out = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
    const u32x4_t x = ((const KTIR_G(u32x4_t)*)src)[i];
    const uint32_t w[4] = {x[0], x[1], x[2], x[3]};
    uint32_t y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t m = w[k] & 0x7fff7fffu;
      out |= (int)(((m + 0x38803880u) & 0x80008000u) != 0);
      const f16x2_t h = __builtin_convertvector((f32x2_t{__uint_as_float(w[k] << 16), __uint_as_float(w[k] & 0xffff0000u)}),
                                                f16x2_t);
      y[k] = __builtin_bit_cast(uint32_t, h);
    }
    ((KTIR_G(u32x4_t)*)dst)[i] = u32x4_t{y[0], y[1], y[2], y[3]};
  }
  if (__any(out) && (threadIdx.x & 63) == 0) atomicOr(bad, 1);
}

__global__ void attn_v16_clear(int* bad) { *bad = 0; }

}  // namespace ktir

using namespace ktir;

extern "C" int ktir_launch_attention(const ktir_attn_t* d) {
  if (!d || d->M != AT || d->N != AT || d->D != AT)
    return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_attention: M = N = D = %d only", AT);
  if (d->dtype != KTIR_BF16 && d->dtype != KTIR_F16)
    return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_attention: bf16 or f16 operands");
  if ((d->q_ptr | d->k_ptr | d->v_ptr) & 15 || (d->q_row | d->k_row | d->v_row | d->k_step | d->v_step) & 7)
    return set_error(KTIR_E_ARG, "ktir_launch_attention: operands must be 16-byte aligned");
  if (d->o_ptr && (d->o_dtype != KTIR_F32 && d->o_dtype != KTIR_BF16 && d->o_dtype != KTIR_F16))
    return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_attention: output dtype %d", d->o_dtype);
  if (d->lanes == 0) return KTIR_OK;
  // predicate keep = pred(kpos, qpos) as a range test on kpos - qpos
  int lo = 0, hi = 0, inv = 0;
  switch (d->pred) {
    case KTIR_CMP_EQ: break;
    case KTIR_CMP_NE: inv = 1; break;
    case KTIR_CMP_SLT: case KTIR_CMP_ULTI: lo = INT_MIN; hi = -1; break;
    case KTIR_CMP_SLE: case KTIR_CMP_ULEI: lo = INT_MIN; hi = 0; break;
    case KTIR_CMP_SGT: case KTIR_CMP_UGTI: lo = 1; hi = INT_MAX; break;
    case KTIR_CMP_SGE: case KTIR_CMP_UGEI: lo = 0; hi = INT_MAX; break;
    default:
      if (d->causal) return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_attention: mask predicate %d", d->pred);
  }
  const dim3 grid((unsigned)d->lanes);
  // P rounded once to f16 only when the launch's one result is O = acc / l:
  // its error there is at most 2^-12 max|V| per element, while an
  // unnormalised acc would carry it l times over
  const bool norm = d->o_ptr && !d->acc_out;
  // the two-group kernel's one softmax form needs scale > 0 and, under a
  // mask, the fill value -inf; anything else runs attn_kernel
  const bool pp = norm && d->pairs && d->n_pairs > 0 && d->n_pairs < (int64_t)0x7fffffff && d->scale > 0.f &&
                  (!d->causal || d->neg == -__builtin_inff());
  const dim3 pgrid((unsigned)(pp ? d->n_pairs : 1));
  if (d->dtype == KTIR_BF16 && d->v16_ptr && norm) {
    if (!d->v16_flag || (d->v16_lo | d->v16_n) & 7 || d->v16_lo < 0 || d->v16_n <= 0 || (d->v16_ptr & 15))
      return set_error(KTIR_E_ARG, "ktir_launch_attention: bad f16 V copy (range %lld + %lld)",
                       (long long)d->v16_lo, (long long)d->v16_n);
    const int64_t n8 = d->v16_n / 8;
    const int64_t blocks = n8 / 256 + 1 < 16384 ? n8 / 256 + 1 : 16384;
    if (!d->v16_ready) {
      hipLaunchKernelGGL(attn_v16_clear, dim3(1), dim3(1), 0, stream(), (int*)d->v16_flag);
      hipLaunchKernelGGL(attn_v16, dim3((unsigned)blocks), dim3(256), 0, stream(),
                         (const uint16_t*)d->v_ptr + d->v16_lo, (uint16_t*)d->v16_ptr, n8, (int*)d->v16_flag);
    }
    if (pp)
      hipLaunchKernelGGL((attn_pp<true>), pgrid, dim3(512), 0, stream(), *d, lo, hi, inv);
    else
      hipLaunchKernelGGL((attn_kernel<true, true>), grid, dim3(256), 0, stream(), *d, lo, hi, inv);
    const dim3 fgrid((unsigned)(d->lanes < 512 ? d->lanes : 512));
    hipLaunchKernelGGL(attn_kernel_gated, fgrid, dim3(256), 0, stream(), *d, lo, hi, inv);
  } else if (d->dtype == KTIR_BF16) {
    hipLaunchKernelGGL((attn_kernel<true, false>), grid, dim3(256), 0, stream(), *d, lo, hi, inv);
  } else if (norm && pp) {
    hipLaunchKernelGGL((attn_pp<false>), pgrid, dim3(512), 0, stream(), *d, lo, hi, inv);
  } else if (norm) {
    hipLaunchKernelGGL((attn_kernel<false, true>), grid, dim3(256), 0, stream(), *d, lo, hi, inv);
  } else {
    hipLaunchKernelGGL((attn_kernel<false, false>), grid, dim3(256), 0, stream(), *d, lo, hi, inv);
  }
  KTIR_HIP_CHECK(hipGetLastError());
  return KTIR_OK;
}
