// Fused online-softmax attention loop (flash attention) on gfx950 MFMA.
//
// One workgroup per lane (a block of 128 query rows); wavefront w owns query
// rows 32w .. 32w+31.  Per KV tile j (128 keys):
//   S^T = K_j Q^T   v_mfma_f32_32x32x16 with A = K rows from LDS and
//                   B = Q^T fragments kept in registers, so the D layout puts
//                   one query row per lane (lanes l and l^32 share a row):
//                   lane l holds row l%32, keys 8g + 4h + t (h = l/32).
//   row max / row sum: 64 values in the lane + one swap with lane l^32.
//   O^T += V_j^T P^T  with A = V^T rows from LDS (V is staged transposed)
//                   and B = P^T fragments: the 8 consecutive keys a lane
//                   needs are 4 of its own values and 4 of lane l^32's.
// so O rows also live in lanes and the per-row rescale by alpha needs no
// communication.  Semantics follow the KTIR loop body (see ktir_hip.h):
// m' = max(m, rowmax S) (NaN-propagating like arith.maximumf),
// P = exp(S - m'), alpha = exp(m - m'), acc' = acc*alpha + P@V,
// l' = l*alpha + rowsum P, all in f32.
#include <climits>

#include "ktir_common.h"

namespace ktir {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int AT = 128;            // M = N = D
constexpr int LDP = AT + 8;        // padded LDS row (elements)

template <bool BF16>
__device__ __forceinline__ f32x16_t mfma_at(const uint4& a, const uint4& b, f32x16_t c) {
  if constexpr (BF16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c,
                                                  0, 0, 0);
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

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

__device__ __forceinline__ uint32_t half16(const uint4& v, int i) {
  const uint32_t w = i < 2 ? v.x : (i < 4 ? v.y : (i < 6 ? v.z : v.w));
  return (i & 1) ? (w >> 16) : (w & 0xffffu);
}

// arith.maximumf: NaN-propagating maximum (v_maximum3_f32 on gfx950)
__device__ __forceinline__ float fmax_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// e^x as 2^(x log2 e) on the hardware exp2 (v_exp_f32)
__device__ __forceinline__ float exp_f(float x) { return __builtin_amdgcn_exp2f(__fmul_rn(x, 1.44269504088896341f)); }

#define AT_S_LOOP(BODY)                     \
  _Pragma("unroll") for (int kt = 0; kt < 4; ++kt) { \
    _Pragma("unroll") for (int i = 0; i < 16; ++i) { BODY; } }

template <bool BF16>
// The position mask keeps score (row, key) iff ((lo <= kpos - qpos <= hi) != inv).
__global__ __launch_bounds__(256, 2) void attn_kernel(const ktir_attn_t d, int mlo, int mhi, int minv) {
  __shared__ __align__(16) uint16_t Ks[AT * LDP];   // K tile, [key][d]
  __shared__ __align__(16) uint16_t Vt[AT * LDP];   // V tile transposed, [d][key]
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, h = l >> 5, r32 = l & 31;
  const int64_t lane = d.order ? ((const int32_t*)d.order)[blockIdx.x] : blockIdx.x;
  const int T = ((const int32_t*)d.trips)[lane];
  const uint16_t* Q = (const uint16_t*)d.q_ptr;
  const uint16_t* K = (const uint16_t*)d.k_ptr;
  const uint16_t* V = (const uint16_t*)d.v_ptr;
  const int row = w * 32 + r32;                      // this lane's query row
  // Q^T fragments: for d-step s, Q[row][16 s + 8 h .. + 8]
  uint4 qf[8];
  if (T > 0) {
    const uint16_t* qr = Q + ((const int64_t*)d.q_base)[lane] + (int64_t)row * d.q_row + 8 * h;
#pragma unroll
    for (int s = 0; s < 8; ++s) qf[s] = *(const uint4*)(qr + 16 * s);
  }
  const int64_t kb0 = ((const int64_t*)d.k_base)[lane], vb0 = ((const int64_t*)d.v_base)[lane];
  const int64_t qpos = ((const int64_t*)d.qpos0)[lane] + row;
  const int64_t kpos00 = ((const int64_t*)d.kpos0)[lane];
  const f32x16_t z16 = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  f32x16_t o0 = z16, o1 = z16, o2 = z16, o3 = z16;   // O^T tiles: d = 32 dt + 8g + 4h + t, row r32
  float m = -__builtin_inff(), lsum = 0.f;
  // staging assignment
  for (int j = 0; j < T; ++j) {
    const int64_t kb = kb0 + (int64_t)j * d.k_step, vb = vb0 + (int64_t)j * d.v_step;
    __syncthreads();   // the previous iteration has finished reading Ks / Vt
    // K: 128 keys x 16 chunks of 8 elements, 8 chunks per thread, row-major into Ks
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = tid + 256 * i, key = c >> 4, dc = (c & 15) * 8;
      *(uint4*)&Ks[key * LDP + dc] = *(const uint4*)(K + kb + (int64_t)key * d.k_row + dc);
    }
    // V transposed: units of 4 keys x 8 d, 2 per thread.  Consecutive lanes
    // take consecutive key quads, so each transposed 8-byte LDS write of a
    // wave covers 256 contiguous bytes per 32 lanes (no bank conflicts).
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int u = tid + 256 * i, kq = (u & 31) * 4, dc = (u >> 5) * 8;
      const uint16_t* vr = V + vb + (int64_t)kq * d.v_row + dc;
      const uint4 v0 = *(const uint4*)(vr), v1 = *(const uint4*)(vr + d.v_row);
      const uint4 v2 = *(const uint4*)(vr + 2 * d.v_row), v3 = *(const uint4*)(vr + 3 * d.v_row);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        *(uint2*)&Vt[(dc + e) * LDP + kq] =
            make_uint2(half16(v0, e) | (half16(v1, e) << 16), half16(v2, e) | (half16(v3, e) << 16));
    }
    __syncthreads();
    // S^T = K Q^T: 4 key tiles x 8 d-steps
    f32x16_t s0 = z16, s1 = z16, s2 = z16, s3 = z16;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int dofs = 16 * s + 8 * h;
      s0 = mfma_at<BF16>(*(const uint4*)&Ks[(0 * 32 + r32) * LDP + dofs], qf[s], s0);
      s1 = mfma_at<BF16>(*(const uint4*)&Ks[(1 * 32 + r32) * LDP + dofs], qf[s], s1);
      s2 = mfma_at<BF16>(*(const uint4*)&Ks[(2 * 32 + r32) * LDP + dofs], qf[s], s2);
      s3 = mfma_at<BF16>(*(const uint4*)&Ks[(3 * 32 + r32) * LDP + dofs], qf[s], s3);
    }
    // scale, causal mask; lane value (kt, i) is key kt*32 + 8(i/4) + 4h + i%4 of row `row`
    const int64_t kpos_j = kpos00 + (int64_t)j * d.kpos_step;
    float sv[4][16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      sv[0][i] = __fmul_rn(d.scale, s0[i]);
      sv[1][i] = __fmul_rn(d.scale, s1[i]);
      sv[2][i] = __fmul_rn(d.scale, s2[i]);
      sv[3][i] = __fmul_rn(d.scale, s3[i]);
    }
    if (d.causal) {
      // kpos - qpos of this lane's key 0; its keys add 0 .. 127 (the 4h lane offset included below)
      const int dbase = (int)(kpos_j - qpos);
      const bool all_keep = minv ? (dbase + 127 < mlo || dbase > mhi) : (dbase >= mlo && dbase + 127 <= mhi);
      if (!__all(all_keep)) {
        AT_S_LOOP({
          const int df = dbase + kt * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
          if ((df >= mlo && df <= mhi) == (bool)minv) sv[kt][i] = d.neg;
        })
      }
    }
    float rm = -__builtin_inff();
    AT_S_LOOP(rm = fmax_nan(rm, sv[kt][i]))
    rm = fmax_nan(rm, __shfl_xor(rm, 32));
    const float mn = fmax_nan(m, rm);
    float ls = 0.f;
    AT_S_LOOP({
      sv[kt][i] = exp_f(__fsub_rn(sv[kt][i], mn));
      ls = __fadd_rn(ls, sv[kt][i]);
    })
    ls = __fadd_rn(ls, __shfl_xor(ls, 32));
    const float alpha = exp_f(__fsub_rn(m, mn));
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      o0[i] = __fmul_rn(o0[i], alpha);
      o1[i] = __fmul_rn(o1[i], alpha);
      o2[i] = __fmul_rn(o2[i], alpha);
      o3[i] = __fmul_rn(o3[i], alpha);
    }
    lsum = __fadd_rn(__fmul_rn(lsum, alpha), ls);
    m = mn;
    // O^T += V^T P^T over 8 key-steps of 16 keys
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      // lane half h owns 4-key group g = 2 (ks & 1) + h of key tile ks / 2 and sends the other one
      const int kt = ks >> 1, g0 = 2 * (ks & 1);
      uint32_t ah0, ah1, al0, al1, bh0, bh1, bl0, bl1;
      split4<BF16>(&sv[kt][4 * g0], ah0, ah1, al0, al1);
      split4<BF16>(&sv[kt][4 * g0 + 4], bh0, bh1, bl0, bl1);
      const uint32_t oh0 = h ? bh0 : ah0, oh1 = h ? bh1 : ah1, ol0 = h ? bl0 : al0, ol1 = h ? bl1 : al1;
      const uint32_t rh0 = __shfl_xor(h ? ah0 : bh0, 32), rh1 = __shfl_xor(h ? ah1 : bh1, 32);
      const uint32_t rl0 = __shfl_xor(h ? al0 : bl0, 32), rl1 = __shfl_xor(h ? al1 : bl1, 32);
      // keys 16 ks + 8 h + [0..3] come from lane half 0, [4..7] from half 1
      const uint4 ph = h == 0 ? make_uint4(oh0, oh1, rh0, rh1) : make_uint4(rh0, rh1, oh0, oh1);
      const uint4 pl = h == 0 ? make_uint4(ol0, ol1, rl0, rl1) : make_uint4(rl0, rl1, ol0, ol1);
      const int kofs = 16 * ks + 8 * h;
      const uint4 a0 = *(const uint4*)&Vt[(0 * 32 + r32) * LDP + kofs];
      const uint4 a1 = *(const uint4*)&Vt[(1 * 32 + r32) * LDP + kofs];
      const uint4 a2 = *(const uint4*)&Vt[(2 * 32 + r32) * LDP + kofs];
      const uint4 a3 = *(const uint4*)&Vt[(3 * 32 + r32) * LDP + kofs];
      o0 = mfma_at<BF16>(a0, ph, o0);
      o1 = mfma_at<BF16>(a1, ph, o1);
      o2 = mfma_at<BF16>(a2, ph, o2);
      o3 = mfma_at<BF16>(a3, ph, o3);
      o0 = mfma_at<BF16>(a0, pl, o0);
      o1 = mfma_at<BF16>(a1, pl, o1);
      o2 = mfma_at<BF16>(a2, pl, o2);
      o3 = mfma_at<BF16>(a3, pl, o3);
    }
  }
  // final state
  if (h == 0) {
    ((float*)d.m_out)[lane * AT + row] = m;
    ((float*)d.l_out)[lane * AT + row] = lsum;
  }
  float* orow = (float*)d.acc_out + (lane * AT + row) * AT + 4 * h;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    *(float4*)(orow + 0 * 32 + 8 * g) = make_float4(o0[4 * g], o0[4 * g + 1], o0[4 * g + 2], o0[4 * g + 3]);
    *(float4*)(orow + 1 * 32 + 8 * g) = make_float4(o1[4 * g], o1[4 * g + 1], o1[4 * g + 2], o1[4 * g + 3]);
    *(float4*)(orow + 2 * 32 + 8 * g) = make_float4(o2[4 * g], o2[4 * g + 1], o2[4 * g + 2], o2[4 * g + 3]);
    *(float4*)(orow + 3 * 32 + 8 * g) = make_float4(o3[4 * g], o3[4 * g + 1], o3[4 * g + 2], o3[4 * g + 3]);
  }
}

}  // namespace ktir

using namespace ktir;

extern "C" int ktir_launch_attention(const ktir_attn_t* d) {
  if (!d || d->M != AT || d->N != AT || d->D != AT)
    return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_attention: M = N = D = %d only", AT);
  if (d->dtype != KTIR_BF16 && d->dtype != KTIR_F16)
    return set_error(KTIR_E_UNSUPPORTED, "ktir_launch_attention: bf16 or f16 operands");
  if ((d->q_ptr | d->k_ptr | d->v_ptr) & 15 || (d->q_row | d->k_row | d->v_row | d->k_step | d->v_step) & 7)
    return set_error(KTIR_E_ARG, "ktir_launch_attention: operands must be 16-byte aligned");
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
  if (d->dtype == KTIR_BF16)
    hipLaunchKernelGGL((attn_kernel<true>), dim3((unsigned)d->lanes), dim3(256), 0, stream(), *d, lo, hi, inv);
  else
    hipLaunchKernelGGL((attn_kernel<false>), dim3((unsigned)d->lanes), dim3(256), 0, stream(), *d, lo, hi, inv);
  KTIR_HIP_CHECK(hipGetLastError());
  return KTIR_OK;
}
