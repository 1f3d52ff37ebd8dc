// gfx950 MFMA matmul tiles: f16 / bf16 operands, f32 accumulation.
//
// One workgroup (4 wavefronts) computes one 128x128 output tile of one lane;
// each wavefront owns a 64x64 quadrant made of 2x2 v_mfma_f32_32x32x16
// tiles.  The K dimension (the fused scf.for steps times the tile's own K)
// advances 64 at a time through double-buffered LDS: A is staged row-major,
// B transposed (k contiguous) so both MFMA operands are 16-byte LDS reads.
// Global loads for step t+1 are issued before the MFMAs of step t.
// Block ids are remapped so consecutive tiles (which share A rows) land on
// the same XCD and its L2.
//
// Operand layout of v_mfma_f32_32x32x16_{f16,bf16} (64 lanes):
//   A (32 x 16): lane l holds row l%32, k = 8*(l/32) .. +8
//   B (16 x 32): lane l holds col l%32, k = 8*(l/32) .. +8
//   D (32 x 32): lane l holds col l%32, rows 8*(i/4) + 4*(l/32) + i%4, i < 16
#include "ktir_common.h"

namespace ktir {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bfx8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int MT = 128, NT = 128, BK = 64, LDK = BK + 8;   // LDS row: 72 halfs (pad breaks bank conflicts)

// 16-bit element i (0..7) of a 128-bit register group
__device__ __forceinline__ uint32_t half_of(const uint4& v, int i) {
  const uint32_t w = i < 2 ? v.x : (i < 4 ? v.y : (i < 6 ? v.z : v.w));
  return (i & 1) ? (w >> 16) : (w & 0xffffu);
}

template <bool BF16>
__device__ __forceinline__ f32x16 mfma32(const uint4& a, const uint4& b, f32x16 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bfx8, a), __builtin_bit_cast(bfx8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0, 0, 0);
  }
}

// one result element of dtype DT (f32, f16 or bf16, round to nearest even)
template <int DT>
__device__ __forceinline__ void mm_put(uint64_t ptr, int64_t off, float v) {
  if constexpr (DT == KTIR_F32)
    ((KTIR_G(float)*)ptr)[off] = v;
  else if constexpr (DT == KTIR_F16)
    ((KTIR_G(_Float16)*)ptr)[off] = (_Float16)v;
  else
    ((KTIR_G(uint16_t)*)ptr)[off] = (uint16_t)(__float_as_uint(round_bf16(v)) >> 16);
}

// a wavefront's 64 x 64 quadrant as 2 x 2 MFMA tiles, starting at element
// offset o (lane l: column l % 32, rows 8 (e / 4) + 4 (l / 32) + e % 4 of
// each tile, the lane's part of the row already in o), each element acc + z
template <int DT>
__device__ __forceinline__ void mm_quadrant_out(uint64_t ptr, int64_t o, int64_t cs, const f32x16& a00,
                                                const f32x16& a01, const f32x16& a10, const f32x16& a11, float z) {
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int64_t r = (8 * (e >> 2) + (e & 3)) * cs;
    mm_put<DT>(ptr, o + r, __fadd_rn(a00[e], z));
    mm_put<DT>(ptr, o + r + 32, __fadd_rn(a01[e], z));
    mm_put<DT>(ptr, o + r + 32 * cs, __fadd_rn(a10[e], z));
    mm_put<DT>(ptr, o + r + 32 * cs + 32, __fadd_rn(a11[e], z));
  }
}

// Epilogue of a 128 x 128 tile (wavefront (wr, wc) holds the 64 x 64
// quadrant as 2 x 2 MFMA tiles): round the product to the operand dtype of
// the KTIR matmul, then accumulate into the outs tile (the reference's two
// roundings).
__device__ __forceinline__ void mm_epilogue(const ktir_mm_t& d, int64_t ln, int64_t m0, int64_t n0, int wr, int wc,
                                            int lane, const f32x16& acc00, const f32x16& acc01, const f32x16& acc10,
                                            const f32x16& acc11) {
  const int64_t cbase = lane_offset(d.c, ln);
  if ((d.c.dtype == KTIR_F32 || d.c.dtype == KTIR_F16 || d.c.dtype == KTIR_BF16) && d.round_dt == KTIR_F32 &&
      d.accumulate != 1 && d.c.strides[1] == 1) {
    // outs absent or a zero splat (accumulate == 2: x + 0.0), rounded to the result dtype
    const int64_t cs = d.c.strides[0];
    const float z = d.accumulate == 2 ? 0.f : -0.f;
    const int64_t r0 = m0 + wr * 64 + 4 * (lane >> 5), c0 = n0 + wc * 64 + (lane & 31);
    if (d.c.dtype == KTIR_F32)
      mm_quadrant_out<KTIR_F32>(d.c.ptr, cbase + r0 * cs + c0, cs, acc00, acc01, acc10, acc11, z);
    else if (d.c.dtype == KTIR_F16)
      mm_quadrant_out<KTIR_F16>(d.c.ptr, cbase + r0 * cs + c0, cs, acc00, acc01, acc10, acc11, z);
    else
      mm_quadrant_out<KTIR_BF16>(d.c.ptr, cbase + r0 * cs + c0, cs, acc00, acc01, acc10, acc11, z);
    return;
  }
  const int64_t c0base = d.accumulate == 1 ? lane_offset(d.c0, ln) : 0;
  for (int q = 0; q < 4; ++q) {
    const int i = q >> 1, j = q & 1;
    const f32x16 a = q == 0 ? acc00 : (q == 1 ? acc01 : (q == 2 ? acc10 : acc11));
    for (int e = 0; e < 16; ++e) {
        const int64_t row = m0 + wr * 64 + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int64_t col = n0 + wc * 64 + j * 32 + (lane & 31);
        float v = round_to(a[e], d.round_dt);
        if (d.accumulate == 1) {
          const int64_t e0 = c0base + row * d.c0.strides[0] + col * d.c0.strides[1];
          v = round_to(__fadd_rn(load_elem(d.c0.ptr, e0, d.c0.dtype), v), d.c.dtype);
        } else if (d.accumulate == 2) {
          v = round_to(__fadd_rn(0.f, v), d.c.dtype);
        }
        store_elem(d.c.ptr, cbase + row * d.c.strides[0] + col * d.c.strides[1], d.c.dtype, v);
    }
  }
}

template <bool BF16>
__global__ __launch_bounds__(256) void mm_mfma(const ktir_mm_t d, int64_t tiles_m, int64_t tiles_n) {
  __shared__ __align__(16) uint16_t As[2][MT * LDK];
  __shared__ __align__(16) uint16_t Bs[2][NT * LDK];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int wr = wave >> 1, wc = wave & 1;
  const int64_t nblk = gridDim.x;
  int64_t bid = blockIdx.x;
  if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
  const int64_t per_lane = tiles_m * tiles_n;
  const int64_t ln = bid / per_lane, t = bid - ln * per_lane;
  const int64_t m0 = (t / tiles_n) * MT, n0 = (t % tiles_n) * NT;
  const uint16_t* A = (const uint16_t*)d.a.ptr;
  const uint16_t* B = (const uint16_t*)d.b.ptr;
  const int64_t a_row = d.a.strides[0], b_row = d.b.strides[0];
  const int64_t abase = lane_offset(d.a, ln) + m0 * a_row;
  const int64_t bbase = lane_offset(d.b, ln) + n0;
  const int64_t kt_per_step = d.K / BK;
  const int64_t nk = d.ksteps * kt_per_step;
  // global -> register assignment
  const int a_r = tid >> 3, a_k = (tid & 7) * 8;      // A rows a_r + 32 j, k-group a_k
  const int b_k = (tid >> 4) * 4, b_n = (tid & 15) * 8; // B rows b_k + r, cols b_n .. +8
  uint4 ra0, ra1, ra2, ra3, rb0, rb1, rb2, rb3;
#define GLOAD(kt)                                                                   \
  do {                                                                              \
    const int64_t s_ = (kt) / kt_per_step, kk0_ = ((kt) - s_ * kt_per_step) * BK;     \
    const uint16_t* pa = A + abase + s_ * d.a_kstep + kk0_ + a_k + (int64_t)a_r * a_row; \
    ra0 = *(const uint4*)(pa);                                                      \
    ra1 = *(const uint4*)(pa + 32 * a_row);                                         \
    ra2 = *(const uint4*)(pa + 64 * a_row);                                         \
    ra3 = *(const uint4*)(pa + 96 * a_row);                                         \
    const uint16_t* pb = B + bbase + s_ * d.b_kstep + (kk0_ + b_k) * b_row + b_n;   \
    rb0 = *(const uint4*)(pb);                                                      \
    rb1 = *(const uint4*)(pb + b_row);                                              \
    rb2 = *(const uint4*)(pb + 2 * b_row);                                          \
    rb3 = *(const uint4*)(pb + 3 * b_row);                                          \
  } while (0)
#define SWRITE(buf)                                                                  \
  do {                                                                               \
    uint16_t* as = &As[buf][a_r * LDK + a_k];                                        \
    *(uint4*)(as) = ra0;                                                             \
    *(uint4*)(as + 32 * LDK) = ra1;                                                  \
    *(uint4*)(as + 64 * LDK) = ra2;                                                  \
    *(uint4*)(as + 96 * LDK) = ra3;                                                  \
    _Pragma("unroll") for (int i = 0; i < 8; ++i) {                                  \
      uint2 v = make_uint2(half_of(rb0, i) | (half_of(rb1, i) << 16), half_of(rb2, i) | (half_of(rb3, i) << 16)); \
      *(uint2*)&Bs[buf][(b_n + i) * LDK + b_k] = v;                                  \
    }                                                                                \
  } while (0)
  const f32x16 zero16 = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  f32x16 acc00 = zero16, acc01 = zero16, acc10 = zero16, acc11 = zero16;
  GLOAD(0);
  SWRITE(0);
  __syncthreads();
  const int frag_r = lane & 31, frag_k = (lane >> 5) * 8;
  for (int64_t kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) GLOAD(kt + 1);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      const uint4 a0 = *(const uint4*)&As[cur][(wr * 64 + frag_r) * LDK + kk + frag_k];
      const uint4 a1 = *(const uint4*)&As[cur][(wr * 64 + 32 + frag_r) * LDK + kk + frag_k];
      const uint4 b0 = *(const uint4*)&Bs[cur][(wc * 64 + frag_r) * LDK + kk + frag_k];
      const uint4 b1 = *(const uint4*)&Bs[cur][(wc * 64 + 32 + frag_r) * LDK + kk + frag_k];
      acc00 = mfma32<BF16>(a0, b0, acc00);
      acc01 = mfma32<BF16>(a0, b1, acc01);
      acc10 = mfma32<BF16>(a1, b0, acc10);
      acc11 = mfma32<BF16>(a1, b1, acc11);
    }
    if (kt + 1 < nk) SWRITE(cur ^ 1);
    __syncthreads();
  }
#undef GLOAD
#undef SWRITE
  mm_epilogue(d, ln, m0, n0, wr, wc, lane, acc00, acc01, acc10, acc11);
}

// ---- 128 x 128 x 64 tiles staged by LDS DMA -------------------------------------
//
// The same tile and wavefront split as mm_mfma, with both operands moving
// HBM -> LDS by buffer_load ... lds (no registers, no transposition on the
// way in), double-buffered in four distinct LDS arrays so the DMA of step
// t + 1 overlaps the MFMAs of step t:
//   A tile: 128 rows x 64 k, 128-byte rows, 16-byte chunk c of row r at slot
//           c ^ (r % 8) ^ ((r / 8) % 2); A fragments are ds_read_b128.
//   B tile: 64 k-rows x 128 columns, row-major as in HBM, 256-byte rows with
//           chunk c at slot c ^ swz16(r); B fragments (column l % 32, k
//           8 (l / 32) .. + 8) are two ds_read_b64_tr_b16 transposing reads.
// Both swizzles make every read phase touch distinct banks (with 32 or 64
// LDS banks alike).
typedef short mm_s16x4 __attribute__((ext_vector_type(4)));

// slot permutation of the 16 chunks of a 256-byte LDS row r (an XOR of row
// bits; conflict-free for ds_read_b64_tr_b16 column reads and ds_read_b128
// row reads)
__device__ __forceinline__ int swz16(int r) {
  return ((r & 1) ? 4 : 0) ^ ((r & 2) ? 10 : 0) ^ ((r & 4) ? 1 : 0) ^ ((r & 8) ? 8 : 0);
}

__device__ __forceinline__ int swz_a(int r) { return (r & 7) ^ ((r >> 3) & 1); }

__device__ __forceinline__ uint2 mm_tr16(const uint16_t* p) {
  const mm_s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) mm_s16x4*)p);
  return __builtin_bit_cast(uint2, v);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t mm_rsrc(const uint16_t* base, int64_t hi_elems) {
  int64_t bytes = hi_elems * 2;
  if (bytes < 0) bytes = 0;
  if (bytes > 0xffffffffll) bytes = 0xffffffffll;
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)(uint32_t)bytes, 0x00020000);
}

struct MmStage {
  __amdgpu_buffer_rsrc_t ra, rb;
  uint32_t ao0, ao1;            // lane byte offsets of A blocks (even / odd)
  uint32_t bo0, bo1, bo2, bo3;  // lane byte offsets of B blocks b % 4
  int64_t a_row, b_row;
};

// wave w's share of step (koff_a, koff_b): A rows 32 w .. + 32 (4 blocks of 8
// rows), B k-rows 16 w .. + 16 (4 blocks of 4 rows)
__device__ __forceinline__ void mm_stage(const MmStage& g, uint16_t* as, uint16_t* bs, int w, int64_t koff_a,
                                         int64_t koff_b) {
#pragma unroll
  for (int b = 0; b < 4; ++b)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(g.ra, (__attribute__((address_space(3))) void*)(as + 64 * (32 * w + 8 * b)),
                                             16, (b & 1) ? g.ao1 : g.ao0, (int)((8 * b * g.a_row + koff_a) * 2), 0, 0);
#pragma unroll
  for (int b = 0; b < 4; ++b)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(g.rb, (__attribute__((address_space(3))) void*)(bs + 128 * (16 * w + 4 * b)),
                                             16, b == 0 ? g.bo0 : (b == 1 ? g.bo1 : (b == 2 ? g.bo2 : g.bo3)),
                                             (int)((4 * b * g.b_row + koff_b) * 2), 0, 0);
}

struct MmAcc {
  f32x16 c00, c01, c10, c11;
};

template <bool BF16>
__device__ __forceinline__ void mm_step(MmAcc& acc, const uint16_t* as, const uint16_t* bs, int wr, int wc, int r32,
                                        int h, const int (&b_off)[2][2]) {
#pragma unroll
  for (int kk = 0; kk < 4; ++kk) {
    const int ar0 = wr * 64 + r32, ar1 = ar0 + 32;
    const int ch = 2 * kk + h;
    const uint4 a0 = *(const uint4*)&as[ar0 * 64 + 8 * (ch ^ swz_a(ar0))];
    const uint4 a1 = *(const uint4*)&as[ar1 * 64 + 8 * (ch ^ swz_a(ar1))];
    const uint16_t* bt = bs + 16 * kk * 128;
    uint4 b[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint2 lo = mm_tr16(bt + b_off[0][j]), hi = mm_tr16(bt + b_off[1][j]);
      b[j] = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
    acc.c00 = mfma32<BF16>(a0, b[0], acc.c00);
    acc.c01 = mfma32<BF16>(a0, b[1], acc.c01);
    acc.c10 = mfma32<BF16>(a1, b[0], acc.c10);
    acc.c11 = mfma32<BF16>(a1, b[1], acc.c11);
  }
}

template <bool BF16>
__global__ __launch_bounds__(256, 2) void mm_mfma_dma(const ktir_mm_t d, int64_t tiles_m, int64_t tiles_n) {
  __shared__ __align__(16) uint16_t As0[MT * BK];
  __shared__ __align__(16) uint16_t As1[MT * BK];
  __shared__ __align__(16) uint16_t Bs0[BK * NT];
  __shared__ __align__(16) uint16_t Bs1[BK * NT];
  const int tid = threadIdx.x, l = tid & 63, h = l >> 5, r32 = l & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = w >> 1, wc = w & 1;
  const int64_t nblk = gridDim.x;
  int64_t bid = blockIdx.x;
  if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
  const int64_t per_lane = tiles_m * tiles_n;
  const int64_t ln = bid / per_lane, t = bid - ln * per_lane;
  const int64_t m0 = (t / tiles_n) * MT, n0 = (t % tiles_n) * NT;
  const int64_t a_row = d.a.strides[0], b_row = d.b.strides[0];
  const int64_t abase = uni(lane_offset(d.a, ln)) + m0 * a_row;
  const int64_t bbase = uni(lane_offset(d.b, ln)) + n0;
  MmStage g;
  const int64_t a0w = abase + 32 * w * a_row, b0w = bbase + 16 * w * b_row;
  g.ra = mm_rsrc((const uint16_t*)d.a.ptr + a0w, d.a.hi - a0w);
  g.rb = mm_rsrc((const uint16_t*)d.b.ptr + b0w, d.b.hi - b0w);
  g.a_row = a_row;
  g.b_row = b_row;
  // block b of A: rows 8 b + l / 8 (row % 16 = 8 (b % 2) + l / 8), slot l % 8;
  // block b of B: k-rows 4 b + l / 16 (row % 16 = 4 b + l / 16), slot l % 16
  g.ao0 = (uint32_t)(((l >> 3) * a_row + 8 * ((l & 7) ^ swz_a(l >> 3))) * 2);
  g.ao1 = (uint32_t)(((l >> 3) * a_row + 8 * ((l & 7) ^ swz_a(8 + (l >> 3)))) * 2);
  g.bo0 = (uint32_t)(((l >> 4) * b_row + 8 * ((l & 15) ^ swz16(l >> 4))) * 2);
  g.bo1 = (uint32_t)(((l >> 4) * b_row + 8 * ((l & 15) ^ swz16(4 + (l >> 4)))) * 2);
  g.bo2 = (uint32_t)(((l >> 4) * b_row + 8 * ((l & 15) ^ swz16(8 + (l >> 4)))) * 2);
  g.bo3 = (uint32_t)(((l >> 4) * b_row + 8 * ((l & 15) ^ swz16(12 + (l >> 4)))) * 2);
  // B fragment offsets inside a 16-row step: member tj of 16-lane group tg
  // reads k-row 8 (tg / 2) + tj / 4 (+ 4), columns 16 (tg % 2) + 4 (tj % 4)
  // of the 32-column group 2 wc + j
  const int tg = l >> 4, tj = l & 15;
  const int br0 = 8 * (tg >> 1) + (tj >> 2);
  const int bc = 2 * (tg & 1) + ((tj >> 1) & 1), bin = 4 * (tj & 1);
  int b_off[2][2];
#pragma unroll
  for (int hi = 0; hi < 2; ++hi)
#pragma unroll
    for (int j = 0; j < 2; ++j)
      b_off[hi][j] = (br0 + 4 * hi) * NT + 8 * ((4 * (2 * wc + j) + bc) ^ swz16(br0 + 4 * hi)) + bin;
  const int64_t kt_per_step = d.K / BK;
  const int64_t nk = d.ksteps * kt_per_step;
  const f32x16 zero16 = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  MmAcc acc{zero16, zero16, zero16, zero16};
  // k offsets (elements) of the staged step for A and B
  int64_t s_ = 0, kk0 = 0;
  int64_t ka = 0, kb = 0;
  mm_stage(g, As0, Bs0, w, ka, kb);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; kt += 2) {
    // even step from buffers 0 while step kt + 1 streams into buffers 1
    kk0 += BK;
    if (kk0 == kt_per_step * BK) { kk0 = 0; ++s_; }
    const bool m1 = kt + 1 < nk;
    if (m1) {
      ka = s_ * d.a_kstep + kk0;
      kb = s_ * d.b_kstep + kk0 * b_row;
      mm_stage(g, As1, Bs1, w, ka, kb);
    }
    mm_step<BF16>(acc, As0, Bs0, wr, wc, r32, h, b_off);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (!m1) break;
    kk0 += BK;
    if (kk0 == kt_per_step * BK) { kk0 = 0; ++s_; }
    const bool m2 = kt + 2 < nk;
    if (m2) {
      ka = s_ * d.a_kstep + kk0;
      kb = s_ * d.b_kstep + kk0 * b_row;
      mm_stage(g, As0, Bs0, w, ka, kb);
    }
    mm_step<BF16>(acc, As1, Bs1, wr, wc, r32, h, b_off);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  mm_epilogue(d, ln, m0, n0, wr, wc, l, acc.c00, acc.c01, acc.c10, acc.c11);
}

// ---- 256 x 256 blocks of four lanes ------------------------------------------------
//
// One workgroup computes a quad of lanes (a 256 x 256 block; the host checks
// the lanes are adjacent): wavefront (wr, wc) computes lane quad[2 wr + wc]'s
// whole 128 x 128 tile as 4 x 4 MFMA tiles (the accumulators live in AGPRs),
// so every byte staged in LDS feeds twice the MFMA work of a 128 x 128 tile
// and a 64-deep k step is 2048 MFMA cycles per wavefront, enough to cover the
// next step's DMA.  A stage holds four 16 KB sub-tiles, each staged by one
// wavefront: A top (rows of the top lanes), A bottom, B left, B right, in the
// layouts of mm_mfma_dma (A: chunk c of row r at c ^ swz_a(r); B: row-major,
// chunk c at c ^ swz16(r)); two stages double-buffered in two LDS arrays.
// Launched for an f32 result without an accumulator input (the K-loop form).
constexpr int QT = MT * BK;                     // halfs per sub-tile (16 KB)

// fragments of one 16-deep slice: A rows 32 i + r32 (chunk 2 kk + h), B
// columns 32 j + l % 32 (two transposing reads each)
__device__ __forceinline__ void q256_frags(const uint16_t* as, const uint16_t* bs, int kk, int r32, int h,
                                           const int (&b_off)[2][4], uint4 (&a)[4], uint4 (&b)[4]) {
  const int ch = 2 * kk + h;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ar = 32 * i + r32;
    a[i] = *(const uint4*)&as[ar * BK + 8 * (ch ^ swz_a(ar))];
  }
  const uint16_t* bt = bs + 16 * kk * NT;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint2 lo = mm_tr16(bt + b_off[0][j]), hi = mm_tr16(bt + b_off[1][j]);
    b[j] = make_uint4(lo.x, lo.y, hi.x, hi.y);
  }
}

#define Q_MFMA16(A, B)                                                                         \
  _Pragma("unroll") for (int i = 0; i < 4; ++i)                                                \
    _Pragma("unroll") for (int j = 0; j < 4; ++j) acc[i][j] = mfma32<BF16>(A[i], B[j], acc[i][j]);

// slices 0..2 of one 64-deep k step (slice 0's fragments already in a0/b0):
// each slice's 16 MFMAs run with the next slice's 12 fragment reads between
// them; slice 3's fragments are left in a1/b1
template <bool BF16>
__device__ __forceinline__ void q256_slices012(f32x16 (&acc)[4][4], const uint16_t* as, const uint16_t* bs, int r32,
                                               int h, const int (&b_off)[2][4], uint4 (&a0)[4], uint4 (&b0)[4],
                                               uint4 (&a1)[4], uint4 (&b1)[4]) {
  q256_frags(as, bs, 1, r32, h, b_off, a1, b1);
  Q_MFMA16(a0, b0)
  q256_frags(as, bs, 2, r32, h, b_off, a0, b0);
  Q_MFMA16(a1, b1)
  q256_frags(as, bs, 3, r32, h, b_off, a1, b1);
  Q_MFMA16(a0, b0)
#pragma unroll
  for (int s = 0; s < 3; ++s) {
#pragma unroll
    for (int x = 0; x < 12; ++x) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
  }
}

// a wavefront's 128 x 128 result (4 x 4 MFMA tiles; lane l holds column
// 32 j + l % 32, rows 32 i + 8 (e / 4) + 4 h + e % 4), each element acc + z
template <int DT>
__device__ __forceinline__ void q256_out(uint64_t ptr, int64_t cb, int64_t cs, int h, int r32,
                                         const f32x16 (&acc)[4][4], float z) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e)
        mm_put<DT>(ptr, cb + (32 * i + 8 * (e >> 2) + 4 * h + (e & 3)) * cs + 32 * j + r32, __fadd_rn(acc[i][j][e], z));
}

// The same 128 x 128 result rounded to a 16-bit dtype, staged through this
// wavefront's 32 KB of LDS (row-major, 128 halfs a row) and written as
// 16-byte row pieces: 32 stores per lane instead of 256 two-byte ones.
// Needs 16-byte aligned result rows (the caller checks).
typedef uint32_t q256_u4 __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ void q256_out16(uint16_t* lds, uint64_t ptr, int64_t cb, int64_t cs, int h, int r32, int l,
                                           const f32x16 (&acc)[4][4], float z) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float v = __fadd_rn(acc[i][j][e], z);
        const uint16_t b = DT == KTIR_F16 ? __builtin_bit_cast(uint16_t, (_Float16)v)
                                          : (uint16_t)(__float_as_uint(round_bf16(v)) >> 16);
        lds[(32 * i + 8 * (e >> 2) + 4 * h + (e & 3)) * 128 + 32 * j + r32] = b;
      }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  KTIR_G(uint16_t)* c = (KTIR_G(uint16_t)*)ptr + cb;
#pragma unroll 4
  for (int it = 0; it < 32; ++it) {
    const int row = 4 * it + (l >> 4), col = 8 * (l & 15);
    const q256_u4 v = *(const q256_u4*)&lds[row * 128 + col];
    __builtin_nontemporal_store(v, (KTIR_G(q256_u4)*)(c + row * cs + col));
  }
}

template <bool BF16>
__global__ __launch_bounds__(256, 1) void mm_mfma_256(const ktir_mm_t d) {
  __shared__ __align__(16) uint16_t P0[4 * QT];
  __shared__ __align__(16) uint16_t P1[4 * QT];
  const int tid = threadIdx.x, l = tid & 63, h = l >> 5, r32 = l & 31;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = w >> 1, wc = w & 1;
  const int64_t nblk = gridDim.x;
  int64_t g = blockIdx.x;
  if ((nblk & 7) == 0) g = (g & 7) * (nblk >> 3) + (g >> 3);
  const int32_t* q = (const int32_t*)d.quads + 4 * g;
  const int64_t q0 = uni(q[0]), q1 = uni(q[1]), q2 = uni(q[2]), q3 = uni(q[3]);
  const int64_t a_row = d.a.strides[0], b_row = d.b.strides[0];
  // this wavefront's sub-tile: 0 A top (lane q0), 1 A bottom (q2), 2 B left (q0), 3 B right (q1)
  const bool is_a = w < 2;
  const int64_t src_lane = w == 0 ? q0 : (w == 1 ? q2 : (w == 2 ? q0 : q1));
  const int64_t base = is_a ? uni(lane_offset(d.a, src_lane)) : uni(lane_offset(d.b, src_lane));
  const __amdgpu_buffer_rsrc_t rs = is_a ? mm_rsrc((const uint16_t*)d.a.ptr + base, d.a.hi - base)
                                         : mm_rsrc((const uint16_t*)d.b.ptr + base, d.b.hi - base);
  // lane byte offsets: A blocks of 8 rows (row % 16 = 8 (b % 2) + l / 8), B
  // blocks of 4 k-rows (row % 16 = 4 (b % 4) + l / 16)
  uint32_t lo[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    lo[k] = is_a ? (uint32_t)(((l >> 3) * a_row + 8 * ((l & 7) ^ swz_a(8 * (k & 1) + (l >> 3)))) * 2)
                 : (uint32_t)(((l >> 4) * b_row + 8 * ((l & 15) ^ swz16(4 * k + (l >> 4)))) * 2);
  const int64_t blk_stride = is_a ? 8 * a_row : 4 * b_row;   // elements per 1 KB block
  const int tg = l >> 4, tj = l & 15;
  const int br0 = 8 * (tg >> 1) + (tj >> 2);
  const int bc = 2 * (tg & 1) + ((tj >> 1) & 1), bin = 4 * (tj & 1);
  int b_off[2][4];
#pragma unroll
  for (int hi = 0; hi < 2; ++hi)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      b_off[hi][j] = (br0 + 4 * hi) * NT + 8 * ((4 * j + bc) ^ swz16(br0 + 4 * hi)) + bin;
  const int64_t kt_per_step = d.K / BK;
  const int64_t nk = d.ksteps * kt_per_step;
  const f32x16 z16 = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = z16;
  int64_t s_ = 0, kk0 = 0, di = 0;
  // element offset of k step (s_, kk0) in this wavefront's operand
  const int64_t kst = uni(is_a ? d.a_kstep : d.b_kstep), kmul = is_a ? 1 : b_row;
  // stage sub-tile w of k step di into P (16 blocks of 1 KB); di stops at
  // the last step, which later calls load again
#define Q_ISSUE(P)                                                                                     \
  do {                                                                                                 \
    const int64_t koff = s_ * kst + kk0 * kmul;                                                        \
    uint16_t* dst = (P) + QT * w;                                                                      \
    _Pragma("unroll") for (int b = 0; b < 16; ++b)                                                     \
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (__attribute__((address_space(3))) void*)(dst + 512 * b), 16, \
                                               lo[b & 3], (int)((b * blk_stride + koff) * 2), 0, 0);   \
    const int64_t adv = di < nk - 1;                                                                   \
    di += adv;                                                                                         \
    kk0 += adv * BK;                                                                                   \
    const int64_t wrap = kk0 == kt_per_step * BK;                                                      \
    kk0 = wrap ? 0 : kk0;                                                                              \
    s_ += wrap;                                                                                        \
  } while (0)
  // The barrier of k step t sits between its slices 2 and 3: by then every
  // wavefront has read all of step t's fragments (so the DMA of step t + 2
  // may overwrite its stage) and waited for its own DMA of step t + 1 (so
  // that stage is whole).  Slice 3's MFMAs then cover the DMA issue and the
  // reads of step t + 1's first slice.
#define Q_STEP(PC, PN)                                                                       \
  do {                                                                                       \
    q256_slices012<BF16>(acc, (PC) + QT * wr, (PC) + QT * (2 + wc), r32, h, b_off, a0, b0, a1, b1); \
    __builtin_amdgcn_sched_barrier(0);                                                       \
    __builtin_amdgcn_s_waitcnt(0);                                                           \
    __syncthreads();                                                                         \
    __builtin_amdgcn_sched_barrier(0);                                                       \
    Q_ISSUE(PC);                                                                             \
    q256_frags((PN) + QT * wr, (PN) + QT * (2 + wc), 0, r32, h, b_off, a0, b0);              \
    Q_MFMA16(a1, b1)                                                                         \
    _Pragma("unroll") for (int x = 0; x < 12; ++x) {                                         \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                     \
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                     \
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                                     \
    }                                                                                        \
    _Pragma("unroll") for (int x = 0; x < 4; ++x) {                                          \
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                     \
      __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);                                     \
    }                                                                                        \
  } while (0)
  uint4 a0[4], b0[4], a1[4], b1[4];
  Q_ISSUE(P0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  Q_ISSUE(P1);
  q256_frags(P0 + QT * wr, P0 + QT * (2 + wc), 0, r32, h, b_off, a0, b0);
  // nk is even (checked at launch): whole pairs of steps, one exit.  The DMA
  // issued in the last two steps reloads step nk - 1 into stages no longer
  // read, and the reads after the last barrier are not used.
  for (int64_t t = 0; t < nk; t += 2) {
    Q_STEP(P0, P1);
    Q_STEP(P1, P0);
  }
  __builtin_amdgcn_s_waitcnt(0);
#undef Q_STEP
#undef Q_ISSUE
#undef Q_MFMA16
  // epilogue: this wavefront's lane tile (4 x 4 MFMA tiles; lane l holds
  // column 32 j + l % 32, rows 32 i + 8 (e / 4) + 4 h + e % 4)
  const int64_t ln = w == 0 ? q0 : (w == 1 ? q1 : (w == 2 ? q2 : q3));
  // outs absent or a zero splat (accumulate == 2: x + 0.0), rounded to the
  // result dtype (the only forms launched here)
  const int64_t cb = lane_offset(d.c, ln), cs = d.c.strides[0];
  const float z = d.accumulate == 2 ? 0.f : -0.f;
  if (d.c.dtype == KTIR_F32) {
    q256_out<KTIR_F32>(d.c.ptr, cb, cs, h, r32, acc, z);
  } else {
    // every wavefront's DMA has landed (waited above) and every wavefront is
    // past its last read of the stages: the LDS is free for the result
    __syncthreads();
    uint16_t* stage = (w < 2 ? P0 : P1) + (w & 1) * (2 * QT);
    const bool vec = ((d.c.ptr + 2 * (uint64_t)cb) & 15) == 0 && (cs & 7) == 0;
    if (d.c.dtype == KTIR_F16) {
      if (vec) q256_out16<KTIR_F16>(stage, d.c.ptr, cb, cs, h, r32, l, acc, z);
      else q256_out<KTIR_F16>(d.c.ptr, cb, cs, h, r32, acc, z);
    } else {
      if (vec) q256_out16<KTIR_BF16>(stage, d.c.ptr, cb, cs, h, r32, l, acc, z);
      else q256_out<KTIR_BF16>(d.c.ptr, cb, cs, h, r32, acc, z);
    }
  }
}

}  // namespace ktir

using namespace ktir;

// Host-side eligibility: f16/bf16 operands, row-major with unit inner strides,
// 16-byte aligned rows, M and N multiples of 128, K a multiple of 64.  The
// caller (the lockstep executor) has already checked that every lane's
// operand range lies inside its allocation.
static int64_t kt_steps(const ktir_mm_t* d) { return d->K / BK; }

int ktir_launch_matmul_mfma(const ktir_mm_t* d, bool* handled) {
  *handled = false;
  const bool f16 = d->a.dtype == KTIR_F16 && d->b.dtype == KTIR_F16;
  const bool bf16 = d->a.dtype == KTIR_BF16 && d->b.dtype == KTIR_BF16;
  if (!(f16 || bf16)) return KTIR_OK;
  if (d->M % MT || d->N % NT || d->K % BK) return KTIR_OK;
  if (d->a.strides[1] != 1 || d->b.strides[1] != 1) return KTIR_OK;
  if (d->a.offsets || d->b.offsets) return KTIR_OK;
  auto al8 = [](int64_t x) { return (x & 7) == 0; };
  if (!al8(d->a.strides[0]) || !al8(d->b.strides[0]) || !al8(d->a_kstep) || !al8(d->b_kstep) ||
      (d->a.ptr & 15) || (d->b.ptr & 15))
    return KTIR_OK;
  // per-lane offset arrays: the host has checked bounds and alignment
  const bool checked = (d->a.flags & KTIR_LEAF_CHECKED) && (d->b.flags & KTIR_LEAF_CHECKED);
  if ((d->a.lane_base || d->b.lane_base) && !checked) return KTIR_OK;
  if (!checked && (!al8(d->a.base) || !al8(d->a.lane_stride) || !al8(d->b.base) || !al8(d->b.lane_stride)))
    return KTIR_OK;
  // every element the kernel reads must be inside [lo, hi) for every lane
  const int64_t L = d->lanes;
  auto span_ok = [&](const ktir_leaf_t& l, int64_t rows, int64_t cols, int64_t kstep) {
    int64_t first = l.base, last_lane = l.base + (L - 1) * l.lane_stride;
    int64_t lo = first < last_lane ? first : last_lane, hi = first < last_lane ? last_lane : first;
    int64_t ext = (rows - 1) * l.strides[0] + (cols - 1) + (d->ksteps - 1) * kstep;
    if (ext < 0 || kstep < 0 || l.strides[0] < 0) return false;
    return lo >= l.lo && hi + ext < l.hi;
  };
  if (!checked && (!span_ok(d->a, d->M, d->K, d->a_kstep) || !span_ok(d->b, d->K, d->N, d->b_kstep)))
    return KTIR_OK;
  const int64_t tm = d->M / MT, tn = d->N / NT;
  const int64_t blocks = L * tm * tn;
  if (blocks >= (int64_t)0x7fffffff) return KTIR_OK;
  // the DMA kernel addresses each wavefront's rows with 32-bit buffer offsets
  const int64_t a_span = (31 + 24) * d->a.strides[0] + (d->ksteps - 1) * d->a_kstep + d->K;
  const int64_t b_span = (15 + 12 + d->K) * d->b.strides[0] + (d->ksteps - 1) * d->b_kstep + NT;
  const bool dma = a_span >= 0 && b_span >= 0 && a_span * 2 < (int64_t)0x7fffffff && b_span * 2 < (int64_t)0x7fffffff &&
                   d->a_kstep >= 0 && d->b_kstep >= 0;
  const bool q256 = dma && d->quads && d->n_quads * 4 == L && d->M == MT && d->N == NT &&
                    (d->ksteps * kt_steps(d)) % 2 == 0 && d->n_quads < (int64_t)0x7fffffff &&
                    (d->c.dtype == KTIR_F32 || d->c.dtype == KTIR_F16 || d->c.dtype == KTIR_BF16) &&
                    d->round_dt == KTIR_F32 && d->accumulate != 1 && d->c.strides[1] == 1 &&
                    (127 * d->a.strides[0] + (d->ksteps - 1) * d->a_kstep + d->K) * 2 < (int64_t)0x7fffffff;
  if (q256) {
    if (f16)
      hipLaunchKernelGGL((mm_mfma_256<false>), dim3((unsigned)d->n_quads), dim3(256), 0, stream(), *d);
    else
      hipLaunchKernelGGL((mm_mfma_256<true>), dim3((unsigned)d->n_quads), dim3(256), 0, stream(), *d);
  } else if (dma) {
    if (f16)
      hipLaunchKernelGGL((mm_mfma_dma<false>), dim3((unsigned)blocks), dim3(256), 0, stream(), *d, tm, tn);
    else
      hipLaunchKernelGGL((mm_mfma_dma<true>), dim3((unsigned)blocks), dim3(256), 0, stream(), *d, tm, tn);
  } else if (f16) {
    hipLaunchKernelGGL((mm_mfma<false>), dim3((unsigned)blocks), dim3(256), 0, stream(), *d, tm, tn);
  } else {
    hipLaunchKernelGGL((mm_mfma<true>), dim3((unsigned)blocks), dim3(256), 0, stream(), *d, tm, tn);
  }
  KTIR_HIP_CHECK(hipGetLastError());
  *handled = true;
  return KTIR_OK;
}
