// Device-side building blocks shared by every Flash-DMLA kernel (gfx950 / CDNA4 only).
//
// Lane layouts below were checked on MI355X with an in-bounds probe of each builtin:
//  * v_mfma_f32_16x16x32_bf16: A[16x32] lane l holds A[l%16][8*(l/16)+j], j=0..7;
//    B[32x16] lane l holds B[8*(l/16)+j][l%16]; C[16x16] lane l holds C[4*(l/16)+i][l%16].
//  * global_load_lds (16 B): lane l writes its 16 bytes at lds_base + 16*l.
//  * ds_read_b64_tr_b16: inside each group of 16 lanes, output lane j element e is element
//    (j%4) of the 8 bytes addressed by lane 4*e + j/4.  Reading row-major [k][n] data with
//    lane 4e+q addressing row k0+e, columns n0+4q..n0+4q+3 therefore hands lane j the
//    column n0+j for rows k0..k0+3 -- an MFMA operand with k running along the rows.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dmla {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

#define DMLA_LDS __attribute__((address_space(3)))

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

__device__ __forceinline__ f32x4 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Same tile shapes and lane layouts as the bf16 form.
__device__ __forceinline__ f32x4 mfma_f16(const f16x8& a, const f16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// bf16 -> fp16 of 8 values.  Exact for |x| in fp16's normal range: bf16's 8-bit significand
// fits fp16's 11 bits, so the round-toward-zero pack never rounds; larger magnitudes saturate
// at +-65504 and values below 2^-14 lose low bits as fp16 subnormals.
__device__ __forceinline__ f16x8 bf16_to_f16(const bf16x4& lo, const bf16x4& hi) {
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 a = __builtin_bit_cast(u32x2, lo), b = __builtin_bit_cast(u32x2, hi);
  const auto p0 = __builtin_amdgcn_cvt_pkrtz(__uint_as_float(a[0] << 16), __uint_as_float(a[0] & 0xffff0000u));
  const auto p1 = __builtin_amdgcn_cvt_pkrtz(__uint_as_float(a[1] << 16), __uint_as_float(a[1] & 0xffff0000u));
  const auto p2 = __builtin_amdgcn_cvt_pkrtz(__uint_as_float(b[0] << 16), __uint_as_float(b[0] & 0xffff0000u));
  const auto p3 = __builtin_amdgcn_cvt_pkrtz(__uint_as_float(b[1] << 16), __uint_as_float(b[1] & 0xffff0000u));
  f16x8 r;
  r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
  r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
  return r;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- gradient exponent of the backward kernels ------------------------------------------------
// Every gradient is linear in dO, so a backward may scale dO (and what is linear in it, such as
// dS) by 2^e before an fp16 rounding and its results by 2^-e.  e >= 0 brings the largest |dO| of
// the call to [4, 8), where fp16 operands keep their full 11-bit significand: small gradients
// would otherwise land in fp16's subnormals.  e = 0 when max |dO| >= 4, which leaves every
// result bit-identical to the unscaled computation.  gmax holds the fp32 bits of max |dO|.
__device__ __forceinline__ int grad_exponent(const unsigned* gmax) {
  const unsigned bits = *gmax;
  const int ex = (int)(bits >> 23);
  return bits == 0u || ex >= 0xff ? 0 : min(max(129 - ex, 0), 100);
}
__device__ __forceinline__ float exp2i(int e) { return __uint_as_float((unsigned)(127 + e) << 23); }
// The c of bf16_to_f16_scaled for exponent e: adds e to the exponents of both values of a pair.
__device__ __forceinline__ unsigned grad_exponent_bits(int e) { return ((unsigned)e << 23) | ((unsigned)e << 7); }

// bf16 -> fp16 of 8 values times 2^e, c = grad_exponent_bits(e): one integer add per value pair
// (no carry between the two values while the scaled exponents stay below 255, as they do for
// |x| 2^e < 8).  A zero turns into 2^(e-127) (or its negative) before the conversion, which
// rounds toward zero to a signed zero for e <= 100; so do bf16 subnormals.
__device__ __forceinline__ f16x8 bf16_to_f16_scaled(const bf16x4& lo, const bf16x4& hi, unsigned c) {
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 a = __builtin_bit_cast(u32x2, lo) + c, b = __builtin_bit_cast(u32x2, hi) + c;
  return bf16_to_f16(__builtin_bit_cast(bf16x4, a), __builtin_bit_cast(bf16x4, b));
}

// Maximum of v over a 256-thread workgroup, returned to every thread.  All threads must call
// it, at most once per kernel (its LDS slots are not guarded against a second use).
__device__ __forceinline__ float workgroup_max256(float v) {
  __shared__ float wmax[4];
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
}

// *gmax = fp32 bits of max(vals[0 .. n)) (values >= 0), by one 256-thread workgroup, eight
// loads per thread and round.  Uses workgroup_max256.
__device__ __forceinline__ void reduce_max_bits(const float* vals, int n, unsigned* gmax) {
  float mx = 0.f;
  for (int i0 = 0; i0 < n; i0 += 8 * 256) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = i0 + 256 * j + (int)threadIdx.x;
      v[j] = i < n ? vals[i] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) mx = fmaxf(mx, v[j]);
  }
  mx = workgroup_max256(mx);
  if (threadIdx.x == 0) *gmax = __float_as_uint(mx);
}

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// The lane index, recomputed where it is called: the compiler can neither hoist it out of an
// enclosing loop nor share it with another call.  Per-lane offsets derived from it are then
// computed where they are used instead of being kept live (and spilled) across a long loop.
__device__ __forceinline__ int fresh_lane_id() {
  int v;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(v));
  return v;
}

// Wave-uniform value of an expression that is already uniform (moves it to an SGPR).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// 16-byte direct global->LDS copy of one wave: lane l reads sbase + voff (voff per lane) and
// lands at LDS byte address lds_addr + 16*l.  Issued as inline assembly so the compiler does not
// treat the in-flight copy as aliasing every later LDS read (it would wait for the copy before
// the first one); completion is awaited explicitly with s_waitcnt vmcnt before the barrier that
// publishes the tile.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is reserved: the clobber only documents it
__device__ __forceinline__ void dma16(const void* sbase, unsigned voff, unsigned lds_addr) {
  // Both scalar operands are wave-uniform by construction; readfirstlane makes that explicit
  // to the compiler (a no-op for values it already holds in SGPRs).
  const uint64_t base = reinterpret_cast<uint64_t>(sbase);
  const uint64_t sb = ((uint64_t)__builtin_amdgcn_readfirstlane((unsigned)(base >> 32)) << 32) |
                      (unsigned)__builtin_amdgcn_readfirstlane((unsigned)base);
  const unsigned sl = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(sl), "v"(voff), "s"(reinterpret_cast<const void*>(sb))
               : "memory", "m0");
}
// The copy without a compiler memory barrier, so the scheduler may move LDS reads across it
// (e.g. the next operand reads of an MFMA loop).  The copy overwrites LDS that this wave read
// as MFMA operands; d0..d3 are results of MFMAs that consumed every one of those reads, and as
// asm inputs they order the copy after the reads have completed without keeping the operand
// registers alive.  The caller guarantees that no other wave still reads the destination.
__device__ __forceinline__ void dma16_after(const void* sbase, unsigned voff, unsigned lds_addr, const f32x4& d0,
                                            const f32x4& d1, const f32x4& d2, const f32x4& d3) {
  const uint64_t base = reinterpret_cast<uint64_t>(sbase);
  const uint64_t sb = ((uint64_t)__builtin_amdgcn_readfirstlane((unsigned)(base >> 32)) << 32) |
                      (unsigned)__builtin_amdgcn_readfirstlane((unsigned)base);
  const unsigned sl = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(sl), "v"(voff), "s"(reinterpret_cast<const void*>(sb)), "v"(d0), "v"(d1), "v"(d2), "v"(d3)
               : "m0");
}
// The same ordered after LDS reads whose results are d0..d3 (here: MFMA operands read from the
// slot being refilled): as asm inputs they make the compiler wait for those reads first.
__device__ __forceinline__ void dma16_after_v(const void* sbase, unsigned voff, unsigned lds_addr, const bf16x8& d0,
                                              const bf16x8& d1, const bf16x8& d2, const bf16x8& d3) {
  const uint64_t base = reinterpret_cast<uint64_t>(sbase);
  const uint64_t sb = ((uint64_t)__builtin_amdgcn_readfirstlane((unsigned)(base >> 32)) << 32) |
                      (unsigned)__builtin_amdgcn_readfirstlane((unsigned)base);
  const unsigned sl = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(sl), "v"(voff), "s"(reinterpret_cast<const void*>(sb)), "v"(d0), "v"(d1), "v"(d2), "v"(d3)
               : "m0");
}
// 4-byte direct global->LDS copy of one wave: lane l reads sbase + voff and lands at
// lds_addr + 4*l (per-row scalars staged beside a tile).
__device__ __forceinline__ void dma4(const void* sbase, unsigned voff, unsigned lds_addr) {
  const uint64_t base = reinterpret_cast<uint64_t>(sbase);
  const uint64_t sb = ((uint64_t)__builtin_amdgcn_readfirstlane((unsigned)(base >> 32)) << 32) |
                      (unsigned)__builtin_amdgcn_readfirstlane((unsigned)base);
  const unsigned sl = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2"
               :
               : "s"(sl), "v"(voff), "s"(reinterpret_cast<const void*>(sb))
               : "memory", "m0");
}
// Same copy with a full 64-bit global address per lane (rows of one tile that are far apart,
// e.g. query rows of different heads).
__device__ __forceinline__ void dma16_addr(const void* gaddr, unsigned lds_addr) {
  const unsigned sl = __builtin_amdgcn_readfirstlane(lds_addr);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" : : "s"(sl), "v"(gaddr) : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ unsigned lds_addr(const DMLA_LDS void* p) {
  return (unsigned)(uintptr_t)p;
}

__device__ __forceinline__ bf16x4 lds_read_tr16(const DMLA_LDS bf16x4* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(const_cast<DMLA_LDS bf16x4*>(p));
}

__device__ __forceinline__ f16x4 lds_read_tr16_f16(const DMLA_LDS f16x4* p) {
  typedef __fp16 fp16v4 __attribute__((__vector_size__(8)));  // the builtin's own operand type
  return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((DMLA_LDS fp16v4*)p));
}

__device__ __forceinline__ bf16x8 lds_read_b128(const DMLA_LDS bf16x8* p) { return *p; }

__device__ __forceinline__ bf16x8 concat(const bf16x4& a, const bf16x4& b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// LDS tile layout shared by every kernel that stages a 32-row bf16 tile (keys, queries or
// output gradients): [chunk group (64 columns, 128 B)][row (32)][8 sixteen-byte chunks].  The
// chunk at logical position j of row r sits at physical position j ^ swz(r & 15) with
// swz(r) = r & 7.  Both operand reads are then conflict-free on MI355X (the LDS bank-conflict
// counter reads 0 for each pattern replayed alone): 16 lanes reading one 16-byte chunk of rows
// r..r+15 (b128 row operand) and 32 lanes reading 32-byte column pairs of rows r..r+7
// (ds_read_b64_tr_b16 column operand).  The former ((r >> 1) & 3) << 1 | (r >> 3) & 1 left a
// quarter of the row-operand cycles in conflicts, and measured 0.5-1 % slower.
__host__ __device__ constexpr int swz(int r) { return r & 7; }
constexpr int kTileRows = 32;                 // rows of a staged tile
constexpr int kGroupBytes = kTileRows * 128;  // one 64-column chunk group of a tile (4 KB)

// Byte offset in a staged tile of the 16-byte chunk holding columns 8*chunk .. 8*chunk+7 of
// tile row `row`.
__device__ __forceinline__ int tile_chunk_off(int row, int chunk) {
  return (chunk >> 3) * kGroupBytes + row * 128 + 16 * ((chunk & 7) ^ swz(row & 15));
}
// Per-lane byte offset of a b128 row-operand read (MFMA A or B operand with k along columns):
// lane l reads row 16*rb + l%16, columns 32*c + 8*(l/16) .. +7.
__device__ __forceinline__ int row_operand_off(int lane, int rb, int c) {
  return tile_chunk_off(16 * rb + (lane & 15), 4 * c + (lane >> 4));
}
// Per-lane byte offset of a ds_read_b64_tr_b16 column-operand read (MFMA operand with k along
// rows): lane 4e+q of group g reads row 4g+e (+16 for the second half), columns
// 16*cb + 4q .. +3; the hardware hands lane j of the group column 16*cb + j for 4 rows.
__device__ __forceinline__ int col_operand_off(int lane, int cb, int half) {
  const int g = lane >> 4, e = (lane & 15) >> 2, q = lane & 3;
  const int row = 16 * half + 4 * g + e;
  return tile_chunk_off(row, 2 * cb + (q >> 1)) + 8 * (q & 1);
}

// Division of 0 <= n < 2^31 by a runtime divisor d >= 1 with one multiply-high.  With
// s = ceil(log2 d) and m = floor(2^(31+s) / d) + 1 (< 2^32), n / d = umulhi(n, m) >> (s - 1):
// m d = 2^(31+s) + e with 0 < e <= d, so the quotient's error term n e / (d 2^(31+s)) stays
// below 2^-s <= 1/d, less than the distance from n/d to the next integer.  d = 1 (m = 0) is the
// identity.
struct FastDiv {
  unsigned m;
  int shift;   // s - 1
};
inline FastDiv make_fastdiv(unsigned d) {
  FastDiv f = {0u, 0};
  if (d <= 1) return f;
  int s = 0;
  while ((1ull << s) < d) ++s;
  f.m = (unsigned)((1ull << (31 + s)) / d + 1);
  f.shift = s - 1;
  return f;
}
__device__ __forceinline__ int fast_div(int n, FastDiv f) {
  return f.m ? (int)(__umulhi((unsigned)n, f.m) >> f.shift) : n;
}

// Reductions over the four 16-lane groups of a wave (lanes l, l^16, l^32, l^48: the lanes that
// share one MFMA column) with the gfx950 row-swap instructions.  Called with the same value in
// both operands, permlane16_swap / permlane32_swap return, in some order, a lane's value and
// its partner's (l^16 / l^32); a symmetric combine of the pair therefore needs no lane select.
__device__ __forceinline__ float group_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float group_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Wait until every outstanding vector-memory op of this wave (including LDS DMA) has landed.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0f70); /* gfx9 encoding: vmcnt(0) expcnt(7) lgkmcnt(15) */ }
// At most N vector-memory loads of this wave outstanding (loads retire in issue order).
template <int N>
__device__ __forceinline__ void wait_vmem_le() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(0x0f70 | N);
}

}  // namespace dmla
