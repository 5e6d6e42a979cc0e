// On-the-fly DMLA backward for gfx950: gradients of
//     O[b,h] = softmax(scale * Q[b,h] K_lat[b,h]^T (+ causal mask)) V_lat[b,h],
//     K_lat = K[b,:,h,:] WK[h],  V_lat = V[b,:,h,:] WV[h]        (README.md:14)
// with respect to Q, K, V, WK and WV, from the forward's saved row statistics m and l
// (README.md:12).  The attention part is the intended FA2 backward of
// csrc/attention/fa2_bwd.cu:198-310 (D = rowsum(dO * O), dS = P * (dP - D), dV = P^T dO,
// dK = scale dS^T Q, dQ = scale dS K) with the softmax scale applied to dQ and dK_lat;
// the projections then give
//     dK = dK_lat WK^T,  dWK[h] = sum_{b,s} K[b,s,h,:]^T dK_lat[b,h,s,:]   (same for V / WV).
// The reference has no on-the-fly backward at all (WK / WV are learnable per README.md:14).
//
// Six kernels run in order on one stream, all deterministic (no atomics):
//   otf_bwd_prep_kernel    per query row: lse2 = (m + ln l) log2(e) and -D;
//   otf_bwd_wt_kernel      WK^T and WV^T;
//   otf_bwd_dkdv_kernel    per 128 keys: projects their K_lat and V_lat (also stored in fp16
//                          for the dQ kernel), then dK_lat, dV_lat over the rows that see them;
//   otf_bwd_dq_kernel      per 128 rows: dQ over the keys they see (S and dP recomputed);
//   otf_bwd_wgrad_kernel   per (tensor, head, 1024 keys): dK / dV and a dWK / dWV partial;
//   otf_bwd_wreduce_kernel sums the partials of each head in a fixed order.
//
// Precision.  dK_lat and dV_lat sum one term per row that sees a key, and through them dk, dv
// and the weight gradients grow with the rows per key (non-causal attention over a few keys,
// large batches): |dwv| passes 100 with two keys under 233 rows.  An operand rounded once to
// 16 bits (2^-11 relative for fp16) then moves them by more than 2e-2.  So the dK / dV side
// carries every rounded operand as a bf16 pair hi + lo (hi + lo within 2^-16 relative):
//   * K_lat (times scale log2 e) and V_lat, projected in the dK/dV kernel itself from the raw
//     rows, for the recomputed S (so P matches the forward's statistics, which the forward
//     also scores with a bf16 hi + lo K_lat) and dP;
//   * P and dS, the operands of dV_lat^T += dO^T P and dK_lat^T += Q^T dS;
//   * dK_lat and dV_lat, stored as two bf16 planes for the weight-gradient kernel.
// Q, dO, K, V and the weights are bf16 already, so they enter the bf16 MFMAs exactly and each
// hi + lo operand costs one more MFMA.  dQ sums over the keys of one row and does not grow
// that way: its kernel keeps fp16 operands (Q, dO, K_lat, V_lat, dS rounded to fp16, ~2^-11).
//
// The one layout trick used throughout: an MFMA C tile (lane l holds rows 4(l/16)+i, column
// l%16) of two 16-row blocks is the B operand of a product contracting over those 32 rows when
// the k-index runs over rows {4g+i} then {16+4g+i} (g = l/16); ds_read_b64_tr_b16 on a
// row-major tile hands the A operand exactly that row order (two reads, rows 4g.. and 16+4g..).
// So P and dS never go through LDS.
#include <type_traits>

#include "dmla_common.h"
#include "dmla_host.h"

namespace dmla {
namespace {

constexpr int kIn = 128;                // raw K / V dims per head
constexpr int kLat = 64;                // latent dims (Q, K_lat, V_lat, O)
constexpr int kRowBlk = 128;            // dQ workgroup rows; row statistics are padded to a multiple
constexpr int kKeyBlk = 128;            // dK/dV workgroup keys; keys are padded to a multiple
constexpr int kChunk = 1024;            // keys per weight-gradient workgroup
constexpr int kTile = 32 * kLat * 2;    // one 32-row tile of 64 16-bit columns (4 KB)
constexpr int kStage = 4 * kTile;       // 64 rows of two tensors (16 KB)
constexpr int kRowStage = kStage + 512; // dK/dV stage: 64 rows of Q and dO, then their lse2 and -D
constexpr int kXTile = 32 * kIn * 2;    // one 32-key tile of 128 raw bf16 columns (8 KB)
constexpr int kWgStage = 2 * kXTile + 4 * kTile;   // 64 keys: raw X, dX_lat hi, dX_lat lo (32 KB)

struct OtfBwdParams {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const bf16* wk;
  const bf16* wv;
  const bf16* o;
  const bf16* dout;
  const float* m;   // [B, H, Sq] contiguous
  const float* l;
  void* dq;             // bf16, or fp32 when dq_fp32
  void* dk;             // bf16, or fp32 when dkv_fp32
  void* dv;
  void* dwk;            // bf16, or fp32 when dw_fp32
  void* dwv;
  int dq_fp32, dkv_fp32, dw_fp32;
  int64_t q_sb, q_sh, q_ss, k_sb, k_ss, k_sh, v_sb, v_ss, v_sh, w_sh, w_si;
  int64_t o_sb, o_sh, o_ss, do_sb, do_sh, do_ss;
  int64_t dq_sb, dq_sh, dq_ss, dk_sb, dk_ss, dk_sh, dw_sh, dw_si;
  int B, H, Sq, Sk, causal;
  int Sqp, Skp;          // rows / keys padded to multiples of 128
  int n_sc;              // 1024-key chunks per batch element (weight gradients)
  float scale, scale_log2;
  float* lse2;           // [B*H][Sqp]: (m + ln l) log2(e); padding and empty rows +inf
  float* nd;             // [B*H][Sqp]: -D = -rowsum(dO * O); padding rows 0
  _Float16* klat;        // [B*H][Skp][64] fp16 K_lat * scale log2(e); padding keys zero
  _Float16* vlat;        // [B*H][Skp][64] fp16 V_lat
  bf16* dxlat;           // [4][B*H][Skp][64]: dK_lat hi, dK_lat lo, dV_lat hi, dV_lat lo
  float* wpart;          // [2][H][B*n_sc][128][64] fp32 partial weight gradients
  bf16* wt;              // [2][H][64][128]: WK^T, WV^T
  float* bmax;           // [B*H][Sqp / 128]: largest |dO| of each prep workgroup
  unsigned* gmax;        // largest |dO| of the call as fp32 bits (otf_bwd_wt reduces bmax into it)
};

__device__ __forceinline__ f16x8 to_f16(const bf16x8& x) {
  return bf16_to_f16(__builtin_shufflevector(x, x, 0, 1, 2, 3), __builtin_shufflevector(x, x, 4, 5, 6, 7));
}
__device__ __forceinline__ f16x8 lds_f16x8(const DMLA_LDS char* p) { return *reinterpret_cast<const DMLA_LDS f16x8*>(p); }
__device__ __forceinline__ bf16x8 lds_bf16x8(const DMLA_LDS char* p) { return *reinterpret_cast<const DMLA_LDS bf16x8*>(p); }
// A column operand (k along tile rows) of a 32-row tile: rows 4g..4g+3 then 16+4g..16+4g+3.
__device__ __forceinline__ f16x8 lds_col_operand(const DMLA_LDS char* tile, int lane, int cb) {
  const f16x4 a = lds_read_tr16_f16(reinterpret_cast<const DMLA_LDS f16x4*>(tile + col_operand_off(lane, cb, 0)));
  const f16x4 b = lds_read_tr16_f16(reinterpret_cast<const DMLA_LDS f16x4*>(tile + col_operand_off(lane, cb, 1)));
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}
__device__ __forceinline__ bf16x8 lds_col_operand_bf(const DMLA_LDS char* tile, int lane, int cb) {
  return concat(lds_read_tr16(reinterpret_cast<const DMLA_LDS bf16x4*>(tile + col_operand_off(lane, cb, 0))),
                lds_read_tr16(reinterpret_cast<const DMLA_LDS bf16x4*>(tile + col_operand_off(lane, cb, 1))));
}

// v as a bf16 pair: hi = v's upper 16 bits (truncation), lo = v - hi (exact in fp32) rounded to
// bf16.  |v - hi| < 2^-7 |v| and lo's rounding is 2^-9 of that, so hi + lo is within 2^-16 |v|.
// Three VALU instructions per value: an AND and a subtract per value, one byte permute per two
// hi halves, one packed conversion per two lo values.
__device__ __forceinline__ void split_bf16(const float (&v)[8], bf16x8& hi, bf16x8& lo) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  u32x4 h;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const unsigned a = __float_as_uint(v[2 * e]), b = __float_as_uint(v[2 * e + 1]);
    h[e] = __builtin_amdgcn_perm(b, a, 0x07060302u);   // [a's upper half, b's upper half]
    lo[2 * e] = (bf16)(v[2 * e] - __uint_as_float(a & 0xffff0000u));
    lo[2 * e + 1] = (bf16)(v[2 * e + 1] - __uint_as_float(b & 0xffff0000u));
  }
  hi = __builtin_bit_cast(bf16x8, h);
}
// The same with hi rounded to nearest (|v - hi| <= 2^-9 |v|, hi + lo within 2^-17 |v|); for
// values computed once per kernel, where the extra instructions do not matter.
template <int N>
__device__ __forceinline__ void split_bf16_rn(const float (&v)[N], __bf16 (&hi)[N], __bf16 (&lo)[N]) {
#pragma unroll
  for (int e = 0; e < N; ++e) {
    hi[e] = (bf16)v[e];
    lo[e] = (bf16)(v[e] - (float)hi[e]);
  }
}

// Copies 64 rows of two [rows][64] 16-bit arrays into a stage: [x0 rows 0-31, x0 rows 32-63,
// x1 rows 0-31, x1 rows 32-63], each a 32-row tile in the tile_chunk_off layout.  Rows
// row0 .. row0+63 of x (row r at x0 + r * ss0); rows at or past `rows` re-read row rows-1.
// Sixteen 1 KB wave copies, four per wave; lane l of copy `part` lands at byte 16 l of that
// 1 KB, i.e. tile row 8 part + l/8, physical chunk l%8.  ss * 128 must stay below 2^32.
__device__ __forceinline__ void stage_pair(const void* x0, int64_t ss0, const void* x1, int64_t ss1, int row0,
                                           int rows, unsigned lds_stage, int wave, int lane) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int n = 4 * wave + c;                  // 0 .. 15
    const int x = n >> 3, t = (n >> 2) & 1, part = n & 3;
    const int row = 8 * part + (lane >> 3);
    const int lc = (lane & 7) ^ swz(row & 15);   // logical chunk stored at this physical slot
    const int64_t ss = x ? ss1 : ss0;
    const int rel = min(row0 + 32 * t + row, rows - 1) - row0;
    const char* base = static_cast<const char*>(x ? x1 : x0) + 2 * (int64_t)row0 * ss;
    dma16(base, 2u * (unsigned)(rel * ss + 8 * lc), lds_stage + (2 * x + t) * kTile + part * 1024);
  }
}

// ---------------------------------------------------------------------------------------------
// Prep: one thread per 8 dims of four rows (32 apart); 128 rows per 256-thread block, grid
// (Sqp / 128, B*H).  The eight row loads and the rows' m, l go out before any is used; O is read
// only here, so its loads are non-temporal (they leave the cached lines of later kernels alone).
// Rows past Sq re-read row Sq - 1 and are written as padding (+inf, 0).
__global__ void __launch_bounds__(256) otf_bwd_prep_kernel(OtfBwdParams p) {
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int c = threadIdx.x & 7;
  const int r0 = (int)blockIdx.x * kRowBlk + (int)(threadIdx.x >> 3);
  bf16x8 ov[4], dv[4];
  float mv[4], lv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = min(r0 + 32 * j, p.Sq - 1);
    ov[j] = __builtin_nontemporal_load(
        reinterpret_cast<const bf16x8*>(p.o + b * p.o_sb + h * p.o_sh + (int64_t)r * p.o_ss + 8 * c));
    dv[j] = *reinterpret_cast<const bf16x8*>(p.dout + b * p.do_sb + h * p.do_sh + (int64_t)r * p.do_ss + 8 * c);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t idx = (int64_t)bh * p.Sq + min(r0 + 32 * j, p.Sq - 1);
    mv[j] = p.m[idx];
    lv[j] = p.l[idx];
  }
  __builtin_amdgcn_sched_barrier(0);
  float amax = 0.f, dsum[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    dsum[j] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      dsum[j] += (float)dv[j][e] * (float)ov[j][e];
      amax = fmaxf(amax, fabsf((float)dv[j][e]));
    }
  }
  // The block's largest |dO| (the gradient exponent's input; re-read rows repeat a real row);
  // otf_bwd_wt reduces them.
  amax = workgroup_max256(amax);
  if (threadIdx.x == 0) p.bmax[(size_t)bh * (p.Sqp / kRowBlk) + blockIdx.x] = amax;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float d = dsum[j];
    d += __shfl_xor(d, 1);
    d += __shfl_xor(d, 2);
    d += __shfl_xor(d, 4);
    const int r = r0 + 32 * j;
    if (c == 0) {
      float lse = __builtin_inff();   // P = 0 for padding rows and rows without keys
      if (r < p.Sq && lv[j] > 0.f) lse = mv[j] * kLog2e + __builtin_log2f(lv[j]);
      p.lse2[(size_t)bh * p.Sqp + r] = lse;
      p.nd[(size_t)bh * p.Sqp + r] = r < p.Sq ? -d : 0.f;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// W^T of both projections into the workspace: wt[x][h][dim][in], x = 0 for WK, 1 for WV.
// Grid (H, 2); thread t reads input dim t/2, latent dims 32 (t%2) .. +31.
__global__ void __launch_bounds__(256) otf_bwd_wt_kernel(OtfBwdParams p) {
  const int h = blockIdx.x, x = blockIdx.y;
  const bf16* w = (x ? p.wv : p.wk) + h * p.w_sh + (threadIdx.x >> 1) * p.w_si + 32 * (threadIdx.x & 1);
  bf16* wt = p.wt + ((size_t)x * p.H + h) * (kLat * kIn) + (threadIdx.x >> 1);
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const bf16x8 a = *reinterpret_cast<const bf16x8*>(w + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) wt[(32 * (threadIdx.x & 1) + 8 * c + e) * kIn] = a[e];
  }
  // The call's largest |dO| from the prep kernel's per-workgroup values (prep runs first).
  if (h == 0 && x == 0) reduce_max_bits(p.bmax, p.B * p.H * (p.Sqp / kRowBlk), p.gmax);
}

// X_lat * mul of keys k0 + 16 kb + l16 (kb = 0, 1) as bf16 pairs (hi, lo), each in the layout
// of an MFMA B operand whose k index runs over dims 32 ks + 8 g .. +7 (lane l, g = l/16).
// Projected here from the raw rows: X_lat^T = W^T X^T over four k-steps of 32 input dims.  A C
// tile's lane holds four consecutive rows 4 g .. 4 g + 3, so the A operand (W^T rows) is taken
// in the row order pi(ks, half, 4 g' + i) = 32 ks + 8 g' + 4 half + i: the C tiles of halves
// 0 and 1 then hold dims 32 ks + 8 g + 0..3 and + 4..7 of each lane's key, the two halves of
// its B operand.  Keys at or past Sk come out zero.
__device__ __forceinline__ void project_keys(const OtfBwdParams& p, int x, int b, int h, int k0, int lane,
                                             bf16x8 (&hi)[2][2], bf16x8 (&lo)[2][2]) {
  const int l16 = lane & 15, g = lane >> 4;
  const bf16* src = x ? p.v + b * p.v_sb + h * p.v_sh : p.k + b * p.k_sb + h * p.k_sh;
  const int64_t ss = x ? p.v_ss : p.k_ss;
  bf16x8 xr[2][4];   // [kb][s]: X[key k0 + 16 kb + l16][32 s + 8 g ..]
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const int gk = min(k0 + 16 * kb + l16, p.Sk - 1);
#pragma unroll
    for (int s = 0; s < 4; ++s) xr[kb][s] = *reinterpret_cast<const bf16x8*>(src + (int64_t)gk * ss + 32 * s + 8 * g);
  }
  const bf16* wt = p.wt + ((size_t)x * p.H + h) * (kLat * kIn) + (8 * (l16 >> 2) + (l16 & 3)) * kIn + 8 * g;
  f32x4 c[2][2][2];   // [ks][half][kb]
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      c[ks][half][0] = f32x4{0.f, 0.f, 0.f, 0.f};
      c[ks][half][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(wt + (32 * ks + 4 * half) * kIn + 32 * s);
        c[ks][half][0] = mfma_bf16(a, xr[0][s], c[ks][half][0]);
        c[ks][half][1] = mfma_bf16(a, xr[1][s], c[ks][half][1]);
      }
    }
  const float mul = x ? 1.f : p.scale_log2;
  _Float16* dst16 = (x ? p.vlat : p.klat) + ((size_t)(b * p.H + h) * p.Skp + k0 + l16) * kLat + 8 * g;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const bool live = k0 + 16 * kb + l16 < p.Sk;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      float v[8];
      __bf16 vh[8], vl[8];
      f16x8 v16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = live ? c[ks][0][kb][i] * mul : 0.f;
        v[4 + i] = live ? c[ks][1][kb][i] * mul : 0.f;
      }
      split_bf16_rn(v, vh, vl);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        hi[kb][ks][j] = vh[j];
        lo[kb][ks][j] = vl[j];
        v16[j] = (_Float16)v[j];
      }
      // the fp16 copy the dQ kernel stages: row key, dims 32 ks + 8 g .. +7
      *reinterpret_cast<f16x8*>(dst16 + 16 * kb * kLat + 32 * ks) = v16;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// dK_lat / dV_lat: block = 128 keys of one (b, h), wave w owns keys k0 = 128 kblk + 32 w .. +31,
// whose K_lat (times scale log2 e) and V_lat it projects into registers as bf16 pairs.  Rows
// stream in stages of 64 (Q and dO rows as they are, bf16, copied global -> LDS one stage ahead),
// from the first row that sees any of the block's keys.  Per 32-row sub-tile and wave:
//   S  = Q K_lat^T, dP = dO V_lat^T    (A = Q / dO rows from LDS, B = hi and lo in registers:
//                                      four MFMAs per 16 x 16 tile)
//   P  = exp2(S - lse2), dS = P (dP - D)   (the S accumulators start at -lse2 and the dP ones at
//        -D, so the products hand over the exp2 argument and dP - D)
//   dV_lat^T += dO^T (P_hi + P_lo), dK_lat^T += Q^T (dS_hi + dS_lo)
//                                      (A = dO^T / Q^T by transposed reads; B = the C tiles of
//                                      S and dP as they are)
// Grid: key blocks heavy first (block 0 sees every row under the causal mask).
__global__ void __launch_bounds__(256, 2) otf_bwd_dkdv_kernel(OtfBwdParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[2 * kRowStage];
  DMLA_LDS char* lds = (DMLA_LDS char*)smem;
  const int wave = uniform(threadIdx.x >> 6), lane = lane_id(), l16 = lane & 15, g = lane >> 4;
  const int BH = p.B * p.H;
  const int bh = (int)blockIdx.x % BH, kblk = (int)blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int off = p.Sk - p.Sq;
  const int k0 = kblk * kKeyBlk + 32 * wave;
  bf16x8 khi[2][2], klo[2][2], vhi[2][2], vlo[2][2];   // [kb][ks]
  project_keys(p, 0, b, h, k0, lane, khi, klo);
  project_keys(p, 1, b, h, k0, lane, vhi, vlo);
  f32x4 dkt[4][2], dvt[4][2];     // [db][kb]: X_lat^T[dim 16 db + 4 g + i][key k0 + 16 kb + l16]
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      dkt[db][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
      dvt[db][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  const int row_first = p.causal ? max(0, kblk * kKeyBlk - off) : 0;
  const int rs0 = row_first / 64 * 64;
  const int n_st = row_first >= p.Sq ? 0 : (p.Sq - rs0 + 63) / 64;
  const bf16* qsrc = p.q + b * p.q_sb + h * p.q_sh;
  const bf16* dsrc = p.dout + b * p.do_sb + h * p.do_sh;
  const float* lse2 = p.lse2 + (size_t)bh * p.Sqp;
  const float* nd = p.nd + (size_t)bh * p.Sqp;
  const unsigned lbase = lds_addr(lds);

  // Rows row0 .. row0+63 of Q and dO (stage_pair) and of lse2 and -D (waves 0 and 1, one
  // 4-byte copy per lane) into the stage at byte address lst.
  auto stage_rows = [&](int row0, unsigned lst) {
    stage_pair(qsrc, p.q_ss, dsrc, p.do_ss, row0, p.Sq, lst, wave, lane);
    if (wave < 2) dma4(wave ? nd : lse2, 4u * (unsigned)(row0 + lane), lst + kStage + 256 * wave);
  };

  // One 32-row sub-tile; kMask applies the causal / key-range mask (only sub-tiles that reach
  // past some pair's limit need it), so the common case is straight-line code.  rs points at
  // the stage's lse2 and -D of the sub-tile's rows.
  auto subtile = [&](const DMLA_LDS char* qt, const DMLA_LDS char* dt, const DMLA_LDS char* rs, int r0,
                     auto mask_tag) {
    constexpr bool kMask = decltype(mask_tag)::value;
    f32x4 sacc[2][2], dpacc[2][2];   // [rb][kb]: rows 16 rb + 4 g + i, key 16 kb + l16
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const f32x4 ls = *reinterpret_cast<const DMLA_LDS f32x4*>(rs + 4 * (16 * rb + 4 * g));
      const f32x4 ndv = *reinterpret_cast<const DMLA_LDS f32x4*>(rs + 256 + 4 * (16 * rb + 4 * g));
      const bf16x8 qa0 = lds_bf16x8(qt + row_operand_off(lane, rb, 0));
      const bf16x8 qa1 = lds_bf16x8(qt + row_operand_off(lane, rb, 1));
      const bf16x8 oa0 = lds_bf16x8(dt + row_operand_off(lane, rb, 0));
      const bf16x8 oa1 = lds_bf16x8(dt + row_operand_off(lane, rb, 1));
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        f32x4 s = mfma_bf16(qa0, klo[kb][0], -ls);
        s = mfma_bf16(qa0, khi[kb][0], s);
        s = mfma_bf16(qa1, klo[kb][1], s);
        sacc[rb][kb] = mfma_bf16(qa1, khi[kb][1], s);
        f32x4 d = mfma_bf16(oa0, vlo[kb][0], ndv);
        d = mfma_bf16(oa0, vhi[kb][0], d);
        d = mfma_bf16(oa1, vlo[kb][1], d);
        dpacc[rb][kb] = mfma_bf16(oa1, vhi[kb][1], d);
      }
    }
    // Column operands of the dV / dK updates (dO^T, Q^T of dims 16 db ..), one step ahead: those
    // of db = 0 go out before the exp2 work (held there by the scheduling barrier), those of
    // db + 1 while the MFMAs of db run.  (Read right before their MFMAs, each group's LDS round
    // trip was waited out.)
    bf16x8 otn = lds_col_operand_bf(dt, lane, 0);
    bf16x8 qtn = lds_col_operand_bf(qt, lane, 0);
    __builtin_amdgcn_sched_barrier(0);
    bf16x8 pbh[2], pbl[2], dsh[2], dsl[2];   // [kb]: B operands, slot 4 rb + i = row 16 rb + 4 g + i
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      float pv[8], dv[8];
#pragma unroll
      for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float e = fast_exp2(sacc[rb][kb][i]);
          if constexpr (kMask) {
            const int row = r0 + 16 * rb + 4 * g + i, key = k0 + 16 * kb + l16;
            const int lim = p.causal ? min(row + off, p.Sk - 1) : p.Sk - 1;
            e = key > lim ? 0.f : e;
          }
          pv[4 * rb + i] = e;
          dv[4 * rb + i] = e * dpacc[rb][kb][i];
        }
      split_bf16(pv, pbh[kb], pbl[kb]);
      split_bf16(dv, dsh[kb], dsl[kb]);
    }
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const bf16x8 ot = otn;    // dO^T[dim 16 db + l16][rows]
      const bf16x8 qtt = qtn;   // Q^T
      if (db + 1 < 4) {
        otn = lds_col_operand_bf(dt, lane, db + 1);
        qtn = lds_col_operand_bf(qt, lane, db + 1);
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        dvt[db][kb] = mfma_bf16(ot, pbl[kb], dvt[db][kb]);
        dvt[db][kb] = mfma_bf16(ot, pbh[kb], dvt[db][kb]);
        dkt[db][kb] = mfma_bf16(qtt, dsl[kb], dkt[db][kb]);
        dkt[db][kb] = mfma_bf16(qtt, dsh[kb], dkt[db][kb]);
      }
      if (db + 1 < 4) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);   // reads of db + 1
      __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);                   // MFMAs of db
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // One stage; the buffer index is a compile-time constant (the loop below is unrolled by two)
  // so that every LDS address is a lane offset plus an instruction immediate.  kAny: the stage
  // may hold sub-tiles to skip or to mask, each picked at run time; otherwise every sub-tile
  // takes the unmasked body with no branch (padding rows past Sq contribute 0: their P is 0
  // through lse2 = +inf).
  auto stage_iter = [&](int s, auto buf_tag, auto any_tag) {
    constexpr int kBuf = decltype(buf_tag)::value;
    wait_vmem();
    __syncthreads();   // stage s complete; every wave is done with stage s-1
    if (s + 1 < n_st) stage_rows(rs0 + 64 * (s + 1), lbase + (1 - kBuf) * kRowStage);
    const DMLA_LDS char* st = lds + kBuf * kRowStage;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r0 = rs0 + 64 * s + 32 * t;
      if constexpr (decltype(any_tag)::value) {
        if (r0 >= p.Sq || (p.causal && k0 > r0 + 31 + off)) continue;   // padding only / all masked
        if (k0 + 31 >= p.Sk || (p.causal && k0 + 31 > r0 + off))
          subtile(st + t * kTile, st + (2 + t) * kTile, st + kStage + 128 * t, r0, std::true_type{});
        else
          subtile(st + t * kTile, st + (2 + t) * kTile, st + kStage + 128 * t, r0, std::false_type{});
      } else {
        subtile(st + t * kTile, st + (2 + t) * kTile, st + kStage + 128 * t, r0, std::false_type{});
      }
    }
  };
  // The stages near the diagonal (and all of them in a key block reaching past Sk) come first,
  // an even number of them; from there on no sub-tile of any wave needs a mask.  Alternating
  // between the two bodies inside one loop had the compiler copy the 64 dK/dV accumulator
  // registers at every join.
  const int key_last = kblk * kKeyBlk + kKeyBlk - 1;   // the workgroup's last key
  int s_split = n_st;
  if (key_last < p.Sk) s_split = p.causal ? max(0, (key_last - off - rs0 + 63) / 64) : 0;
  s_split = min(n_st, (s_split + 1) & ~1);
  using Any = std::true_type;
  using Clean = std::false_type;
  if (n_st > 0) stage_rows(rs0, lbase);
  for (int s = 0; s < s_split; s += 2) {
    stage_iter(s, std::integral_constant<int, 0>{}, Any{});
    if (s + 1 < n_st) stage_iter(s + 1, std::integral_constant<int, 1>{}, Any{});
  }
  for (int s = s_split; s < n_st; s += 2) {
    stage_iter(s, std::integral_constant<int, 0>{}, Clean{});
    if (s + 1 < n_st) stage_iter(s + 1, std::integral_constant<int, 1>{}, Clean{});
  }
  // dK_lat = scale dS^T Q and dV_lat = P^T dO as bf16 hi / lo planes (keys past Sk hold zeros:
  // P = 0 there).  A lane holds dims 16 db + 4 g .. + 3 of key 16 kb + l16; one lane-row swap
  // (rows of 16 lanes) per dword between the pieces of db = 2 dp and 2 dp + 1 leaves lane g with
  // dims 32 dp + 16 (g & 1) + 8 (g >> 1) .. + 7, so each store is 16 bytes a lane and 64
  // contiguous bytes a key row.
  typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  const size_t plane = (size_t)BH * p.Skp * kLat;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    bf16* row = p.dxlat + ((size_t)bh * p.Skp + k0 + 16 * kb + l16) * kLat + 16 * (g & 1) + 8 * (g >> 1);
#pragma unroll
    for (int dp = 0; dp < 2; ++dp) {
      u32x2 pc[4][2];   // [plane][db - 2 dp]
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int db = 2 * dp + j;
        float a[4], c[4];
        __bf16 ah[4], al[4], ch[4], cl[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a[i] = dkt[db][kb][i] * p.scale;
          c[i] = dvt[db][kb][i];
        }
        split_bf16_rn(a, ah, al);
        split_bf16_rn(c, ch, cl);
        bf16x4 vah, val, vch, vcl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          vah[i] = ah[i];
          val[i] = al[i];
          vch[i] = ch[i];
          vcl[i] = cl[i];
        }
        pc[0][j] = __builtin_bit_cast(u32x2, vah);
        pc[1][j] = __builtin_bit_cast(u32x2, val);
        pc[2][j] = __builtin_bit_cast(u32x2, vch);
        pc[3][j] = __builtin_bit_cast(u32x2, vcl);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        u32x4 v;
#pragma unroll
        for (int w = 0; w < 2; ++w) {
          const auto r = __builtin_amdgcn_permlane16_swap(pc[q][0][w], pc[q][1][w], false, false);
          v[w] = r[0];
          v[2 + w] = r[1];
        }
        *reinterpret_cast<u32x4*>(row + q * plane + 32 * dp) = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// dQ: block = 128 rows of one (b, h), wave w owns rows r0 = 128 rblk + 32 w .. +31, whose Q and
// dO it holds in registers as fp16 (converted exactly from bf16).  Keys stream in stages of 64
// (fp16 K_lat and V_lat, copied one stage ahead) up to the last key any row sees.
// Per 32-key sub-tile and wave:
//   S^T = K_lat Q^T, dP^T = V_lat dO^T   (A = K_lat / V_lat rows from LDS, B = Q / dO in registers)
//   dS^T = P^T (dP^T - D)
//   dQ += dS K_lat                        (A = dS straight from the C tiles of S^T; B = K_lat by
//                                          transposed reads, keys in the same order)
// Grid: row blocks heavy (last) first.  Three workgroups per CU (168 registers, 32 KB of LDS
// each): a sub-tile is one dependent chain (S and dP, then exp2 and dS, then the dQ MFMAs), and
// a third wave per SIMD covers more of its latency than two (191 -> 184 us at the cfg-4 shapes).
__global__ void __launch_bounds__(256, 3) otf_bwd_dq_kernel(OtfBwdParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[2 * kStage];
  DMLA_LDS char* lds = (DMLA_LDS char*)smem;
  const int wave = uniform(threadIdx.x >> 6), lane = lane_id(), l16 = lane & 15, g = lane >> 4;
  const int BH = p.B * p.H;
  const int bh = (int)blockIdx.x % BH;
  const int rblk = p.Sqp / kRowBlk - 1 - (int)blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int off = p.Sk - p.Sq;
  const int r0 = rblk * kRowBlk + 32 * wave;
  // dO, and with it dP, D, dS and dQ, carry 2^e (the gradient exponent) through the fp16 products.
  const int gexp = grad_exponent(p.gmax);
  const unsigned gexp_bits = grad_exponent_bits(gexp);
  const float gscale = exp2i(gexp);
  f16x8 qreg[2][2], oreg[2][2];   // [rb][ks]: X[r0 + 16 rb + l16][32 ks + 8 g ..] as fp16 (dO times 2^e)
  float lse[2];
  f32x4 ndv[2];   // -D 2^e of row r0 + 16 rb + l16 in all four elements: the dP^T accumulator start
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    // Rows past Sq re-read row Sq-1: their lse2 is +inf, so their P is 0.
    const int row = min(r0 + 16 * rb + l16, p.Sq - 1);
    const bf16* qrow = p.q + b * p.q_sb + h * p.q_sh + (int64_t)row * p.q_ss + 8 * g;
    const bf16* orow = p.dout + b * p.do_sb + h * p.do_sh + (int64_t)row * p.do_ss + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      qreg[rb][ks] = to_f16(*reinterpret_cast<const bf16x8*>(qrow + 32 * ks));
      const bf16x8 ox = *reinterpret_cast<const bf16x8*>(orow + 32 * ks);
      oreg[rb][ks] = bf16_to_f16_scaled(__builtin_shufflevector(ox, ox, 0, 1, 2, 3),
                                        __builtin_shufflevector(ox, ox, 4, 5, 6, 7), gexp_bits);
    }
    lse[rb] = p.lse2[(size_t)bh * p.Sqp + r0 + 16 * rb + l16];
    const float n = p.nd[(size_t)bh * p.Sqp + r0 + 16 * rb + l16] * gscale;
    ndv[rb] = f32x4{n, n, n, n};
  }
  f32x4 dq[2][4];   // [rb][db]: dQ[r0 + 16 rb + 4 g + i][16 db + l16]
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int db = 0; db < 4; ++db) dq[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int last_row = min(p.Sq, rblk * kRowBlk + kRowBlk) - 1;
  const int key_end = p.causal ? min(p.Sk, last_row + off + 1) : p.Sk;
  const int n_st = key_end > 0 ? (key_end + 63) / 64 : 0;
  const _Float16* ksrc = p.klat + (size_t)bh * p.Skp * kLat;
  const _Float16* vsrc = p.vlat + (size_t)bh * p.Skp * kLat;
  const unsigned lbase = lds_addr(lds);

  auto subtile = [&](const DMLA_LDS char* kt, const DMLA_LDS char* vt, int c0, auto mask_tag) {
    constexpr bool kMask = decltype(mask_tag)::value;
    // The dQ product's K_lat column operands do not depend on S or dP: their reads go out first
    // (kept there by the scheduling barrier), so they have landed by the time dS is formed.
    f16x8 kcol[4];   // K_lat[keys][dim 16 db + l16]
#pragma unroll
    for (int db = 0; db < 4; ++db) kcol[db] = lds_col_operand(kt, lane, db);
    __builtin_amdgcn_sched_barrier(0);
    f32x4 sT[2][2], dpT[2][2];   // [kb][rb]: keys 16 kb + 4 g + i, row 16 rb + l16
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const f16x8 ka0 = lds_f16x8(kt + row_operand_off(lane, kb, 0));
      const f16x8 ka1 = lds_f16x8(kt + row_operand_off(lane, kb, 1));
      const f16x8 va0 = lds_f16x8(vt + row_operand_off(lane, kb, 0));
      const f16x8 va1 = lds_f16x8(vt + row_operand_off(lane, kb, 1));
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        sT[kb][rb] = mfma_f16(ka0, qreg[rb][0], f32x4{-lse[rb], -lse[rb], -lse[rb], -lse[rb]});
        sT[kb][rb] = mfma_f16(ka1, qreg[rb][1], sT[kb][rb]);
        dpT[kb][rb] = mfma_f16(va0, oreg[rb][0], ndv[rb]);
        dpT[kb][rb] = mfma_f16(va1, oreg[rb][1], dpT[kb][rb]);
      }
    }
    f16x8 dsa[2];   // [rb]: A operand, slot 4 kb + i = key 16 kb + 4 g + i
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float pv = fast_exp2(sT[kb][rb][i]);
          if constexpr (kMask) {
            const int row = r0 + 16 * rb + l16, key = c0 + 16 * kb + 4 * g + i;
            const int lim = p.causal ? min(row + off, p.Sk - 1) : p.Sk - 1;
            pv = key > lim ? 0.f : pv;
          }
          dsa[rb][4 * kb + i] = (_Float16)(pv * dpT[kb][rb][i]);
        }
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) dq[rb][db] = mfma_f16(dsa[rb], kcol[db], dq[rb][db]);
  };

  // Unrolled by two stages so that the buffer offset is an instruction immediate.  kAny: the
  // stage may hold sub-tiles to skip or to mask, picked at run time; otherwise every sub-tile
  // takes the unmasked body with no branch.
  auto stage_iter = [&](int s, auto buf_tag, auto any_tag) {
    constexpr int kBuf = decltype(buf_tag)::value;
    wait_vmem();
    __syncthreads();
    if (s + 1 < n_st) stage_pair(ksrc, kLat, vsrc, kLat, 64 * (s + 1), p.Skp, lbase + (1 - kBuf) * kStage, wave, lane);
    const DMLA_LDS char* st = lds + kBuf * kStage;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int c0 = 64 * s + 32 * t;
      if constexpr (decltype(any_tag)::value) {
        if (c0 >= key_end || (p.causal && c0 > r0 + 31 + off)) continue;
        if (c0 + 31 >= p.Sk || (p.causal && c0 + 31 > r0 + off))
          subtile(st + t * kTile, st + (2 + t) * kTile, c0, std::true_type{});
        else
          subtile(st + t * kTile, st + (2 + t) * kTile, c0, std::false_type{});
      } else {
        subtile(st + t * kTile, st + (2 + t) * kTile, c0, std::false_type{});
      }
    }
  };
  // The stages whose keys every row of the block sees come first, an even number of them; the
  // ones reaching the diagonal (or past Sk) follow.  With both sub-tile bodies in one loop, the
  // compiler had copied the 32 dQ accumulator registers at every join.
  const int lim_all = min(min(p.Sk, key_end) - 1, p.causal ? rblk * kRowBlk + off : p.Sk);
  const int s_split = min(n_st, lim_all >= 0 ? ((lim_all + 1) / 64) & ~1 : 0);
  using Any = std::true_type;
  using Clean = std::false_type;
  if (n_st > 0) stage_pair(ksrc, kLat, vsrc, kLat, 0, p.Skp, lbase, wave, lane);
  for (int s = 0; s < s_split; s += 2) {
    stage_iter(s, std::integral_constant<int, 0>{}, Clean{});
    if (s + 1 < n_st) stage_iter(s + 1, std::integral_constant<int, 1>{}, Clean{});
  }
  for (int s = s_split; s < n_st; s += 2) {
    stage_iter(s, std::integral_constant<int, 0>{}, Any{});
    if (s + 1 < n_st) stage_iter(s + 1, std::integral_constant<int, 1>{}, Any{});
  }
  const float unscale = kLn2 * exp2i(-gexp);   // scale / (scale log2 e), and 2^-e
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = r0 + 16 * rb + 4 * g + i;
      if (row >= p.Sq) continue;
      const int64_t at = b * p.dq_sb + h * p.dq_sh + (int64_t)row * p.dq_ss + l16;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const float v = dq[rb][db][i] * unscale;
        if (p.dq_fp32) static_cast<float*>(p.dq)[at + 16 * db] = v;
        else static_cast<bf16*>(p.dq)[at + 16 * db] = (bf16)v;
      }
    }
}

// ---------------------------------------------------------------------------------------------
// Weight side: block = (tensor x in {K, V}, head h, batch b, chunk c of 1024 keys), grid
// (n_sc, H, 2 B).  Per 64-key block (raw X rows and the dX_lat hi / lo planes copied global ->
// LDS directly, one block ahead):
//   dX^T[in][key] = W[in][:] dX_lat^T       wave w: keys 16 w .. +15 (A = W rows in registers,
//                                           B = dX_lat hi, lo rows from LDS); written as dX rows
//   dW[in][dim]  += X^T[in][key] dX_lat     wave w: input dims 32 w .. +31 (both operands by
//                                           transposed reads, keys in the same order)
// The fp32 dW partial of the chunk goes to wpart; otf_bwd_wreduce_kernel sums the chunks.
__global__ void __launch_bounds__(256, 2) otf_bwd_wgrad_kernel(OtfBwdParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[2 * kWgStage];
  DMLA_LDS char* lds = (DMLA_LDS char*)smem;
  const int wave = uniform(threadIdx.x >> 6), lane = lane_id(), l16 = lane & 15, g = lane >> 4;
  const int c = blockIdx.x, h = blockIdx.y, x = blockIdx.z & 1, b = blockIdx.z >> 1;
  const int bh = b * p.H + h;
  const bf16* X = x ? p.v + b * p.v_sb + h * p.v_sh : p.k + b * p.k_sb + h * p.k_sh;
  const int64_t x_ss = x ? p.v_ss : p.k_ss;
  const bf16* W = (x ? p.wv : p.wk) + h * p.w_sh;
  const size_t plane = (size_t)p.B * p.H * p.Skp * kLat;
  const bf16* dxh = p.dxlat + 2 * x * plane + (size_t)bh * p.Skp * kLat;
  const bf16* dxl = dxh + plane;
  const int64_t dx_at = b * p.dk_sb + h * p.dk_sh;
  const int key_lo = c * kChunk, key_hi = min(p.Sk, key_lo + kChunk);
  const int n_blk = (key_hi - key_lo + 63) / 64;
  const unsigned lbase = lds_addr(lds);

  bf16x8 wa[8][2];   // [ib][ks]: W[16 ib + l16][32 ks + 8 g ..]
#pragma unroll
  for (int ib = 0; ib < 8; ++ib)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) wa[ib][ks] = *reinterpret_cast<const bf16x8*>(W + (16 * ib + l16) * p.w_si + 32 * ks + 8 * g);
  f32x4 dw[2][4];   // [ib - 2 w][db]: dW[16 ib + 4 g + i][16 db + l16]
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int db = 0; db < 4; ++db) dw[a][db] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One 64-key block into stage buffer buf: raw X as two 32-key tiles of two chunk groups
  // (16 wave copies of 1 KB), then the hi and lo dX_lat planes as two 32-key tiles each
  // (16 copies); eight per wave.  Keys past Sk re-read key Sk-1 (their dX_lat rows are zero).
  auto stage_block = [&](int blk, int buf) {
    const int key0 = key_lo + 64 * blk;
    const unsigned sbuf = lbase + buf * kWgStage;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int n = 4 * wave + cc;
      const int t = n >> 3, grp = (n >> 2) & 1, part = n & 3;
      const int row = 8 * part + (lane >> 3);
      const int lc = (lane & 7) ^ swz(row & 15);
      const int rel = min(key0 + 32 * t + row, p.Sk - 1) - key0;
      dma16(X + key0 * x_ss, 2u * (unsigned)(rel * x_ss + 64 * grp + 8 * lc), sbuf + t * kXTile + grp * kGroupBytes + part * 1024);
    }
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      const int n = 4 * wave + cc;
      const int pl = n >> 3, t = (n >> 2) & 1, part = n & 3;
      const int row = 8 * part + (lane >> 3);
      const int lc = (lane & 7) ^ swz(row & 15);
      dma16(pl ? dxl : dxh, 2u * (unsigned)((key0 + 32 * t + row) * kLat + 8 * lc),
            sbuf + 2 * kXTile + (2 * pl + t) * kTile + part * 1024);
    }
  };

  if (n_blk > 0) stage_block(0, 0);
  for (int blk = 0; blk < n_blk; ++blk) {
    wait_vmem();
    __syncthreads();   // block blk complete in buffer blk & 1; buffer (blk + 1) & 1 free
    if (blk + 1 < n_blk) stage_block(blk + 1, (blk + 1) & 1);
    const DMLA_LDS char* xs = lds + (blk & 1) * kWgStage;
    const DMLA_LDS char* dhs = xs + 2 * kXTile;     // hi tiles (keys 0-31, 32-63)
    const DMLA_LDS char* dls = dhs + 2 * kTile;     // lo tiles
    // dX^T for keys 16 wave + l16 of the block
    {
      const int tt = (wave >> 1) * kTile, rb = wave & 1;
      const bf16x8 h0 = lds_bf16x8(dhs + tt + row_operand_off(lane, rb, 0));
      const bf16x8 h1 = lds_bf16x8(dhs + tt + row_operand_off(lane, rb, 1));
      const bf16x8 lo0 = lds_bf16x8(dls + tt + row_operand_off(lane, rb, 0));
      const bf16x8 lo1 = lds_bf16x8(dls + tt + row_operand_off(lane, rb, 1));
      const int key = key_lo + 64 * blk + 16 * wave + l16;
#pragma unroll
      for (int ib = 0; ib < 8; ++ib) {
        f32x4 cacc = mfma_bf16(wa[ib][0], lo0, f32x4{0.f, 0.f, 0.f, 0.f});
        cacc = mfma_bf16(wa[ib][0], h0, cacc);
        cacc = mfma_bf16(wa[ib][1], lo1, cacc);
        cacc = mfma_bf16(wa[ib][1], h1, cacc);    // dX^T[in 16 ib + 4 g + i][key]
        if (key < key_hi) {
          const int64_t at = dx_at + (int64_t)key * p.dk_ss + 16 * ib + 4 * g;
          if (p.dkv_fp32) {
            *reinterpret_cast<f32x4*>(static_cast<float*>(x ? p.dv : p.dk) + at) = cacc;
          } else {
            bf16x4 v;
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = (bf16)cacc[i];
            *reinterpret_cast<bf16x4*>(static_cast<bf16*>(x ? p.dv : p.dk) + at) = v;
          }
        }
      }
    }
    // dW over the block's 64 keys (two k-steps of 32)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const bf16x8 a0 = lds_col_operand_bf(xs + t * kXTile, lane, 2 * wave);
      const bf16x8 a1 = lds_col_operand_bf(xs + t * kXTile, lane, 2 * wave + 1);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const bf16x8 bl = lds_col_operand_bf(dls + t * kTile, lane, db);
        const bf16x8 bh2 = lds_col_operand_bf(dhs + t * kTile, lane, db);
        dw[0][db] = mfma_bf16(a0, bl, dw[0][db]);
        dw[0][db] = mfma_bf16(a0, bh2, dw[0][db]);
        dw[1][db] = mfma_bf16(a1, bl, dw[1][db]);
        dw[1][db] = mfma_bf16(a1, bh2, dw[1][db]);
      }
    }
  }
  float* part = p.wpart + (((size_t)x * p.H + h) * ((size_t)p.B * p.n_sc) + (size_t)b * p.n_sc + c) * (kIn * kLat);
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[(16 * (2 * wave + a) + 4 * g + i) * kLat + 16 * db + l16] = dw[a][db][i];
}

// dW[h] = sum of the B * n_sc chunk partials in chunk order; one element per thread,
// grid (128 * 64 / 256, H, 2).
__global__ void __launch_bounds__(256) otf_bwd_wreduce_kernel(OtfBwdParams p) {
  const int h = blockIdx.y, x = blockIdx.z;
  const int e = blockIdx.x * 256 + threadIdx.x;
  const int np = p.B * p.n_sc;
  const float* part = p.wpart + ((size_t)x * p.H + h) * (size_t)np * (kIn * kLat) + e;
  float acc = 0.f;
  for (int j = 0; j < np; ++j) acc += part[(size_t)j * (kIn * kLat)];
  const int64_t at = h * p.dw_sh + (e / kLat) * p.dw_si + (e % kLat);
  if (p.dw_fp32) static_cast<float*>(x ? p.dwv : p.dwk)[at] = acc;
  else static_cast<bf16*>(x ? p.dwv : p.dwk)[at] = (bf16)acc;
}

struct OtfBwdPlan {
  int Sqp, Skp, n_sc;
  size_t off_lse2, off_nd, off_klat, off_vlat, off_dx, off_wpart, off_wt, off_bmax, off_gmax, bytes;
};

OtfBwdPlan make_otf_plan(int64_t B, int64_t H, int64_t Sq, int64_t Sk) {
  OtfBwdPlan pl = {};
  pl.Sqp = (int)((Sq + kRowBlk - 1) / kRowBlk * kRowBlk);
  pl.Skp = (int)((Sk + kKeyBlk - 1) / kKeyBlk * kKeyBlk);
  pl.n_sc = (int)((Sk + kChunk - 1) / kChunk);
  auto up = [](size_t n) { return (n + 255) / 256 * 256; };
  const size_t rows = (size_t)B * H * pl.Sqp, keys = (size_t)B * H * pl.Skp;
  size_t o = 0;
  pl.off_lse2 = o;  o += up(rows * sizeof(float));
  pl.off_nd = o;    o += up(rows * sizeof(float));
  pl.off_klat = o;  o += up(keys * kLat * 2);
  pl.off_vlat = o;  o += up(keys * kLat * 2);
  pl.off_dx = o;    o += up(4 * keys * kLat * 2);
  pl.off_wpart = o; o += up((size_t)2 * H * B * pl.n_sc * kIn * kLat * sizeof(float));
  pl.off_wt = o;    o += up((size_t)2 * H * kIn * kLat * 2);
  pl.off_bmax = o;  o += up(rows / kRowBlk * sizeof(float));
  pl.off_gmax = o;  o += 256;
  pl.bytes = o;
  return pl;
}

constexpr int64_t kOtfBwdMaxSeq = (int64_t)1 << 24;    // keeps the 32-bit copy offsets in range
constexpr int64_t kOtfBwdMaxRowStride = (int64_t)1 << 24;   // q / dout / k / v row strides (elements)

}  // namespace
}  // namespace dmla

using namespace dmla;

extern "C" int64_t dmla_bwd_onthefly_workspace_bytes(int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t d_in,
                                                     int64_t d_lat) {
  if (B <= 0 || H <= 0 || Sq <= 0 || Sk <= 0 || d_in != kIn || d_lat != kLat) return 0;
  if (Sq > kOtfBwdMaxSeq || Sk > kOtfBwdMaxSeq) return 0;
  return (int64_t)make_otf_plan(B, H, Sq, Sk).bytes;
}

extern "C" int dmla_bwd_onthefly(const void* q, const void* k, const void* v, const void* wk, const void* wv,
                                 const void* o, const void* dout, const float* m, const float* l, void* dq,
                                 void* dk, void* dv, void* dwk, void* dwv, int64_t B, int64_t H, int64_t Sq,
                                 int64_t Sk, int64_t d_in, int64_t d_lat, int64_t q_sb, int64_t q_sh,
                                 int64_t q_ss, int64_t k_sb, int64_t k_ss, int64_t k_sh, int64_t v_sb,
                                 int64_t v_ss, int64_t v_sh, int64_t w_sh, int64_t w_si, int64_t o_sb,
                                 int64_t o_sh, int64_t o_ss, int64_t do_sb, int64_t do_sh, int64_t do_ss,
                                 int64_t dq_sb, int64_t dq_sh, int64_t dq_ss, int64_t dk_sb, int64_t dk_ss,
                                 int64_t dk_sh, int64_t dw_sh, int64_t dw_si, int dq_fp32, int dkv_fp32,
                                 int dw_fp32, float softmax_scale, int causal, void* workspace,
                                 int64_t workspace_bytes, dmla_stream_t stream) {
  clear_error();
  if (!q || !k || !v || !wk || !wv || !o || !dout || !m || !l || !dq || !dk || !dv || !dwk || !dwv)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_bwd_onthefly: null pointer argument");
  if (B < 0 || H < 0 || Sq < 0 || Sk < 0) return fail(DMLA_ERR_INVALID_ARG, "dmla_bwd_onthefly: negative size");
  if (d_in != kIn || d_lat != kLat)
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_bwd_onthefly: only d_in=128, d_lat=64 is compiled (got %lld, %lld)",
                (long long)d_in, (long long)d_lat);
  if (!(softmax_scale > 0.f) || !__builtin_isfinite(softmax_scale))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_bwd_onthefly: softmax_scale must be finite and > 0");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(wk) || !aligned16(wv) || !aligned16(o) ||
      !aligned16(dout) || !aligned16(m) || !aligned16(l) || !aligned16(dq) || !aligned16(dk) || !aligned16(dv) ||
      !aligned16(dwk) || !aligned16(dwv))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_bwd_onthefly: tensors must be 16-byte aligned");
  if (!mult8(q_sb) || !mult8(q_sh) || !mult8(q_ss) || !mult8(k_sb) || !mult8(k_ss) || !mult8(k_sh) ||
      !mult8(v_sb) || !mult8(v_ss) || !mult8(v_sh) || !mult8(w_sh) || !mult8(w_si) || !mult8(o_sb) ||
      !mult8(o_sh) || !mult8(o_ss) || !mult8(do_sb) || !mult8(do_sh) || !mult8(do_ss) || !mult8(dk_sb) ||
      !mult8(dk_ss) || !mult8(dk_sh))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_bwd_onthefly: strides must be multiples of 8 elements");
  if (q_ss < 0 || do_ss < 0 || k_ss < 0 || v_ss < 0 || q_ss >= kOtfBwdMaxRowStride || do_ss >= kOtfBwdMaxRowStride ||
      k_ss >= kOtfBwdMaxRowStride || v_ss >= kOtfBwdMaxRowStride)
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_bwd_onthefly: row strides of q, dout, k and v must be in [0, 2^24)");
  if (Sq > kOtfBwdMaxSeq || Sk > kOtfBwdMaxSeq)
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_bwd_onthefly: Sq and Sk must be at most 2^24");
  if (B == 0 || H == 0) return DMLA_OK;
  if (Sq == 0 || Sk == 0)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_bwd_onthefly: Sq and Sk must be > 0 (zero the gradients instead)");
  const OtfBwdPlan pl = make_otf_plan(B, H, Sq, Sk);
  if (workspace_bytes < (int64_t)pl.bytes || !workspace)
    return fail(DMLA_ERR_WORKSPACE, "dmla_bwd_onthefly: workspace of %lld bytes needed, got %lld",
                (long long)pl.bytes, (long long)workspace_bytes);
  if (!aligned16(workspace)) return fail(DMLA_ERR_INVALID_ARG, "dmla_bwd_onthefly: workspace must be 16-byte aligned");
  const int64_t grid_kv = B * H * (pl.Skp / kKeyBlk), grid_q = B * H * (pl.Sqp / kRowBlk);
  if (grid_kv > 0x7fffffff || grid_q > 0x7fffffff || B * H > 65535 || 2 * B > 65535)
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_bwd_onthefly: grid too large");

  OtfBwdParams p = {};
  p.q = static_cast<const bf16*>(q);
  p.k = static_cast<const bf16*>(k);
  p.v = static_cast<const bf16*>(v);
  p.wk = static_cast<const bf16*>(wk);
  p.wv = static_cast<const bf16*>(wv);
  p.o = static_cast<const bf16*>(o);
  p.dout = static_cast<const bf16*>(dout);
  p.m = m;
  p.l = l;
  p.dq = dq;
  p.dk = dk;
  p.dv = dv;
  p.dwk = dwk;
  p.dwv = dwv;
  p.dq_fp32 = dq_fp32 ? 1 : 0;
  p.dkv_fp32 = dkv_fp32 ? 1 : 0;
  p.dw_fp32 = dw_fp32 ? 1 : 0;
  p.q_sb = q_sb; p.q_sh = q_sh; p.q_ss = q_ss;
  p.k_sb = k_sb; p.k_ss = k_ss; p.k_sh = k_sh;
  p.v_sb = v_sb; p.v_ss = v_ss; p.v_sh = v_sh;
  p.w_sh = w_sh; p.w_si = w_si;
  p.o_sb = o_sb; p.o_sh = o_sh; p.o_ss = o_ss;
  p.do_sb = do_sb; p.do_sh = do_sh; p.do_ss = do_ss;
  p.dq_sb = dq_sb; p.dq_sh = dq_sh; p.dq_ss = dq_ss;
  p.dk_sb = dk_sb; p.dk_ss = dk_ss; p.dk_sh = dk_sh;
  p.dw_sh = dw_sh; p.dw_si = dw_si;
  p.B = (int)B; p.H = (int)H; p.Sq = (int)Sq; p.Sk = (int)Sk;
  p.causal = causal ? 1 : 0;
  p.Sqp = pl.Sqp; p.Skp = pl.Skp; p.n_sc = pl.n_sc;
  p.scale = softmax_scale;
  p.scale_log2 = softmax_scale * kLog2e;
  char* ws = static_cast<char*>(workspace);
  p.lse2 = reinterpret_cast<float*>(ws + pl.off_lse2);
  p.nd = reinterpret_cast<float*>(ws + pl.off_nd);
  p.klat = reinterpret_cast<_Float16*>(ws + pl.off_klat);
  p.vlat = reinterpret_cast<_Float16*>(ws + pl.off_vlat);
  p.dxlat = reinterpret_cast<bf16*>(ws + pl.off_dx);
  p.wpart = reinterpret_cast<float*>(ws + pl.off_wpart);
  p.wt = reinterpret_cast<bf16*>(ws + pl.off_wt);
  p.bmax = reinterpret_cast<float*>(ws + pl.off_bmax);
  p.gmax = reinterpret_cast<unsigned*>(ws + pl.off_gmax);

  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(otf_bwd_prep_kernel, dim3((unsigned)(pl.Sqp / kRowBlk), (unsigned)(B * H)), dim3(256), 0, s, p);
  hipLaunchKernelGGL(otf_bwd_wt_kernel, dim3((unsigned)H, 2), dim3(256), 0, s, p);
  hipLaunchKernelGGL(otf_bwd_dkdv_kernel, dim3((unsigned)grid_kv), dim3(256), 0, s, p);
  hipLaunchKernelGGL(otf_bwd_dq_kernel, dim3((unsigned)grid_q), dim3(256), 0, s, p);
  hipLaunchKernelGGL(otf_bwd_wgrad_kernel, dim3((unsigned)pl.n_sc, (unsigned)H, (unsigned)(2 * B)), dim3(256), 0, s, p);
  hipLaunchKernelGGL(otf_bwd_wreduce_kernel, dim3(kIn * kLat / 256, (unsigned)H, 2), dim3(256), 0, s, p);
  return check_launch("dmla_bwd_onthefly");
}
