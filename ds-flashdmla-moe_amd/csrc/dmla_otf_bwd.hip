// On-the-fly DMLA backward for gfx950: gradients of
//     O[b,h] = softmax(scale * Q[b,h] K_lat[b,h]^T (+ causal mask)) V_lat[b,h],
//     K_lat = K[b,:,h,:] WK[h],  V_lat = V[b,:,h,:] WV[h]        (README.md:14)
// with respect to Q, K, V, WK and WV, from the forward's saved row statistics m and l
// (README.md:12).  The attention part is the intended FA2 backward of
// csrc/attention/fa2_bwd.cu:198-310 (D = rowsum(dO * O), dS = P * (dP - D), dV_lat = P^T dO,
// dK_lat = scale dS^T Q, dQ = scale dS K_lat) with the softmax scale applied to dQ and dK_lat;
// the projections then give
//     dK = dK_lat WK^T,  dWK[h] = sum_{b,s} K[b,s,h,:]^T dK_lat[b,h,s,:]   (same for V / WV).
// The reference has no on-the-fly backward at all (WK / WV are learnable per README.md:14).
//
// Seven kernels run in order on one stream, all deterministic (no atomics):
//   otf_bwd_prep_kernel    per query row: Q and dO as fp16, lse2 = (m + ln l) log2(e), D;
//   otf_bwd_wt_kernel      WK^T and WV^T;
//   otf_bwd_proj_kernel    K_lat and V_lat as fp16 (the forward's projection products);
//   otf_bwd_dkdv_kernel    per 128 keys: dK_lat, dV_lat over the rows that see them;
//   otf_bwd_dq_kernel      per 128 rows: dQ over the keys they see (S and dP recomputed);
//   otf_bwd_wgrad_kernel   per (tensor, head, 1024 keys): dK / dV and a dWK / dWV partial;
//   otf_bwd_wreduce_kernel sums the partials of each head in a fixed order.
//
// Every product runs on v_mfma_f32_16x16x32_f16 with fp32 accumulation: Q, dO, K, V and the
// weights are converted to fp16 exactly (bf16's significand fits fp16's; |x| <= 65504), and the
// rounded intermediates (K_lat, V_lat, P, dS, dK_lat, dV_lat) are fp16.  V_lat equals the
// forward's (same operands, same order, same rounding); K_lat is the forward's fp32 projection
// rounded once to fp16, where the forward keeps a bf16 hi + lo pair for its scores, so the
// recomputed P carries the fp16 rounding of the scores (~2^-12 relative) against the forward's
// exact statistics -- well inside the gradients' tolerance.  The one layout trick used
// throughout: an MFMA C tile (lane l holds rows 4(l/16)+i, column l%16) of two 16-row blocks is
// the B operand of a product contracting over those 32 rows when the k-index runs over rows
// {4g+i} then {16+4g+i} (g = l/16); ds_read_b64_tr_b16 on a row-major tile hands the A operand
// exactly that row order (two reads, rows 4g.. and 16+4g..).  So P and dS never go through LDS.
#include <type_traits>

#include "dmla_common.h"
#include "dmla_host.h"

namespace dmla {
namespace {

constexpr int kIn = 128;                // raw K / V dims per head
constexpr int kLat = 64;                // latent dims (Q, K_lat, V_lat, O)
constexpr int kRowBlk = 128;            // dQ workgroup rows; Q rows are padded to a multiple
constexpr int kKeyBlk = 128;            // dK/dV workgroup keys; keys are padded to a multiple
constexpr int kChunk = 1024;            // keys per weight-gradient workgroup
constexpr int kTile = 32 * kLat * 2;    // one 32-row fp16 tile of 64 columns (4 KB)
constexpr int kStage = 4 * kTile;       // 64 rows of two tensors (16 KB)
constexpr int kXTile = 32 * kIn * 2;    // one 32-key fp16 tile of 128 raw columns (8 KB)
constexpr int kWgStage = 2 * kXTile + 2 * kTile;   // 64 keys: raw X and dX_lat (24 KB)

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
  bf16* dq;
  bf16* dk;
  bf16* dv;
  void* dwk;            // bf16, or fp32 when dw_fp32
  void* dwv;
  int dw_fp32;
  int64_t q_sb, q_sh, q_ss, k_sb, k_ss, k_sh, v_sb, v_ss, v_sh, w_sh, w_si;
  int64_t o_sb, o_sh, o_ss, do_sb, do_sh, do_ss;
  int64_t dq_sb, dq_sh, dq_ss, dk_sb, dk_ss, dk_sh, dw_sh, dw_si;
  int B, H, Sq, Sk, causal;
  int Sqp, Skp;          // rows / keys padded to multiples of 128
  int n_sc;              // 1024-key chunks per batch element (weight gradients)
  float scale, scale_log2;
  _Float16* q16;         // [B*H][Sqp][64]; padding rows zero
  _Float16* do16;        // [B*H][Sqp][64]
  float* lse2;           // [B*H][Sqp]: (m + ln l) log2(e); padding and empty rows +inf
  float* nd;             // [B*H][Sqp]: -D = -rowsum(dO * O); padding rows 0
  _Float16* klat;        // [B*H][Skp][64]; padding keys zero
  _Float16* vlat;
  _Float16* dklat;       // [B*H][Skp][64]; padding keys zero
  _Float16* dvlat;
  float* wpart;          // [2][H][B*n_sc][128][64] fp32 partial weight gradients
  bf16* wt;              // [2][H][64][128]: WK^T, WV^T
};

__device__ __forceinline__ f16x8 to_f16(const bf16x8& x) {
  return bf16_to_f16(__builtin_shufflevector(x, x, 0, 1, 2, 3), __builtin_shufflevector(x, x, 4, 5, 6, 7));
}
__device__ __forceinline__ f16x8 lds_f16x8(const DMLA_LDS char* p) { return *reinterpret_cast<const DMLA_LDS f16x8*>(p); }
// A column operand (k along tile rows) of a 32-row tile: rows 4g..4g+3 then 16+4g..16+4g+3.
__device__ __forceinline__ f16x8 lds_col_operand(const DMLA_LDS char* tile, int lane, int cb) {
  const f16x4 a = lds_read_tr16_f16(reinterpret_cast<const DMLA_LDS f16x4*>(tile + col_operand_off(lane, cb, 0)));
  const f16x4 b = lds_read_tr16_f16(reinterpret_cast<const DMLA_LDS f16x4*>(tile + col_operand_off(lane, cb, 1)));
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Copies 64 rows of two [rows][64] fp16 arrays (rows row0 .. row0+63 of each) into a stage:
// [x0 rows 0-31, x0 rows 32-63, x1 rows 0-31, x1 rows 32-63], each a 32-row tile in the
// tile_chunk_off layout.  Sixteen 1 KB wave copies, four per wave; lane l of copy `part` lands
// at byte 16 l of that 1 KB, i.e. tile row 8 part + l/8, physical chunk l%8.
__device__ __forceinline__ void stage_pair(const _Float16* x0, const _Float16* x1, int row0, unsigned lds_stage,
                                           int wave, int lane) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int n = 4 * wave + c;                  // 0 .. 15
    const int x = n >> 3, t = (n >> 2) & 1, part = n & 3;
    const int row = 8 * part + (lane >> 3);
    const int lc = (lane & 7) ^ swz(row & 15);   // logical chunk stored at this physical slot
    const unsigned voff = 2u * (unsigned)((row0 + 32 * t + row) * kLat + 8 * lc);
    dma16(x ? x1 : x0, voff, lds_stage + (2 * x + t) * kTile + part * 1024);
  }
}

// ---------------------------------------------------------------------------------------------
// Prep: one thread per 8 dims of a row; 32 rows per 256-thread block, grid (Sqp / 32, B*H).
__global__ void __launch_bounds__(256) otf_bwd_prep_kernel(OtfBwdParams p) {
  const int bh = blockIdx.y;
  const int b = bh / p.H, h = bh % p.H;
  const int r = blockIdx.x * 32 + (threadIdx.x >> 3), c = threadIdx.x & 7;
  f16x8 q16 = {}, d16 = {};
  float dsum = 0.f;
  if (r < p.Sq) {
    const bf16x8 qv = *reinterpret_cast<const bf16x8*>(p.q + b * p.q_sb + h * p.q_sh + (int64_t)r * p.q_ss + 8 * c);
    const bf16x8 ov = *reinterpret_cast<const bf16x8*>(p.o + b * p.o_sb + h * p.o_sh + (int64_t)r * p.o_ss + 8 * c);
    const bf16x8 dv = *reinterpret_cast<const bf16x8*>(p.dout + b * p.do_sb + h * p.do_sh + (int64_t)r * p.do_ss + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) dsum += (float)dv[e] * (float)ov[e];
    q16 = to_f16(qv);
    d16 = to_f16(dv);
  }
  const size_t out = ((size_t)bh * p.Sqp + r) * kLat + 8 * c;
  *reinterpret_cast<f16x8*>(p.q16 + out) = q16;
  *reinterpret_cast<f16x8*>(p.do16 + out) = d16;
  dsum += __shfl_xor(dsum, 1);
  dsum += __shfl_xor(dsum, 2);
  dsum += __shfl_xor(dsum, 4);
  if (c == 0) {
    float lse = __builtin_inff();   // P = 0 for padding rows and rows without keys
    if (r < p.Sq) {
      const int64_t idx = (int64_t)bh * p.Sq + r;
      const float lv = p.l[idx];
      if (lv > 0.f) lse = p.m[idx] * kLog2e + __builtin_log2f(lv);
    }
    p.lse2[(size_t)bh * p.Sqp + r] = lse;
    p.nd[(size_t)bh * p.Sqp + r] = -dsum;
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
}

// Projection as the forward computes it, rounded to fp16 as there: X_lat^T = W^T X^T with
// A = W^T rows and B = raw X rows (K: the forward's own operand order; V: the forward's
// V_lat = V WV with A and B swapped, which v_mfma_f32_16x16x32_bf16 computes bit for bit as
// the transpose), four k-steps of 32 input dims each.  Block = 256 keys of one (b, h); waves
// 0-1 project K, waves 2-3 V, each taking every other 16-key block with the next block's rows
// loaded while the current one is multiplied.  Grid (Skp / 256 rounded up, H, B).
__global__ void __launch_bounds__(256) otf_bwd_proj_kernel(OtfBwdParams p) {
  // Heads fastest in the grid: workgroups issued together read neighbouring 256-byte pieces of
  // the same [B, S, H, 128] rows (the 16 key blocks of one head lie 8 KB apart per key).
  const int h = blockIdx.x, b = blockIdx.z, bh = b * p.H + h;
  const int wave = uniform(threadIdx.x >> 6), lane = lane_id(), l16 = lane & 15, g = lane >> 4;
  const int x = wave >> 1;
  bf16x8 wa[4][4];   // [db][ks]: W^T row 16 db + l16, input dims 32 ks + 8 g ..
  {
    const bf16* wt = p.wt + ((size_t)x * p.H + h) * (kLat * kIn) + l16 * kIn + 8 * g;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) wa[db][ks] = *reinterpret_cast<const bf16x8*>(wt + 16 * db * kIn + 32 * ks);
  }
  const bf16* src = x ? p.v + b * p.v_sb + h * p.v_sh : p.k + b * p.k_sb + h * p.k_sh;
  const int64_t ss = x ? p.v_ss : p.k_ss;
  _Float16* dst = (x ? p.vlat : p.klat) + (size_t)bh * p.Skp * kLat;
  const int key_base = blockIdx.y * 256;
  const int n_kb = min(16, (p.Skp - key_base) / 16);
  bf16x8 xr[4];
  auto load = [&](int kb) {
    const int gk = min(key_base + 16 * kb + l16, p.Sk - 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) xr[ks] = *reinterpret_cast<const bf16x8*>(src + (int64_t)gk * ss + 32 * ks + 8 * g);
  };
  int kb = wave & 1;
  if (kb < n_kb) load(kb);
  for (; kb < n_kb; kb += 2) {
    bf16x8 cur[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) cur[ks] = xr[ks];
    if (kb + 2 < n_kb) load(kb + 2);
    const int key = key_base + 16 * kb + l16;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) c = mfma_bf16(wa[db][ks], cur[ks], c);   // X_lat^T[dim 16 db + 4 g + i][key]
      f16x4 o;
      // K_lat is stored multiplied by scale log2(e): S then comes out in log2 units and the
      // score accumulators can start at -lse2 (dQ takes ln 2 instead of the scale).
      const float mul = x ? 1.f : p.scale_log2;
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = key < p.Sk ? (_Float16)(c[i] * mul) : (_Float16)0.f;
      *reinterpret_cast<f16x4*>(dst + (size_t)key * kLat + 16 * db + 4 * g) = o;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// dK_lat / dV_lat: block = 128 keys of one (b, h), wave w owns keys k0 = 128 kblk + 32 w .. +31.
// Rows stream in stages of 64 (Q and dO as fp16, copied global -> LDS one stage ahead), from
// the first row that sees any of the block's keys.  Per 32-row sub-tile and wave:
//   S  = Q K_lat^T, dP = dO V_lat^T    (A = Q / dO rows from LDS, B = K_lat / V_lat in registers)
//   P  = exp2(S scale log2e - lse2), dS = P (dP - D)   (K_lat stored times scale log2e; the S
//        accumulators start at -lse2, so the product is the exp2 argument)
//   dV_lat^T += dO^T P, dK_lat^T += Q^T dS   (A = dO^T / Q^T by transposed reads; B = P / dS
//                                           straight from the C tiles of S and dP)
// Grid: key blocks heavy first (block 0 sees every row under the causal mask).
__global__ void __launch_bounds__(256, 2) otf_bwd_dkdv_kernel(OtfBwdParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[2 * kStage];
  DMLA_LDS char* lds = (DMLA_LDS char*)smem;
  const int wave = uniform(threadIdx.x >> 6), lane = lane_id(), l16 = lane & 15, g = lane >> 4;
  const int BH = p.B * p.H;
  const int bh = (int)blockIdx.x % BH, kblk = (int)blockIdx.x / BH;
  const int off = p.Sk - p.Sq;
  const int k0 = kblk * kKeyBlk + 32 * wave;
  f16x8 kreg[2][2], vreg[2][2];   // [kb][ks]: X_lat[k0 + 16 kb + l16][32 ks + 8 g ..]
  {
    const size_t base = ((size_t)bh * p.Skp + k0 + l16) * kLat + 8 * g;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        kreg[kb][ks] = *reinterpret_cast<const f16x8*>(p.klat + base + 16 * kb * kLat + 32 * ks);
        vreg[kb][ks] = *reinterpret_cast<const f16x8*>(p.vlat + base + 16 * kb * kLat + 32 * ks);
      }
  }
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
  const _Float16* qsrc = p.q16 + (size_t)bh * p.Sqp * kLat;
  const _Float16* dsrc = p.do16 + (size_t)bh * p.Sqp * kLat;
  const float* lse2 = p.lse2 + (size_t)bh * p.Sqp;
  const float* nd = p.nd + (size_t)bh * p.Sqp;
  const unsigned lbase = lds_addr(lds);

  // One 32-row sub-tile; kMask applies the causal / key-range mask (only sub-tiles that reach
  // past some pair's limit need it), so the common case is straight-line code.
  // dP - D comes straight out of the dP product: its accumulator starts at -D of the row.
  auto subtile = [&](const DMLA_LDS char* qt, const DMLA_LDS char* dt, int r0, const f32x4 (&ls)[2],
                     const f32x4 (&ndv)[2], auto mask_tag) {
    constexpr bool kMask = decltype(mask_tag)::value;
    f32x4 sacc[2][2], dpacc[2][2];   // [rb][kb]: rows 16 rb + 4 g + i, key 16 kb + l16
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const f16x8 qa0 = lds_f16x8(qt + row_operand_off(lane, rb, 0));
      const f16x8 qa1 = lds_f16x8(qt + row_operand_off(lane, rb, 1));
      const f16x8 oa0 = lds_f16x8(dt + row_operand_off(lane, rb, 0));
      const f16x8 oa1 = lds_f16x8(dt + row_operand_off(lane, rb, 1));
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        sacc[rb][kb] = mfma_f16(qa0, kreg[kb][0], -ls[rb]);   // S log2(e) scale - lse2
        sacc[rb][kb] = mfma_f16(qa1, kreg[kb][1], sacc[rb][kb]);
        dpacc[rb][kb] = mfma_f16(oa0, vreg[kb][0], ndv[rb]);
        dpacc[rb][kb] = mfma_f16(oa1, vreg[kb][1], dpacc[rb][kb]);
      }
    }
    f16x8 pb[2], dsb[2];   // [kb]: B operands, slot 4 rb + i = row 16 rb + 4 g + i
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float pv = fast_exp2(sacc[rb][kb][i]);
          if constexpr (kMask) {
            const int row = r0 + 16 * rb + 4 * g + i, key = k0 + 16 * kb + l16;
            const int lim = p.causal ? min(row + off, p.Sk - 1) : p.Sk - 1;
            pv = key > lim ? 0.f : pv;
          }
          pb[kb][4 * rb + i] = (_Float16)pv;
          dsb[kb][4 * rb + i] = (_Float16)(pv * dpacc[rb][kb][i]);
        }
    }
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const f16x8 ot = lds_col_operand(dt, lane, db);   // dO^T[dim 16 db + l16][rows]
      const f16x8 qtt = lds_col_operand(qt, lane, db);  // Q^T
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        dvt[db][kb] = mfma_f16(ot, pb[kb], dvt[db][kb]);
        dkt[db][kb] = mfma_f16(qtt, dsb[kb], dkt[db][kb]);
      }
    }
  };

  // One stage; the buffer index is a compile-time constant (the loop below is unrolled by two)
  // so that every LDS address is a lane offset plus an instruction immediate.
  auto stage_iter = [&](int s, auto buf_tag) {
    constexpr int kBuf = decltype(buf_tag)::value;
    wait_vmem();
    __syncthreads();   // stage s complete; every wave is done with stage s-1
    // lse2 and -D of rows r0 + 16 rb + 4 g + i, loaded before the next stage's copies so that
    // waiting for them does not wait for the copies.
    f32x4 ls[2][2], ndv[2][2];   // [t][rb]
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        const int r = rs0 + 64 * s + 32 * t + 16 * rb + 4 * g;
        ls[t][rb] = *reinterpret_cast<const f32x4*>(lse2 + r);
        ndv[t][rb] = *reinterpret_cast<const f32x4*>(nd + r);
      }
    if (s + 1 < n_st) stage_pair(qsrc, dsrc, rs0 + 64 * (s + 1), lbase + (1 - kBuf) * kStage, wave, lane);
    const DMLA_LDS char* st = lds + kBuf * kStage;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int r0 = rs0 + 64 * s + 32 * t;
      if (r0 >= p.Sq || (p.causal && k0 > r0 + 31 + off)) continue;   // padding only / all masked
      if (k0 + 31 >= p.Sk || (p.causal && k0 + 31 > r0 + off))
        subtile(st + t * kTile, st + (2 + t) * kTile, r0, ls[t], ndv[t], std::true_type{});
      else
        subtile(st + t * kTile, st + (2 + t) * kTile, r0, ls[t], ndv[t], std::false_type{});
    }
  };
  if (n_st > 0) stage_pair(qsrc, dsrc, rs0, lbase, wave, lane);
  for (int s = 0; s < n_st; s += 2) {
    stage_iter(s, std::integral_constant<int, 0>{});
    if (s + 1 < n_st) stage_iter(s + 1, std::integral_constant<int, 1>{});
  }
  // dK_lat = scale dS^T Q and dV_lat = P^T dO as fp16 rows (keys past Sk hold zeros: P = 0 there)
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const size_t row = ((size_t)bh * p.Skp + k0 + 16 * kb + l16) * kLat;
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      f16x4 a, c;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = (_Float16)(dkt[db][kb][i] * p.scale);
        c[i] = (_Float16)dvt[db][kb][i];
      }
      *reinterpret_cast<f16x4*>(p.dklat + row + 16 * db + 4 * g) = a;
      *reinterpret_cast<f16x4*>(p.dvlat + row + 16 * db + 4 * g) = c;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// dQ: block = 128 rows of one (b, h), wave w owns rows r0 = 128 rblk + 32 w .. +31.  Keys stream
// in stages of 64 (K_lat and V_lat, copied one stage ahead) up to the last key any row sees.
// Per 32-key sub-tile and wave:
//   S^T = K_lat Q^T, dP^T = V_lat dO^T   (A = K_lat / V_lat rows from LDS, B = Q / dO in registers)
//   dS^T = P^T (dP^T - D)
//   dQ += dS K_lat                        (A = dS straight from the C tiles of S^T; B = K_lat by
//                                          transposed reads, keys in the same order)
// Grid: row blocks heavy (last) first.
__global__ void __launch_bounds__(256, 2) otf_bwd_dq_kernel(OtfBwdParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[2 * kStage];
  DMLA_LDS char* lds = (DMLA_LDS char*)smem;
  const int wave = uniform(threadIdx.x >> 6), lane = lane_id(), l16 = lane & 15, g = lane >> 4;
  const int BH = p.B * p.H;
  const int bh = (int)blockIdx.x % BH;
  const int rblk = p.Sqp / kRowBlk - 1 - (int)blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int off = p.Sk - p.Sq;
  const int r0 = rblk * kRowBlk + 32 * wave;
  f16x8 qreg[2][2], oreg[2][2];   // [rb][ks]: X16[r0 + 16 rb + l16][32 ks + 8 g ..]
  float lse[2];
  f32x4 ndv[2];   // -D of row r0 + 16 rb + l16 in all four elements: the dP^T accumulator start
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const size_t base = ((size_t)bh * p.Sqp + r0 + 16 * rb + l16) * kLat + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      qreg[rb][ks] = *reinterpret_cast<const f16x8*>(p.q16 + base + 32 * ks);
      oreg[rb][ks] = *reinterpret_cast<const f16x8*>(p.do16 + base + 32 * ks);
    }
    lse[rb] = p.lse2[(size_t)bh * p.Sqp + r0 + 16 * rb + l16];
    const float n = p.nd[(size_t)bh * p.Sqp + r0 + 16 * rb + l16];
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
    for (int db = 0; db < 4; ++db) {
      const f16x8 kb_t = lds_col_operand(kt, lane, db);   // K_lat[keys][dim 16 db + l16]
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) dq[rb][db] = mfma_f16(dsa[rb], kb_t, dq[rb][db]);
    }
  };

  // Unrolled by two stages so that the buffer offset is an instruction immediate.
  auto stage_iter = [&](int s, auto buf_tag) {
    constexpr int kBuf = decltype(buf_tag)::value;
    wait_vmem();
    __syncthreads();
    if (s + 1 < n_st) stage_pair(ksrc, vsrc, 64 * (s + 1), lbase + (1 - kBuf) * kStage, wave, lane);
    const DMLA_LDS char* st = lds + kBuf * kStage;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int c0 = 64 * s + 32 * t;
      if (c0 >= key_end || (p.causal && c0 > r0 + 31 + off)) continue;
      if (c0 + 31 >= p.Sk || (p.causal && c0 + 31 > r0 + off))
        subtile(st + t * kTile, st + (2 + t) * kTile, c0, std::true_type{});
      else
        subtile(st + t * kTile, st + (2 + t) * kTile, c0, std::false_type{});
    }
  };
  if (n_st > 0) stage_pair(ksrc, vsrc, 0, lbase, wave, lane);
  for (int s = 0; s < n_st; s += 2) {
    stage_iter(s, std::integral_constant<int, 0>{});
    if (s + 1 < n_st) stage_iter(s + 1, std::integral_constant<int, 1>{});
  }
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = r0 + 16 * rb + 4 * g + i;
      if (row >= p.Sq) continue;
      bf16* out = p.dq + b * p.dq_sb + h * p.dq_sh + (int64_t)row * p.dq_ss + l16;
#pragma unroll
      for (int db = 0; db < 4; ++db) out[16 * db] = (bf16)(dq[rb][db][i] * kLn2);   // scale / (scale log2 e)
    }
}

// ---------------------------------------------------------------------------------------------
// Weight side: block = (tensor x in {K, V}, head h, batch b, chunk c of 1024 keys), grid
// (n_sc, H, 2 B).  Per 64-key block (raw X as fp16 through registers, dX_lat copied directly,
// both one block ahead):
//   dX^T[in][key] = W[in][:] dX_lat^T       wave w: keys 16 w .. +15 (A = W rows in registers,
//                                           B = dX_lat rows from LDS); written as bf16 rows of dX
//   dW[in][dim]  += X^T[in][key] dX_lat     wave w: input dims 32 w .. +31 (both operands by
//                                           transposed reads, keys in the same order)
// The fp32 dW partial of the chunk goes to wpart; otf_bwd_wreduce_kernel sums the chunks.
__global__ void __launch_bounds__(256) otf_bwd_wgrad_kernel(OtfBwdParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[2 * kWgStage];
  DMLA_LDS char* lds = (DMLA_LDS char*)smem;
  const int wave = uniform(threadIdx.x >> 6), lane = lane_id(), l16 = lane & 15, g = lane >> 4;
  const int c = blockIdx.x, h = blockIdx.y, x = blockIdx.z & 1, b = blockIdx.z >> 1;
  const int bh = b * p.H + h;
  const bf16* X = x ? p.v + b * p.v_sb + h * p.v_sh : p.k + b * p.k_sb + h * p.k_sh;
  const int64_t x_ss = x ? p.v_ss : p.k_ss;
  const bf16* W = (x ? p.wv : p.wk) + h * p.w_sh;
  const _Float16* dxl = (x ? p.dvlat : p.dklat) + (size_t)bh * p.Skp * kLat;
  bf16* dX = (x ? p.dv : p.dk) + b * p.dk_sb + h * p.dk_sh;
  const int key_lo = c * kChunk, key_hi = min(p.Sk, key_lo + kChunk);
  const int n_blk = (key_hi - key_lo + 63) / 64;
  const unsigned lbase = lds_addr(lds);

  f16x8 wa[8][2];   // [ib][ks]: W[16 ib + l16][32 ks + 8 g ..]
#pragma unroll
  for (int ib = 0; ib < 8; ++ib)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      wa[ib][ks] = to_f16(*reinterpret_cast<const bf16x8*>(W + (16 * ib + l16) * p.w_si + 32 * ks + 8 * g));
  f32x4 dw[2][4];   // [ib - 2 w][db]: dW[16 ib + 4 g + i][16 db + l16]
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int db = 0; db < 4; ++db) dw[a][db] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Raw X block: 64 keys x 16 chunks of 16 B, four chunks per thread (q = tid + 256 j).
  bf16x8 xr[4];
  auto load_x = [&](int blk) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = threadIdx.x + 256 * j;
      const int gk = min(key_lo + 64 * blk + (q >> 4), p.Sk - 1);
      xr[j] = *reinterpret_cast<const bf16x8*>(X + (int64_t)gk * x_ss + 8 * (q & 15));
    }
  };
  auto put_x = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int q = threadIdx.x + 256 * j;
      const int kk = q >> 4, ch = q & 15;
      *reinterpret_cast<DMLA_LDS f16x8*>(lds + buf * kWgStage + (kk >> 5) * kXTile + tile_chunk_off(kk & 31, ch)) =
          to_f16(xr[j]);
    }
  };
  // dX_lat block: 8 KB as two 32-key tiles, eight 1 KB wave copies, two per wave.
  auto dma_dxl = [&](int blk, int buf) {
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
      const int n = 2 * wave + cc;
      const int t = n >> 2, part = n & 3;
      const int row = 8 * part + (lane >> 3);
      const int lc = (lane & 7) ^ swz(row & 15);
      const unsigned voff = 2u * (unsigned)((key_lo + 64 * blk + 32 * t + row) * kLat + 8 * lc);
      dma16(dxl, voff, lbase + buf * kWgStage + 2 * kXTile + t * kTile + part * 1024);
    }
  };

  if (n_blk > 0) {
    load_x(0);
    dma_dxl(0, 0);
    put_x(0);
  }
  for (int blk = 0; blk < n_blk; ++blk) {
    wait_vmem();
    __syncthreads();   // block blk complete in buffer blk & 1; buffer (blk + 1) & 1 free
    if (blk + 1 < n_blk) {
      load_x(blk + 1);
      dma_dxl(blk + 1, (blk + 1) & 1);
    }
    const DMLA_LDS char* xs = lds + (blk & 1) * kWgStage;
    const DMLA_LDS char* ds = xs + 2 * kXTile;
    // dX^T for keys 16 wave + l16 of the block
    {
      const DMLA_LDS char* dt = ds + (wave >> 1) * kTile;
      const f16x8 b0 = lds_f16x8(dt + row_operand_off(lane, wave & 1, 0));
      const f16x8 b1 = lds_f16x8(dt + row_operand_off(lane, wave & 1, 1));
      const int key = key_lo + 64 * blk + 16 * wave + l16;
#pragma unroll
      for (int ib = 0; ib < 8; ++ib) {
        f32x4 cacc = mfma_f16(wa[ib][0], b0, f32x4{0.f, 0.f, 0.f, 0.f});
        cacc = mfma_f16(wa[ib][1], b1, cacc);    // dX^T[in 16 ib + 4 g + i][key]
        if (key < key_hi) {
          bf16x4 v;
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = (bf16)cacc[i];
          *reinterpret_cast<bf16x4*>(dX + (int64_t)key * p.dk_ss + 16 * ib + 4 * g) = v;
        }
      }
    }
    // dW over the block's 64 keys (two k-steps of 32)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const f16x8 a0 = lds_col_operand(xs + t * kXTile, lane, 2 * wave);
      const f16x8 a1 = lds_col_operand(xs + t * kXTile, lane, 2 * wave + 1);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const f16x8 bm = lds_col_operand(ds + t * kTile, lane, db);
        dw[0][db] = mfma_f16(a0, bm, dw[0][db]);
        dw[1][db] = mfma_f16(a1, bm, dw[1][db]);
      }
    }
    if (blk + 1 < n_blk) put_x((blk + 1) & 1);
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
  size_t off_q16, off_do16, off_lse2, off_nd, off_klat, off_vlat, off_dklat, off_dvlat, off_wpart, off_wt, bytes;
};

OtfBwdPlan make_otf_plan(int64_t B, int64_t H, int64_t Sq, int64_t Sk) {
  OtfBwdPlan pl = {};
  pl.Sqp = (int)((Sq + kRowBlk - 1) / kRowBlk * kRowBlk);
  pl.Skp = (int)((Sk + kKeyBlk - 1) / kKeyBlk * kKeyBlk);
  pl.n_sc = (int)((Sk + kChunk - 1) / kChunk);
  auto up = [](size_t n) { return (n + 255) / 256 * 256; };
  const size_t rows = (size_t)B * H * pl.Sqp, keys = (size_t)B * H * pl.Skp;
  size_t o = 0;
  pl.off_q16 = o;   o += up(rows * kLat * 2);
  pl.off_do16 = o;  o += up(rows * kLat * 2);
  pl.off_lse2 = o;  o += up(rows * sizeof(float));
  pl.off_nd = o;    o += up(rows * sizeof(float));
  pl.off_klat = o;  o += up(keys * kLat * 2);
  pl.off_vlat = o;  o += up(keys * kLat * 2);
  pl.off_dklat = o; o += up(keys * kLat * 2);
  pl.off_dvlat = o; o += up(keys * kLat * 2);
  pl.off_wpart = o; o += up((size_t)2 * H * B * pl.n_sc * kIn * kLat * sizeof(float));
  pl.off_wt = o;    o += up((size_t)2 * H * kIn * kLat * 2);
  pl.bytes = o;
  return pl;
}

constexpr int64_t kOtfBwdMaxSeq = (int64_t)1 << 24;   // keeps the 32-bit copy offsets in range

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
                                 int64_t dk_sh, int64_t dw_sh, int64_t dw_si, int dw_fp32, float softmax_scale,
                                 int causal, void* workspace, int64_t workspace_bytes, dmla_stream_t stream) {
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
  if (grid_kv > 0x7fffffff || grid_q > 0x7fffffff || B * H > 65535 || 2 * B > 65535 || (pl.Skp + 255) / 256 > 65535)
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
  p.dq = static_cast<bf16*>(dq);
  p.dk = static_cast<bf16*>(dk);
  p.dv = static_cast<bf16*>(dv);
  p.dwk = dwk;
  p.dwv = dwv;
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
  p.q16 = reinterpret_cast<_Float16*>(ws + pl.off_q16);
  p.do16 = reinterpret_cast<_Float16*>(ws + pl.off_do16);
  p.lse2 = reinterpret_cast<float*>(ws + pl.off_lse2);
  p.nd = reinterpret_cast<float*>(ws + pl.off_nd);
  p.klat = reinterpret_cast<_Float16*>(ws + pl.off_klat);
  p.vlat = reinterpret_cast<_Float16*>(ws + pl.off_vlat);
  p.dklat = reinterpret_cast<_Float16*>(ws + pl.off_dklat);
  p.dvlat = reinterpret_cast<_Float16*>(ws + pl.off_dvlat);
  p.wpart = reinterpret_cast<float*>(ws + pl.off_wpart);
  p.wt = reinterpret_cast<bf16*>(ws + pl.off_wt);

  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(otf_bwd_prep_kernel, dim3((unsigned)(pl.Sqp / 32), (unsigned)(B * H)), dim3(256), 0, s, p);
  hipLaunchKernelGGL(otf_bwd_wt_kernel, dim3((unsigned)H, 2), dim3(256), 0, s, p);
  hipLaunchKernelGGL(otf_bwd_proj_kernel, dim3((unsigned)H, (unsigned)((pl.Skp + 255) / 256), (unsigned)B), dim3(256),
                     0, s, p);
  hipLaunchKernelGGL(otf_bwd_dkdv_kernel, dim3((unsigned)grid_kv), dim3(256), 0, s, p);
  hipLaunchKernelGGL(otf_bwd_dq_kernel, dim3((unsigned)grid_q), dim3(256), 0, s, p);
  hipLaunchKernelGGL(otf_bwd_wgrad_kernel, dim3((unsigned)pl.n_sc, (unsigned)H, (unsigned)(2 * B)), dim3(256), 0, s, p);
  hipLaunchKernelGGL(otf_bwd_wreduce_kernel, dim3(kIn * kLat / 256, (unsigned)H, 2), dim3(256), 0, s, p);
  return check_launch("dmla_bwd_onthefly");
}
