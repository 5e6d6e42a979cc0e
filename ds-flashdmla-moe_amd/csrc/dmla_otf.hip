// On-the-fly DMLA forward for gfx950: the per-head latent projections K_lat = K WK and
// V_lat = V WV are computed inside the attention kernel (README.md:14, the on-the-fly mode of
// the absent csrc/attention/fa2_dmla_fwd.cu, README.md:45), then
//     O[b,h] = softmax(scale * Q[b,h] K_lat[b,h]^T (+ causal mask)) V_lat[b,h].
// Shapes: Q [B,H,Sq,64], K and V [B,Sk,H,128], WK and WV [H,128,64], O [B,H,Sq,64].
//
// Workgroup = 8 waves on 512 query rows of one (batch, head); wave w owns rows 64w .. +63.
// Key tiles of 64 keys flow through a one-barrier-per-tile pipeline:
//   * the raw K / V rows of tile t+2 are copied global -> LDS (direct copies, two stages);
//   * tile t+1 is projected on MFMA: waves 0-3 compute K_lat^T (16 latent dims each, WK^T in
//     registers), waves 4-7 compute V_lat (WV^T in registers), both written to LDS as fp16 --
//     once per key tile for all 512 rows, so the projection adds 1/4 to the attention MFMAs
//     (a 128-row tile would double them);
//   * tile t is attended: S^T = K_lat Q^T (Q in registers), P in the exp2 domain, O += P V_lat.
// Scores: Q stays in bf16 (exact) and K_lat, multiplied by scale log2(e), is stored as a bf16
// pair hi + lo (hi = bf16(c), lo = bf16(c - hi)), two bf16 MFMAs per k-step: the scores carry
// ~2^-17 relative error, where one fp16 rounding of K_lat (2^-12) moved the row statistics
// m, l by ~1.7e-3 at the benchmark's config 4.  (An fp16 pair does not work: most residuals
// are fp16 subnormals, which the fp16 MFMA loses.)  V_lat and P enter the PV product as fp16,
// rounded from fp32: 3 more significand bits than bf16, which keeps their rounding well inside
// the output tolerance even for rows that see only a few keys.  The score accumulators start
// at -m_ref, so the MFMA hands the softmax its exp2 arguments directly.
// Every MFMA operand read from LDS is a conflict-free 16-byte read: K_lat rows for S^T and a
// V_lat^T tile whose key order matches the C layout of S^T (so P needs no transposition).
//
// Softmax: in log2 units against a per-row reference max m_ref that only moves when a tile's
// max exceeds it by more than kSlack (p <= 2^kSlack in between); moving it rescales O and l.  The exact running max is tracked beside it for the m / l outputs, which
// follow the cache-latent forward's convention (natural-log units).
#include <type_traits>

#include "dmla_common.h"
#include "dmla_host.h"

namespace dmla {
namespace {

constexpr int kDin = 128;          // raw K / V dims per head
constexpr int kDlat = 64;          // latent dims (Q, K_lat, V_lat, O)
constexpr int kOtfWaves = 8;
constexpr int kOtfThreads = 64 * kOtfWaves;
constexpr int kOtfRows = 64 * kOtfWaves;   // 512 query rows per workgroup
constexpr int kOtfKeys = 64;               // keys per tile
constexpr float kSlack = 8.0f;             // log2 slack of the reference max
// LDS: W^T (2 x 64 x 128 bf16), raw K / V stages (2 x 2 x 64 x 128), K_lat hi and V_lat^T
// (2 x 2 x 64 x 64), K_lat lo (2 x 64 x 64)
constexpr int kWBytes = kDlat * kDin * 2;          // 16 KB
constexpr int kRawBytes = kOtfKeys * kDin * 2;     // 16 KB
constexpr int kLatBytes = kOtfKeys * kDlat * 2;    // 8 KB
constexpr int kWOff = 0;                           // [WK^T, WV^T]
constexpr int kRawOff = 2 * kWBytes;               // [stage][K, V]
constexpr int kLatOff = kRawOff + 4 * kRawBytes;   // [buffer][K_lat, V_lat^T]
constexpr int kLatLoOff = kLatOff + 4 * kLatBytes; // [buffer] K_lat lo
constexpr int kOtfLds = kLatLoOff + 2 * kLatBytes; // 144 KB
static_assert(kOtfLds <= 160 * 1024, "LDS budget");

struct OtfParams {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  const bf16* wk;
  const bf16* wv;
  bf16* o;
  float* m;
  float* l;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_ss, k_sh;
  int64_t v_sb, v_ss, v_sh;
  int64_t w_sh, w_si;          // WK / WV: head stride, row (input dim) stride; latent dims contiguous
  int64_t o_sb, o_sh, o_ss;
  int B, H, Sq, Sk, causal;
  float scale_log2;
  int n_qt;                    // ceil(Sq / 512)
};

// Raw tile layout: [key (64)][16 chunks of 16 B], physical chunk = c ^ (key & 15): 16 lanes
// reading one chunk of 16 consecutive keys hit 16 different bank groups.
__device__ __forceinline__ int raw_off(int key, int chunk) { return key * 256 + 16 * (chunk ^ (key & 15)); }
// Latent tiles (K_lat [key][64 dims] and V_lat^T [dim][64 key positions]): 128-byte rows,
// chunk c of row r at c ^ swz(r & 15) as in the cache-latent tiles.
__device__ __forceinline__ int lat_off(int row, int chunk) { return row * 128 + 16 * (chunk ^ swz(row & 15)); }

__global__ void __launch_bounds__(kOtfThreads, 1) otf_fwd_kernel(OtfParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[kOtfLds];
  DMLA_LDS char* lds = (DMLA_LDS char*)smem;
  const int wave = uniform(threadIdx.x >> 6);
  const int lane = lane_id();
  const int l16 = lane & 15, g = lane >> 4;
  const int bh = (int)blockIdx.x % (p.B * p.H);
  const int qt = p.n_qt - 1 - (int)blockIdx.x / (p.B * p.H);   // heaviest (latest) tiles first
  const int b = bh / p.H, h = bh % p.H;
  const int off = p.Sk - p.Sq;
  const int row0 = qt * kOtfRows + 64 * wave;                  // this wave's first query row
  const int last_row = min(p.Sq, qt * kOtfRows + kOtfRows) - 1;
  const int key_end = p.causal ? min(p.Sk, last_row + off + 1) : p.Sk;
  const int n_t = key_end > 0 ? (key_end + kOtfKeys - 1) / kOtfKeys : 0;
  const unsigned lds_base = lds_addr(lds);

  // ---- WK^T and WV^T into LDS ([latent][input] rows of 256 B, same swizzle as raw tiles) ----
  {
    const bf16* wk = p.wk + h * p.w_sh;
    const bf16* wv = p.wv + h * p.w_sh;
    for (int idx = threadIdx.x; idx < kDin * kDlat / 8; idx += kOtfThreads) {
      const int i = idx / (kDlat / 8), j8 = idx % (kDlat / 8);   // input dim i, latent dims 8 j8 ..
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(wk + i * p.w_si + 8 * j8);
      const bf16x8 c = *reinterpret_cast<const bf16x8*>(wv + i * p.w_si + 8 * j8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int j = 8 * j8 + e;
        const int o = raw_off(j, i >> 3) + 2 * (i & 7);
        *reinterpret_cast<DMLA_LDS bf16*>(lds + kWOff + o) = a[e];
        *reinterpret_cast<DMLA_LDS bf16*>(lds + kWOff + kWBytes + o) = c[e];
      }
    }
  }

  // ---- raw K / V tile copies: 16 per tensor (4 keys x 256 B each), 4 per wave ----
  // Wave w copies tensor x = w / 4 (K, then V): copy c covers keys 4n .. 4n+3 with
  // n = 4 (w % 4) + c; lane l -> key 4n + l/16 (= 16 (w % 4) + 4c + g), physical chunk
  // l16 ^ (key % 16) = l16 ^ (4c + g).  The address is a wave-uniform base (the tile's first key
  // plus 4c rows, scalar arithmetic) and a lane offset that does not change from tile to tile
  // (row strides < 2^24 elements keep it below 2^31 bytes).  Computed per copy from 64-bit
  // strides instead, the addresses had cost ~30 quarter-rate integer multiplies per wave and
  // tile.  Only a tile that reaches past Sk takes per-lane addresses, clamped to the last key
  // (those keys are masked).
  const int xw = wave >> 2;
  const bf16* xbase = xw == 0 ? p.k + b * p.k_sb + h * p.k_sh : p.v + b * p.v_sb + h * p.v_sh;
  const int64_t xss = xw == 0 ? p.k_ss : p.v_ss;
  const unsigned raw_lane = (unsigned)((16 * (wave & 3) + g) * xss * 2);
  auto stage_raw = [&](int t, int st) {
    const unsigned ldst = lds_base + kRawOff + (st * 2 + xw) * kRawBytes + (wave & 3) * 4 * 1024;
    if (t * kOtfKeys + kOtfKeys <= p.Sk) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        dma16(xbase + (int64_t)(t * kOtfKeys + 4 * c) * xss, raw_lane + 16u * (unsigned)(l16 ^ (4 * c + g)),
              ldst + c * 1024);
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int key = 16 * (wave & 3) + 4 * c + g;
        const int gk = min(t * kOtfKeys + key, p.Sk - 1);
        dma16_addr(xbase + (int64_t)gk * xss + 8 * (l16 ^ (4 * c + g)), ldst + c * 1024);
      }
    }
  };
  if (n_t > 0) stage_raw(0, 0);
  if (n_t > 1) stage_raw(1, 1);

  // ---- Q rows of this wave as the B operand of S^T: qreg[rb][ks] = Q[row0 + 16 rb + l16][32 ks + 8 g ..]
  bf16x8 qreg[4][2];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const int r = min(row0 + 16 * rb + l16, p.Sq - 1);
    const bf16* qrow = p.q + b * p.q_sb + h * p.q_sh + (int64_t)r * p.q_ss + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      qreg[rb][ks] = *reinterpret_cast<const bf16x8*>(qrow + 32 * ks);
    }
  }
  wait_vmem();
  __syncthreads();   // W^T written, raw tile 0 (and 1) landed

  // Projection operand of this wave: waves 0-3 hold WK^T rows 16 w .. +15 (A operand of
  // K_lat^T), waves 4-7 WV^T rows 16 (w-4) .. (B operand of V_lat); 4 k-steps of 32 input dims.
  const int pdb = wave & 3;
  const bool pk = wave < 4;
  bf16x8 wreg[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    wreg[ks] = *reinterpret_cast<const DMLA_LDS bf16x8*>(lds + kWOff + (pk ? 0 : kWBytes) +
                                                         raw_off(16 * pdb + l16, 4 * ks + g));

  // Project tile t (raw stage st) into latent buffer lb.  One wave-uniform branch for the
  // whole projection (a select per MFMA compiles to a branch around every MFMA).
  auto project = [&](int st, int lb) {
    auto proj = [&](auto is_k) {
      constexpr bool kK = decltype(is_k)::value;
      const DMLA_LDS char* raw = lds + kRawOff + (st * 2 + (kK ? 0 : 1)) * kRawBytes;
      DMLA_LDS char* lat = lds + kLatOff + (lb * 2 + (kK ? 0 : 1)) * kLatBytes;
      // The four key blocks' accumulations run interleaved (k-step outer), so consecutive MFMAs
      // are independent, and each k-step's raw reads go out one k-step ahead.  (Key block by key
      // block, every MFMA waited for the previous one's result and every read was awaited
      // right before its MFMA.)
      f32x4 cacc[4];
      bf16x8 xr[2][4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        cacc[kb] = f32x4{0.f, 0.f, 0.f, 0.f};
        xr[0][kb] = *reinterpret_cast<const DMLA_LDS bf16x8*>(raw + raw_off(16 * kb + l16, g));
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (ks + 1 < 4) {
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
            xr[(ks + 1) & 1][kb] = *reinterpret_cast<const DMLA_LDS bf16x8*>(raw + raw_off(16 * kb + l16, 4 * (ks + 1) + g));
        }
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          if constexpr (kK) cacc[kb] = mfma_bf16(wreg[ks], xr[ks & 1][kb], cacc[kb]);   // K_lat^T[dim 16 pdb + 4g + i][key 16 kb + l16]
          else cacc[kb] = mfma_bf16(xr[ks & 1][kb], wreg[ks], cacc[kb]);                // V_lat[key 16 kb + 4g + i][dim 16 pdb + l16]
        }
      }
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        f32x4 c = cacc[kb];
        if constexpr (kK) {
          // K_lat is stored pre-multiplied by scale log2(e), so that scores come out of the MFMA
          // in log2 units, as hi + lo with hi = bf16(c) and lo = bf16(c - hi):
          // K_lat[key 16 kb + l16][dims 16 pdb + 4g .. +3]
          c *= p.scale_log2;
          bf16x4 hi, lo;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            hi[i] = (bf16)c[i];
            lo[i] = (bf16)(c[i] - (float)hi[i]);
          }
          const int key = 16 * kb + l16;
          const int o = lat_off(key, 2 * pdb + (g >> 1)) + 8 * (g & 1);
          *reinterpret_cast<DMLA_LDS bf16x4*>(lat + o) = hi;
          *reinterpret_cast<DMLA_LDS bf16x4*>(lds + kLatLoOff + lb * kLatBytes + o) = lo;
        } else {
          f16x4 v;
          v[0] = (_Float16)c[0]; v[1] = (_Float16)c[1]; v[2] = (_Float16)c[2]; v[3] = (_Float16)c[3];
          // V_lat^T[dim 16 pdb + l16][position]: keys 4g + i of key block kb sit at positions
          // 32 (kb/2) + 8 g + 4 (kb&1) + i, the key order of the P operand (S^T C layout).
          const int dim = 16 * pdb + l16;
          *reinterpret_cast<DMLA_LDS f16x4*>(lat + lat_off(dim, 4 * (kb >> 1) + g) + 8 * (kb & 1)) = v;
        }
      }
    };
    if (pk) proj(std::true_type{});
    else proj(std::false_type{});
  };

  f32x4 oacc[4][4];   // O[row0 + 16 rb + 4 g + i][16 db + l16]
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int db = 0; db < 4; ++db) oacc[rb][db] = f32x4{0.f, 0.f, 0.f, 0.f};
  float mref[4], mtrue[4], lsum[4];   // per own row 16 rb + l16 (log2 units; lsum lane-partial)
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    mref[rb] = kNegInf;
    mtrue[rb] = kNegInf;
    lsum[rb] = 0.f;
  }
  const int own_pos0 = row0 + l16;   // position of own row 16 rb + l16 is own_pos0 + 16 rb

  if (n_t > 0) project(0, 0);
  for (int t = 0; t < n_t; ++t) {
    wait_vmem();
    __syncthreads();   // latent tile t written, raw tile t+1 landed, raw stage t%2 and latent buffer (t+1)%2 free
    if (t + 1 < n_t) project((t + 1) & 1, (t + 1) & 1);
    // Tile t+2's raw copies go out after the projection: issued straight after the barrier, the
    // 32 KB of copies of all waves queue in the CU's vector-memory path ahead of the work.
    if (t + 2 < n_t) stage_raw(t + 2, t & 1);

    const DMLA_LDS char* klat = lds + kLatOff + ((t & 1) * 2) * kLatBytes;
    const DMLA_LDS char* vlat = klat + kLatBytes;
    const DMLA_LDS char* klo = lds + kLatLoOff + (t & 1) * kLatBytes;
    // x[kb][rb] = S^T in log2 units minus the row's reference: keys 16 kb + 4g + i, row 16 rb +
    // l16.  The MFMA accumulators start at -m_ref (0 while a row has no reference), so x is the
    // exp2 argument as it leaves the matrix core.
    float nmr[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) nmr[rb] = mref[rb] == kNegInf ? 0.f : -mref[rb];
    f32x4 s[4][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int o0 = lat_off(16 * kb + l16, g), o1 = lat_off(16 * kb + l16, 4 + g);
      const bf16x8 k0 = *reinterpret_cast<const DMLA_LDS bf16x8*>(klat + o0);
      const bf16x8 k1 = *reinterpret_cast<const DMLA_LDS bf16x8*>(klat + o1);
      const bf16x8 k0l = *reinterpret_cast<const DMLA_LDS bf16x8*>(klo + o0);
      const bf16x8 k1l = *reinterpret_cast<const DMLA_LDS bf16x8*>(klo + o1);
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        s[kb][rb] = mfma_bf16(k0l, qreg[rb][0], f32x4{nmr[rb], nmr[rb], nmr[rb], nmr[rb]});
        s[kb][rb] = mfma_bf16(k1l, qreg[rb][1], s[kb][rb]);
        s[kb][rb] = mfma_bf16(k0, qreg[rb][0], s[kb][rb]);
        s[kb][rb] = mfma_bf16(k1, qreg[rb][1], s[kb][rb]);
      }
    }
    // Only tiles that reach past some row's limit or past Sk are masked, in a block of their own.
    const int key0 = t * kOtfKeys;
    if (key0 + kOtfKeys > p.Sk || (p.causal && key0 + kOtfKeys - 1 > row0 + off)) {
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        const int lim = p.causal ? min(own_pos0 + 16 * rb + off, p.Sk - 1) : p.Sk - 1;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (key0 + 16 * kb + 4 * g + i > lim) s[kb][rb][i] = kNegInf;
      }
    }
    // Tile max per own row (lane-partial, log2 units), exact running max, and the slack test.
    bool raise = false;
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      float mx = kNegInf;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        mx = fmaxf(mx, fmaxf(fmaxf(s[kb][rb][0], s[kb][rb][1]), fmaxf(s[kb][rb][2], s[kb][rb][3])));
      mx -= nmr[rb];   // the tile's max score in log2 units
      mtrue[rb] = fmaxf(mtrue[rb], mx);
      raise |= mx > mref[rb] + kSlack;
    }
    if (__any(raise)) {
      // Move the reference to the exact row max so far; rescale l and the O rows.
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        const float mrow = group_max(mtrue[rb]);
        const float mnew = fmaxf(mref[rb], mrow);
        const float f = mnew == kNegInf ? 1.f : fast_exp2(mref[rb] - mnew);   // 0 when mref = -inf
        lsum[rb] *= f;
        mref[rb] = mnew;
        // this tile's arguments move to the new reference
        const float dn = (mnew == kNegInf ? 0.f : -mnew) - nmr[rb];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) s[kb][rb] += dn;
        // O rows 16 rb + 4 g + i are own rows of lanes with l16 = 4 g + i.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float fi = __shfl(f, 4 * g + i);
#pragma unroll
          for (int db = 0; db < 4; ++db) oacc[rb][db][i] *= fi;
        }
      }
    }
    // P = exp2(s scale - mref) (0 for masked keys and for rows without a finite reference yet).
    // The row sums add the fp16 P that the PV product multiplies, two per v_dot2c_f32_f16 (fp32
    // accumulation): half the instructions of one fp32 add per score.
    f16x8 pa[4][2];   // A operand of O += P V_lat: [rb][ks], keys of k-step ks in V_lat^T order
    const f16x2 ones = {(_Float16)1.f, (_Float16)1.f};
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float e = fast_exp2(s[kb][rb][i]);
          pa[rb][kb >> 1][4 * (kb & 1) + i] = (_Float16)e;
        }
      }
      float ps = lsum[rb];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          ps = __builtin_amdgcn_fdot2(f16x2{pa[rb][ks][2 * j], pa[rb][ks][2 * j + 1]}, ones, ps, false);
      lsum[rb] = ps;
    }
#pragma unroll
    for (int db = 0; db < 4; ++db) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const f16x8 vb = *reinterpret_cast<const DMLA_LDS f16x8*>(vlat + lat_off(16 * db + l16, 4 * ks + g));
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) oacc[rb][db] = mfma_f16(pa[rb][ks], vb, oacc[rb][db]);
      }
    }
  }

  // ---- epilogue: row sums, statistics, normalised O ----
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const float ltot = group_sum(lsum[rb]);
    const float mrow = group_max(mtrue[rb]);
    const float inv = ltot > 0.f ? 1.f / ltot : 0.f;
    const int r = own_pos0 + 16 * rb;
    if (g == 0 && r < p.Sq && p.m) {
      const int64_t idx = ((int64_t)b * p.H + h) * p.Sq + r;
      const bool any = ltot > 0.f;
      p.m[idx] = any ? mrow * kLn2 : kNegInf;
      p.l[idx] = any ? ltot * fast_exp2(mref[rb] - mrow) : 0.f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float fi = __shfl(inv, 4 * g + i);
      const int ro = row0 + 16 * rb + 4 * g + i;
      if (ro >= p.Sq) continue;
      bf16* orow = p.o + b * p.o_sb + h * p.o_sh + (int64_t)ro * p.o_ss + l16;
#pragma unroll
      for (int db = 0; db < 4; ++db) orow[16 * db] = (bf16)(oacc[rb][db][i] * fi);
    }
  }
}

}  // namespace
}  // namespace dmla

using namespace dmla;

extern "C" int dmla_fwd_onthefly(const void* q, const void* k, const void* v, const void* wk, const void* wv,
                                 void* o, float* m, float* l, int64_t B, int64_t H, int64_t Sq, int64_t Sk,
                                 int64_t d_in, int64_t d_lat, int64_t q_sb, int64_t q_sh, int64_t q_ss,
                                 int64_t k_sb, int64_t k_ss, int64_t k_sh, int64_t v_sb, int64_t v_ss,
                                 int64_t v_sh, int64_t w_sh, int64_t w_si, int64_t o_sb, int64_t o_sh,
                                 int64_t o_ss, float softmax_scale, int causal, dmla_stream_t stream) {
  clear_error();
  if (!q || !k || !v || !wk || !wv || !o) return fail(DMLA_ERR_INVALID_ARG, "dmla_fwd_onthefly: null pointer argument");
  if ((m == nullptr) != (l == nullptr))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_fwd_onthefly: m and l must both be set or both be NULL");
  if (B < 0 || H < 0 || Sq < 0 || Sk < 0) return fail(DMLA_ERR_INVALID_ARG, "dmla_fwd_onthefly: negative size");
  if (d_in != kDin || d_lat != kDlat)
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_fwd_onthefly: only d_in=128, d_lat=64 is compiled (got %lld, %lld)",
                (long long)d_in, (long long)d_lat);
  if (!(softmax_scale > 0.f) || !__builtin_isfinite(softmax_scale))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_fwd_onthefly: softmax_scale must be finite and > 0");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(wk) || !aligned16(wv) || !aligned16(o))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_fwd_onthefly: tensors must be 16-byte aligned");
  if (!mult8(q_sb) || !mult8(q_sh) || !mult8(q_ss) || !mult8(k_sb) || !mult8(k_ss) || !mult8(k_sh) ||
      !mult8(v_sb) || !mult8(v_ss) || !mult8(v_sh) || !mult8(w_sh) || !mult8(w_si))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_fwd_onthefly: input strides must be multiples of 8 elements");
  if (Sq > ((int64_t)1 << 30) || Sk > ((int64_t)1 << 30))
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_fwd_onthefly: size too large");
  if (k_ss < 0 || v_ss < 0 || k_ss >= ((int64_t)1 << 24) || v_ss >= ((int64_t)1 << 24))
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_fwd_onthefly: row strides of k and v must be in [0, 2^24)");
  if (B == 0 || H == 0 || Sq == 0) return DMLA_OK;
  OtfParams p = {};
  p.q = static_cast<const bf16*>(q);
  p.k = static_cast<const bf16*>(k);
  p.v = static_cast<const bf16*>(v);
  p.wk = static_cast<const bf16*>(wk);
  p.wv = static_cast<const bf16*>(wv);
  p.o = static_cast<bf16*>(o);
  p.m = m;
  p.l = l;
  p.q_sb = q_sb; p.q_sh = q_sh; p.q_ss = q_ss;
  p.k_sb = k_sb; p.k_ss = k_ss; p.k_sh = k_sh;
  p.v_sb = v_sb; p.v_ss = v_ss; p.v_sh = v_sh;
  p.w_sh = w_sh; p.w_si = w_si;
  p.o_sb = o_sb; p.o_sh = o_sh; p.o_ss = o_ss;
  p.B = (int)B; p.H = (int)H; p.Sq = (int)Sq; p.Sk = (int)Sk;
  p.causal = causal ? 1 : 0;
  p.scale_log2 = softmax_scale * kLog2e;
  p.n_qt = (int)((Sq + kOtfRows - 1) / kOtfRows);
  const int64_t grid = (int64_t)p.n_qt * B * H;
  if (grid > 0x7fffffff) return fail(DMLA_ERR_UNSUPPORTED, "dmla_fwd_onthefly: grid too large");
  hipLaunchKernelGGL(otf_fwd_kernel, dim3((unsigned)grid), dim3(kOtfThreads), 0, (hipStream_t)stream, p);
  return check_launch("dmla_fwd_onthefly");
}
