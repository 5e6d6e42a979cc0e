// Cache-latent DMLA backward for gfx950 from the saved row statistics m and l.
//
// What it computes is the intended FA2 backward of csrc/attention/fa2_bwd.cu:198-310 (D_i =
// rowsum(dO_i * O_i), dS = P * (dP - D), dV += P^T dO, dK += dS^T Q, dQ += dS K) applied to
// the DMLA cache-latent layout of README.md:12-15: one latent K_lat[b] shared by every head and
// V_lat = K_lat[..., :512], so
//     dQ      = scale * dS K_lat
//     dK_lat  = scale * sum_heads dS^T Q  +  [sum_heads P^T dO, 0]
// with P = exp(scale q.k - m) / l rebuilt from the forward's statistics (README.md:12).
//
// Rows are (query position, head) pairs with the head fastest, as in the forward, so the 16
// heads of a position share one causal key range.  Four kernels run in order on one stream:
//   bwd_prep_kernel       per row: lse2 = (m + ln l) log2(e) and D = rowsum(dO * O);
//   bwd_kt_kernel         K_lat^T in fp16 (32-key tiles of dims x keys, zero padded): dQ's B operand;
//   bwd_dkdv_kernel       per 64-key block, streaming 32-row tiles: S, P, dP and dS' = scale dS
//                         on MFMA, dK_lat accumulated in registers (V fold included), dS'
//                         written once to HBM as fp16 16x16 blocks;
//   bwd_dq_kernel         dQ = dS' K_lat per 128-row tile over its causal key range; its
//                         trailing workgroups sum the dK_lat partials of the row segments in
//                         a fixed order.
// No atomics anywhere: the result is bitwise deterministic.
//
// dS' is stored only where it is written: for each 128-row group, the 64-key blocks that some
// of its rows can see (a prefix of the key blocks; all of them without a causal mask), packed
// group after group through an offset table (bwd_prep_kernel builds it).  When that storage
// would pass DMLA_BWD_DS_CAP_BYTES, the rows are cut into chunks of whole groups, each run
// through dK/dV, dQ and the reduction in turn: a chunk's dQ rows are complete, and dK_lat
// accumulates over the chunks in fp32 (the fp32 output itself, or a workspace buffer when dK_lat
// is bf16), so the workspace stays bounded whatever S is.
//
// Operand precision: S = Q K^T and dP = dO V^T multiply the bf16 inputs as they are.  The
// second-stage products dS'^T Q, P^T dO and dS' K take fp16 operands: P and dS' are rounded to
// fp16 (11-bit significand) instead of bf16 (8-bit), and Q, dO, K_lat are converted to fp16
// exactly.  A key that every later row of every head attends to sums thousands of such terms;
// with bf16 P and dS' that rounding alone costs ~1e-3 of |dK_lat| (2e-2 at the config-5
// magnitudes of ~20), with fp16 an eighth of it -- within a few 1e-3 of exact fp32 operands.
// fp16's narrow exponent range is handled by a power-of-two gradient scale: dS' and dO enter the
// fp16 products times 2^e, with e chosen on the device from the largest |dO| of the call, and
// dq and dK_lat leave times 2^-e, so the relative error does not grow as dO gets small.
#include <cstdlib>

#include "dmla_common.h"
#include "dmla_host.h"

namespace dmla {
namespace {

constexpr int kDqk = 576;
constexpr int kDv = 512;
constexpr int kKeys = 64;                           // keys per dK/dV work block
constexpr int kRows = kTileRows;                    // rows per staged row tile (32)
constexpr int kBwdThreads = 256;                    // 4 waves, one per SIMD
constexpr int kQGroups = kDqk / 64;                 // 9 chunk groups of a Q tile
constexpr int kOGroups = kDv / 64;                  // 8 chunk groups of a dO tile
constexpr int kQBytes = kQGroups * kGroupBytes;     // 36 KB
constexpr int kStageBytes = kQBytes + kOGroups * kGroupBytes;   // 68 KB: Q and dO of one tile
constexpr int kXOffset = 2 * kStageBytes;           // P^T / dS'^T exchange: [2][4 kb][64 lanes][16 B]
constexpr int kDkdvLds = kXOffset + 2 * 4 * 1024 + 4 * 4096;   // 160 KB: stages, exchange, swap
constexpr int kCb = kDqk / 16;                      // 36 column blocks of dK / dQ
constexpr int kPartFloats = kKeys * kDqk;           // one dK partial: 64 keys x 576 fp32
constexpr int kMaxParts = 64;
// dQ kernel: stage = dS' blocks of 128 rows x 32 keys (8 KB) + K^T of 576 dims x 32 keys (36 KB)
constexpr int kDqRows = 128;                        // rows per dQ workgroup (8 waves, two row halves)
constexpr int kDqThreads = 512;
constexpr int kDqDsBytes = 8192;
constexpr int kDqStageBytes = kDqDsBytes + kDqk * 64;
constexpr int kDqStages = 3;
constexpr int kDqLds = kDqStages * kDqStageBytes;   // 132 KB
static_assert(kDkdvLds <= 160 * 1024 && kDqLds <= 160 * 1024, "LDS budget");

struct BwdParams {
  const bf16* q;
  const bf16* k;
  const bf16* o;
  const bf16* dout;
  const float* m;       // [B, H, Sq] contiguous
  const float* l;
  void* dq;
  void* dk;
  int dq_fp32, dk_fp32;
  int dq_rows16;        // bf16 dq whose strides are multiples of 8 elements: stored as whole rows
  int64_t q_sb, q_sh, q_ss, k_sb, k_ss, o_sb, o_sh, o_ss, do_sb, do_sh, do_ss;
  int64_t dq_sb, dq_sh, dq_ss, dk_sb, dk_ss;
  int B, H, Sq, Sk, causal;
  FastDiv hdiv;         // row -> position (rows are position * H + head)
  float scale, scale_log2;
  int R;                // H * Sq rows per batch element
  int n_rt;             // 32-row tiles per batch element, even: 2 * ceil(R / 64)
  int n_kb;             // 64-key blocks: ceil(Sk / 64)
  int n_pairs;          // ceil(n_kb / 2)
  int parts;            // row segments per key-block pair (this chunk)
  int n_items;          // B * n_pairs * parts
  int kt_ld;            // keys K^T covers (zero padded): 64 * n_kb, kt_ld / 32 tiles
  int n_groups;         // 128-row groups: ceil(n_rt / 4)
  int rt_begin, rt_end; // this chunk's row tiles (group aligned)
  int chunk_pairs;      // (group, 64-key block) pairs of this chunk: dS' blocks per batch element
  int chunk, last_chunk;
  float4* rstat;        // [B][32 n_rt] (lse2, D, key limit as int bits, 0); padding rows (+inf, 0, -1)
  int64_t* roff;        // [B][32 n_rt][2]: element offsets of the row's q and dout rows within the batch
                        // element (those of the last row for padding rows)
  _Float16* kt;         // [B][kt_ld / 32][576][32] fp16: K^T in 32-key tiles, each tile contiguous
  int32_t* goff;        // [n_groups + 1]: first (group, key block) pair of each group
  _Float16* ds;         // [B][chunk_pairs][8 row blocks][4 key blocks][256]: fp16 dS' 16x16 blocks, MFMA C order
                        // with lane c's 4 values at slot ds_slot(c)
  float* part;          // [n_items][2][4 kb][36 cb][64 lanes][4]: dK_lat partials in MFMA C order
  float* dk_acc;        // fp32 dK_lat of the chunks so far: [B][Sk][576], or the fp32 output itself
  float* bmax;          // [B][n_rt]: largest |dO| of each bwd_prep workgroup
  unsigned* gmax;       // largest |dO| of the call as fp32 bits (bwd_kt reduces bmax into it)
};

// ---- work split of the dK/dV kernel, shared by the host and the reduction ------------------
// Key block kb needs the row tiles from first_row_tile(kb) on (causal: rows whose position can
// see key 64 kb), rounded down to a multiple of four tiles so that every 128-row dQ tile that
// reads a dS' block of kb finds it written; within a chunk, the row tiles [rt_begin, rt_end) of
// those.  Blocks kb and n_kb-1-kb form a pair: the first is walked from the chunk's last row
// tile down, the second from its first row tile up, so every pair has about the same length and,
// at any moment, all pairs of a batch element read the same one or two row tiles (L2 sharing).
// Each pair's steps are cut into `parts` equal segments.
__host__ __device__ inline int first_row_tile(int causal, int Sq, int Sk, int H, int kb) {
  if (!causal) return 0;
  const int first_pos = max(0, kKeys * kb - (Sk - Sq));
  return 4 * (int)(((int64_t)first_pos * H) / 128);
}
// 64-key blocks that write dS' for 128-row group t: those with first_row_tile <= 4 t, a prefix
// of the key blocks since first_row_tile does not decrease.
__host__ __device__ inline int group_key_blocks(int causal, int Sq, int Sk, int H, int n_kb, int t) {
  int lo = 0, hi = n_kb;   // first kb with first_row_tile(kb) > 4 t
  while (lo < hi) {
    const int mid = (lo + hi) / 2;
    if (first_row_tile(causal, Sq, Sk, H, mid) <= 4 * t) lo = mid + 1; else hi = mid;
  }
  return lo;
}
struct PairPlan {
  int kb_a, kb_b, first_a, first_b, steps_a, total;
};
__host__ __device__ inline PairPlan pair_plan(int causal, int Sq, int Sk, int H, int rt_begin, int rt_end, int n_kb,
                                              int i) {
  PairPlan pp;
  pp.kb_a = i;
  pp.kb_b = n_kb - 1 - i;
  pp.first_a = max(rt_begin, first_row_tile(causal, Sq, Sk, H, pp.kb_a));
  pp.first_b = max(rt_begin, first_row_tile(causal, Sq, Sk, H, pp.kb_b));
  pp.steps_a = max(0, rt_end - pp.first_a);
  pp.total = pp.steps_a + (pp.kb_b != pp.kb_a ? max(0, rt_end - pp.first_b) : 0);
  return pp;
}
__host__ __device__ inline int part_begin(int total, int parts, int j) {
  return (int)(((int64_t)total * j) / parts);
}

// Slot of C-order lane c in a stored 16x16 dS' block (8 bytes per slot): bit 2 of the lane
// index flipped for lanes 32-63.  The dQ kernel's transposed reads of a block then take 32
// distinct slots modulo 32 (the 64 LDS banks) per 32 lanes; plain C order put lanes q and q + 2
// of a read on the same banks (a 2-way conflict on every dS' read).
__host__ __device__ inline int ds_slot(int c) { return c ^ ((c >> 3) & 4); }

__device__ __forceinline__ f16x4 to_f16x4(float a, float b, float c, float d) {
  f16x4 r;
  r[0] = (_Float16)a; r[1] = (_Float16)b; r[2] = (_Float16)c; r[3] = (_Float16)d;
  return r;
}

// ---- 1. row statistics -------------------------------------------------------------------
// One workgroup per 32-row tile; 8 lanes per row.  Load c of lane p covers elements
// 8 (8c + p) .. +7, so the 8 lanes of a row read 128 contiguous bytes per instruction, and
// each lane keeps its 16 row loads and the row's m, l in flight together.  The workgroup also
// records its largest |dO| for the gradient exponent.
__global__ void __launch_bounds__(256) bwd_prep_kernel(BwdParams p) {
  const int b = blockIdx.y;
  const int t = threadIdx.x;
  if (blockIdx.x == 0 && blockIdx.y == 0) {
    // goff: exclusive prefix of group_key_blocks over the groups, 256 groups per round (a
    // shuffle scan per wave, the four wave totals through LDS).
    __shared__ int wsum[4];
    int carry = 0;
    for (int base = 0; base <= p.n_groups; base += 256) {
      const int gi = base + t;
      const int v = gi < p.n_groups ? group_key_blocks(p.causal, p.Sq, p.Sk, p.H, p.n_kb, gi) : 0;
      int x = v;
      const int ln = t & 63, wv = t >> 6;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (ln >= o) x += y;
      }
      if (ln == 63) wsum[wv] = x;
      __syncthreads();
      int before = carry;
      for (int w = 0; w < wv; ++w) before += wsum[w];
      if (gi <= p.n_groups) p.goff[gi] = before + x - v;
      carry += wsum[0] + wsum[1] + wsum[2] + wsum[3];
      __syncthreads();
    }
  }
  const int row = blockIdx.x * kRows + (t >> 3);
  const int part = t & 7;
  const bool valid = row < p.R;
  // Rows past R read row R - 1 (in bounds); their statistics are replaced below.
  const int rr = valid ? row : p.R - 1;
  const int pos = fast_div(rr, p.hdiv), h = rr - pos * p.H;
  const bf16* orow = p.o + b * p.o_sb + h * p.o_sh + pos * p.o_ss + 8 * part;
  const bf16* drow = p.dout + b * p.do_sb + h * p.do_sh + pos * p.do_ss + 8 * part;
  const int64_t sidx = ((int64_t)b * p.H + h) * p.Sq + pos;
  bf16x8 ov[8], dv[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    ov[c] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(orow + 64 * c));
    dv[c] = *reinterpret_cast<const bf16x8*>(drow + 64 * c);
  }
  const float mv = p.m[sidx], lv = p.l[sidx];
  // All 18 loads are in flight before the first is used: left to the scheduler, each group of
  // loads was awaited before the next went out.  O is read only here, so its loads are
  // non-temporal: they do not displace the dO, Q and K_lat lines the dK/dV kernel reads next
  // (prep 61 -> 55 us and dK/dV -6 us at config 5).
  __builtin_amdgcn_sched_barrier(0);
  float dsum = 0.f, amax = 0.f;
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = (float)dv[c][e];
      dsum += (float)ov[c][e] * d;
      amax = fmaxf(amax, fabsf(d));
    }
  // The block's largest |dO|, one value per workgroup; bwd_kt, launched next, reduces them into
  // the call's maximum (the gradient exponent's input).
  amax = workgroup_max256(amax);
  if (t == 0) p.bmax[(int64_t)b * p.n_rt + blockIdx.x] = amax;
  dsum += __shfl_xor(dsum, 1, 8);
  dsum += __shfl_xor(dsum, 2, 8);
  dsum += __shfl_xor(dsum, 4, 8);
  if (part == 0) {
    float lse2 = __builtin_inff();
    if (valid) {
      // Rows that see no key (l = 0) get +inf, so that P = exp2(s - lse2) = 0 everywhere.
      if (lv > 0.f && __builtin_isfinite(mv)) lse2 = (mv + __logf(lv)) * kLog2e;
    } else {
      dsum = 0.f;
    }
    // The row's key limit (-1: no key) and its q / dout offsets, so that the dK/dV kernel's
    // tile loop needs neither a division nor 64-bit stride products per row.
    const int lim = valid ? (p.causal ? min(pos + (p.Sk - p.Sq), p.Sk - 1) : p.Sk - 1) : -1;
    const int64_t ri = (int64_t)b * p.n_rt * kRows + row;
    p.rstat[ri] = make_float4(lse2, dsum, __int_as_float(lim), 0.f);
    *reinterpret_cast<longlong2*>(p.roff + 2 * ri) = make_longlong2(h * p.q_sh + pos * p.q_ss, h * p.do_sh + pos * p.do_ss);
  }
}

// ---- 2. K_lat^T ----------------------------------------------------------------------------
// One workgroup per (64 keys, 64 dims) block through an LDS transpose; keys >= Sk are zero.
// The bf16 -> fp16 conversion is exact for |K| in fp16's normal range.
__global__ void __launch_bounds__(256) bwd_kt_kernel(BwdParams p) {
  __shared__ _Float16 tile[64][64 + 8];
  const int b = blockIdx.z, kb = blockIdx.y, db = blockIdx.x;
  const int t = threadIdx.x;
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int idx = t + 256 * r;
    const int key = idx >> 3, c = idx & 7;
    const int gk = kb * 64 + key;
    bf16x8 v = {};
    if (gk < p.Sk) v = *reinterpret_cast<const bf16x8*>(p.k + b * p.k_sb + gk * p.k_ss + 64 * db + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[key][8 * c + e] = (_Float16)(float)v[e];
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int idx = t + 256 * r;
    const int d = idx >> 3, c = idx & 7;
    f16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = tile[8 * c + e][d];
    // 32-key tile 2 kb + c / 4, keys 8 (c % 4) .. +7 of its dim row 64 db + d
    const int64_t tile_idx = (int64_t)b * (p.kt_ld / 32) + 2 * kb + (c >> 2);
    *reinterpret_cast<f16x8*>(p.kt + (tile_idx * kDqk + 64 * db + d) * 32 + 8 * (c & 3)) = v;
  }
  // The call's largest |dO| from bwd_prep's per-workgroup values (bwd_prep runs first).
  if (db == 0 && kb == 0 && b == 0) reduce_max_bits(p.bmax, p.B * p.n_rt, p.gmax);
}

// ---- 3. dK_lat / dV: key-block-stationary sweep over row tiles ----------------------------
//
// Workgroup = 4 waves (one per SIMD, up to 512 registers each) on 64 keys.  Per 32-row tile:
//   S-phase:  wave w = (row block rb = w>>1, dim half dh = w&1) computes partial S and dP for
//             rows 16 rb .. +15 and all 64 keys over its half of the contraction (S: dims
//             256 dh .. +255 and rope dims 512 + 32 dh .. +31; dP: dims 256 dh .. +255).  The
//             64 keys' K_lat columns of that half are the B operand, held in the AGPR file (144
//             registers), so each Q / dO row read from LDS feeds four MFMAs: with one wave per
//             SIMD the LDS delivers about 1 KB per wave every ~70 cycles, and this halves the
//             reads per MFMA against two keys blocks per wave.  The pair (rb, 0) / (rb, 1) swaps
//             the fp32 partials of the key blocks the other one finishes (4 KB each way); wave
//             (rb, dh) then forms P and dS' = scale P (dP - D), masked, for key blocks 2 dh,
//             2 dh + 1.  The MFMA C layout (lane: one key, 4 rows) is exactly half of the A
//             operand the dK update needs (lane: one key, 8 rows), so the two row blocks meet
//             in a 4 KB exchange without transposition; dS' also goes to HBM for dQ.
//   dK-phase: wave w owns column blocks w, w+4, .., w+32 of all 64 keys (36 accumulators in
//             arch VGPRs): dK += dS'^T Q (9 blocks) and dK[:, :512] += P^T dO (8 blocks), fp16
//             operands; Q and dO columns come from ds_read_b64_tr_b16 so that k runs along
//             the tile's rows.
// Row tiles stream through two LDS stages (Q + dO = 68 KB each) with direct global->LDS
// copies; three barriers per tile (tile landed / partials swapped / exchange written).
constexpr int kXchOffset = kXOffset + 2 * 4 * 1024;   // partial swap: [wave][4 tiles][64 lanes][16 B]
static_assert(kXchOffset + 4 * 4096 == kDkdvLds, "LDS layout");

__global__ void __launch_bounds__(kBwdThreads, 1) __attribute__((amdgpu_waves_per_eu(1, 1)))
bwd_dkdv_kernel(BwdParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[kDkdvLds];
  DMLA_LDS char* lds = (DMLA_LDS char*)smem;
  const int wave = uniform(threadIdx.x >> 6);
  const int lane = lane_id();
  // Consecutive work items share (batch, segment) and so read the same row tiles: keep them on
  // one XCD (workgroups are dealt to the 8 XCDs round robin).
  const int per_xcd = (p.n_items + 7) >> 3;
  const int u = (int)(blockIdx.x & 7) * per_xcd + (int)(blockIdx.x >> 3);
  if (u >= p.n_items) return;
  const int pi = u % p.n_pairs;
  const int pj = (u / p.n_pairs) % p.parts;
  const int b = u / (p.n_pairs * p.parts);
  const PairPlan pp = pair_plan(p.causal, p.Sq, p.Sk, p.H, p.rt_begin, p.rt_end, p.n_kb, pi);
  const int lo = part_begin(pp.total, p.parts, pj), hi = part_begin(pp.total, p.parts, pj + 1);
  const int goff0 = p.goff[p.rt_begin / 4];

  const int l16 = lane & 15, g = lane >> 4;
  const int rb = wave >> 1;      // S-phase row block
  const int dh = wave & 1;       // S-phase dim half; this wave finishes key blocks 2 dh, 2 dh + 1
  const int gexp = grad_exponent(p.gmax);
  const float scale = p.scale * exp2i(gexp), scale_log2 = p.scale_log2;   // dS' carries 2^e
  const unsigned gexp_bits = grad_exponent_bits(gexp);   // dO operands: 2^e
  const unsigned lds_base = lds_addr(lds);
  DMLA_LDS char* xbuf = lds + kXOffset;
  DMLA_LDS char* xch = lds + kXchOffset;

  // Per-lane LDS offsets (tile-relative).  S-phase A operand (row operand) of row block rb and
  // k-step c (dims 32c ..): chunk 4c + g of row 16 rb + l16 = group c/2, in-group chunk
  // 4 (c&1) + g.
  const int arow = 16 * rb + l16;
  const int a_off[2] = {arow * 128 + 16 * (g ^ swz(arow & 15)), arow * 128 + 16 * ((4 + g) ^ swz(arow & 15))};
  // dK-phase B operand (column operand) of column block cb = wave + 4u: group u, in-group chunk
  // 2 wave + (q >> 1) of rows 4g + e (+16 for the second half).
  const int e = l16 >> 2, qq = l16 & 3;
  const int brow = 4 * g + e;
  const int b_off = brow * 128 + 16 * ((2 * wave + (qq >> 1)) ^ swz(brow)) + 8 * (qq & 1);
  // Copies: wave w moves rows 8w .. 8w+7 of every chunk group; lane l -> row 8w + l/8, physical
  // chunk l%8 = logical chunk (l%8) ^ swz(row).
  const int crow = 8 * wave + (lane >> 3);
  const int cchunk = (lane & 7) ^ swz(crow & 15);

  bool first_segment = true;
  for (int ph = 0; ph < 2; ++ph) {
    const int g_lo = ph == 0 ? lo : max(lo, pp.steps_a);
    const int g_hi = ph == 0 ? min(hi, pp.steps_a) : hi;
    if (g_lo >= g_hi) continue;
    const int count = g_hi - g_lo;
    const int kb = ph == 0 ? pp.kb_a : pp.kb_b;
    const int dir = ph == 0 ? -1 : 1;
    const int rt_first = ph == 0 ? p.rt_end - 1 - g_lo : pp.first_b + (g_lo - pp.steps_a);
    if (!first_segment) __syncthreads();   // the previous segment's last tile is still being read
    first_segment = false;
    const int key0 = kb * kKeys;

    // K_lat columns of this wave's dim half for all 64 keys, B operand of S = Q K^T (zero past
    // Sk): kreg[kb][j] = K[key0 + 16 kb + l16][32 step(j) + 8 g .. +7], step(j) = 8 dh + j for
    // j < 8 (also the V_lat columns of dP) and 16 + dh for j = 8.
    bf16x8 kreg[4][9];
#pragma unroll
    for (int kbl = 0; kbl < 4; ++kbl) {
      const int key = key0 + 16 * kbl + l16;
      const bf16* krow = p.k + b * p.k_sb + (int64_t)(key < p.Sk ? key : 0) * p.k_ss + 8 * g;
#pragma unroll
      for (int j = 0; j < 9; ++j) {
        const int step = j < 8 ? 8 * dh + j : 16 + dh;
        kreg[kbl][j] = *reinterpret_cast<const bf16x8*>(krow + 32 * step);
      }
    }
    // All 36 loads are issued before any is used (the scheduling barrier keeps them together):
    // left to the scheduler, each load was awaited before the next was issued, 36 memory round
    // trips in a row per segment.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kbl = 0; kbl < 4; ++kbl)
      if (key0 + 16 * kbl + l16 >= p.Sk)
#pragma unroll
        for (int j = 0; j < 9; ++j) kreg[kbl][j] = bf16x8{};   // zero past Sk
    // K_lat lives in the AGPR file (MFMA reads A/B operands from AGPRs directly): the arch VGPRs
    // hold the 144 accumulators and the LDS operands in flight.
#pragma unroll
    for (int kbl = 0; kbl < 4; ++kbl)
      asm volatile("" : "+a"(kreg[kbl][0]), "+a"(kreg[kbl][1]), "+a"(kreg[kbl][2]), "+a"(kreg[kbl][3]),
                   "+a"(kreg[kbl][4]), "+a"(kreg[kbl][5]), "+a"(kreg[kbl][6]), "+a"(kreg[kbl][7]),
                   "+a"(kreg[kbl][8]));

    f32x4 acc[4][9];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int v = 0; v < 9; ++v) acc[a][v] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Staging of row tile rt into LDS stage st (rows past R re-read row R-1: finite, and masked
    // by their +inf lse2): this lane's row sources, then 17 copies: the 9 Q chunk groups one per
    // S-phase step, the 8 dO groups two per step in the first four dK-phase steps.  The CU's
    // vector-memory path moves about 64 B per clock (~1000 clocks for the 68 KB tile), so the
    // copies are spread under the MFMAs instead of stalling the wave in one burst.  Measured
    // alternatives (kernel-trace A/B at config 5): all 17 in the S-phase stalled it by ~1000
    // clocks per tile; the dO copies one per step over the first eight dK steps left the next
    // tile's barrier ~1000 clocks of wait (2 % slower); issued around the partial swap or with
    // the dS' stores, they slowed every phase after them (8 % slower).
    const char* qsrc = nullptr;
    const char* osrc = nullptr;
    unsigned cdst = 0;
    // The segment's first tile from the row index; the later ones from the offsets bwd_prep
    // stored for each row (loaded a tile ahead with the statistics), which spares the tile loop
    // a division and four 64-bit stride products per lane.
    auto stage_begin_first = [&](int rt, int st) {
      const int r = min(rt * kRows + crow, p.R - 1);
      const int pos = fast_div(r, p.hdiv), h = r - pos * p.H;
      qsrc = reinterpret_cast<const char*>(p.q + b * p.q_sb + h * p.q_sh + pos * p.q_ss + 8 * cchunk);
      osrc = reinterpret_cast<const char*>(p.dout + b * p.do_sb + h * p.do_sh + pos * p.do_ss + 8 * cchunk);
      cdst = lds_base + st * kStageBytes + wave * 1024;
    };
    longlong2 roff_next = {};   // q / dout offsets of the copy row of the tile staged next
    auto roff_load = [&](int rt) {
      roff_next = *reinterpret_cast<const longlong2*>(p.roff + 2 * ((int64_t)b * p.n_rt * kRows + rt * kRows + crow));
    };
    auto stage_begin = [&](int st) {
      qsrc = reinterpret_cast<const char*>(p.q + b * p.q_sb + roff_next.x + 8 * cchunk);
      osrc = reinterpret_cast<const char*>(p.dout + b * p.do_sb + roff_next.y + 8 * cchunk);
      cdst = lds_base + st * kStageBytes + wave * 1024;
    };
    auto stage_copy = [&](int i) {   // i < 9: Q chunk group i; else dO chunk group i - 9
      if (i < kQGroups) dma16_addr(qsrc + 128 * i, cdst + i * kGroupBytes);
      else dma16_addr(osrc + 128 * (i - kQGroups), cdst + kQBytes + (i - kQGroups) * kGroupBytes);
    };
    // (lse2, D) and key limit of this lane's 4 rows 32 rt + 16 rb + 4 g + i, and the dS' pair of
    // (rt's group, kb).  Loaded one tile ahead, with the statistics: a load issued after the
    // tile's copies would wait for all of them (vector-memory loads complete in order).
    float lse2[4], dval[4];
    int lim[4];
    int64_t ds_pair = 0;
    auto row_stats = [&](int rt) {
      ds_pair = (int64_t)b * p.chunk_pairs + p.goff[rt >> 2] - goff0 + kb;
      const int r0 = rt * kRows + 16 * rb + 4 * g;
      const float4* src = p.rstat + (int64_t)b * p.n_rt * kRows + r0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 a = src[i];
        lse2[i] = a.x;
        dval[i] = a.y;
        lim[i] = __float_as_int(a.z);
      }
    };

    stage_begin_first(rt_first, 0);
#pragma unroll
    for (int i = 0; i < kQGroups + kOGroups; ++i) stage_copy(i);
    row_stats(rt_first);
    roff_load(count > 1 ? rt_first + dir : rt_first);
    for (int s = 0; s < count; ++s) {
      const int rt = rt_first + dir * s;
      const int st = s & 1;
      wait_vmem();
      __syncthreads();   // tile s landed everywhere; the other stage and the exchanges are free
      const bool more = s + 1 < count;
      // The copies run unconditionally (branch-free loop body): past the segment's last tile they
      // re-read this tile into the idle stage, and the segment end waits for them.
      stage_begin(st ^ 1);   // tile s + 1, or tile s again past the segment's last
      const DMLA_LDS char* qt = lds + st * kStageBytes;
      const DMLA_LDS char* ot = qt + kQBytes;

      // ---- S-phase: partial S (9 reads, 36 MFMAs) and dP (8 reads, 32 MFMAs) ----
      // Step j < 8 reads Q and dO of row block rb at dims 32 (8 dh + j) and feeds 8 MFMAs into
      // 8 different accumulators (S and dP x 4 key blocks); step 8 is Q's rope slice.  Reads
      // run two steps ahead of their MFMAs.
      f32x4 sacc[4], pacc[4];
#pragma unroll
      for (int kbl = 0; kbl < 4; ++kbl) sacc[kbl] = pacc[kbl] = f32x4{0.f, 0.f, 0.f, 0.f};
      auto s_read = [&](const DMLA_LDS char* base, int j) -> bf16x8 {
        const int step = j < 8 ? 8 * dh + j : 16 + dh;
        return lds_read_b128(reinterpret_cast<const DMLA_LDS bf16x8*>(base + (step >> 1) * kGroupBytes + a_off[step & 1]));
      };
      bf16x8 qa[3], oa[3];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        qa[j] = s_read(qt, j);
        oa[j] = s_read(ot, j);
      }
#pragma unroll
      for (int j = 0; j < 9; ++j) {
        if (j + 2 < 9) {
          qa[(j + 2) % 3] = s_read(qt, j + 2);
          if (j + 2 < 8) oa[(j + 2) % 3] = s_read(ot, j + 2);
        }
#pragma unroll
        for (int kbl = 0; kbl < 4; ++kbl) {
          sacc[kbl] = mfma_bf16(qa[j % 3], kreg[kbl][j], sacc[kbl]);
          if (j < 8) pacc[kbl] = mfma_bf16(oa[j % 3], kreg[kbl][j], pacc[kbl]);
        }
        stage_copy(j);   // the next tile's Q chunk group j into the other stage
      }
      // Swap: send the partials of the key blocks the partner finishes (2 (1 - dh), +1),
      // [wave][tile][lane] x 16 B; selects rather than indexing by the wave-dependent dh, which
      // the compiler would turn into register-indexed moves.
      f32x4 s_own[2], p_own[2];
      {
        DMLA_LDS f32x4* dst = reinterpret_cast<DMLA_LDS f32x4*>(xch + wave * 4096) + lane;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          s_own[kk] = dh ? sacc[2 + kk] : sacc[kk];
          p_own[kk] = dh ? pacc[2 + kk] : pacc[kk];
          dst[64 * kk] = dh ? sacc[kk] : sacc[2 + kk];
          dst[128 + 64 * kk] = dh ? pacc[kk] : pacc[2 + kk];
        }
      }
      __syncthreads();   // partials swapped
      {
        const DMLA_LDS f32x4* src = reinterpret_cast<const DMLA_LDS f32x4*>(xch + (wave ^ 1) * 4096) + lane;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          s_own[kk] += src[64 * kk];
          p_own[kk] += src[128 + 64 * kk];
        }
      }
      // P and dS' for keys key0 + 32 dh + 16 kk + l16, rows 16 rb + 4 g + i of the tile.
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int key = key0 + 32 * dh + 16 * kk + l16;
        float pv[4], dsv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float pr = key <= lim[i] ? fast_exp2(s_own[kk][i] * scale_log2 - lse2[i]) : 0.f;
          pv[i] = pr;
          dsv[i] = scale * pr * (p_own[kk][i] - dval[i]);
        }
        const f16x4 pb = to_f16x4(pv[0], pv[1], pv[2], pv[3]);
        const f16x4 db = to_f16x4(dsv[0], dsv[1], dsv[2], dsv[3]);
        const int kbl = 2 * dh + kk;
        *reinterpret_cast<DMLA_LDS f16x4*>(xbuf + kbl * 1024 + lane * 16 + 8 * rb) = pb;
        *reinterpret_cast<DMLA_LDS f16x4*>(xbuf + 4096 + kbl * 1024 + lane * 16 + 8 * rb) = db;
        _Float16* dsblk = p.ds + ((ds_pair * 8 + 2 * (rt & 3) + rb) * 4 + kbl) * 256;
        *reinterpret_cast<f16x4*>(dsblk + 4 * ds_slot(lane)) = db;
      }
      __syncthreads();   // exchange written
      if (more) {
        row_stats(rt + dir);
        roff_load(s + 2 < count ? rt + 2 * dir : rt + dir);   // the tile the next iteration stages
      }

      // ---- dK-phase ----
      f16x8 pT[4], dsT[4];
#pragma unroll
      for (int kbl = 0; kbl < 4; ++kbl) {
        pT[kbl] = *reinterpret_cast<const DMLA_LDS f16x8*>(xbuf + kbl * 1024 + lane * 16);
        dsT[kbl] = *reinterpret_cast<const DMLA_LDS f16x8*>(xbuf + 4096 + kbl * 1024 + lane * 16);
      }
      // A operands of the whole phase: AGPR file.  One statement for all eight, so the reads go
      // out together and are awaited once (one statement per operand had the compiler issue
      // them two at a time, each pair awaited before the next).
      asm volatile("" : "+a"(pT[0]), "+a"(pT[1]), "+a"(pT[2]), "+a"(pT[3]), "+a"(dsT[0]), "+a"(dsT[1]),
                   "+a"(dsT[2]), "+a"(dsT[3]));
      // Column operands of column block wave + 4v (v < 9: Q; v >= 9: dO block v - 9), as two
      // transposed half reads each.  Software pipeline over the 17 operands: step v issues the
      // reads of operand v + 3, the 4 MFMAs of operand v and, between them, the fp16
      // conversion of operand v + 1 (a dO operand times 2^e, one more instruction per value
      // pair), so each read has two steps (8 MFMAs) to land.  The
      // schedule is pinned with scheduling-group barriers: left to itself the compiler issued
      // each operand's reads right before its conversion and waited for them there, one LDS
      // round trip per operand.
      auto k_read = [&](int v, bf16x4& lo, bf16x4& hi) {
        const DMLA_LDS char* c = v < 9 ? qt + v * kGroupBytes + b_off : ot + (v - 9) * kGroupBytes + b_off;
        lo = lds_read_tr16(reinterpret_cast<const DMLA_LDS bf16x4*>(c));
        hi = lds_read_tr16(reinterpret_cast<const DMLA_LDS bf16x4*>(c + 16 * 128));
      };
      bf16x4 kl[4], kh[4];   // raw operands, ring slot v & 3
#pragma unroll
      for (int j = 0; j < 3; ++j) k_read(j, kl[j], kh[j]);
      f16x8 bnext = bf16_to_f16(kl[0], kh[0]);
#pragma unroll
      for (int v = 0; v < 17; ++v) {
        if (v + 3 < 17) k_read(v + 3, kl[(v + 3) & 3], kh[(v + 3) & 3]);
        if (v < kOGroups / 2) {   // the next tile's dO chunk groups 2v, 2v + 1
          stage_copy(kQGroups + 2 * v);
          stage_copy(kQGroups + 2 * v + 1);
        }
        const f16x8 bop = bnext;
        if (v + 1 < 9) bnext = bf16_to_f16(kl[(v + 1) & 3], kh[(v + 1) & 3]);
        else if (v + 1 < 17) bnext = bf16_to_f16_scaled(kl[(v + 1) & 3], kh[(v + 1) & 3], gexp_bits);
        if (v < 9) {
#pragma unroll
          for (int kbl = 0; kbl < 4; ++kbl) acc[kbl][v] = mfma_f16(dsT[kbl], bop, acc[kbl][v]);
        } else {
#pragma unroll
          for (int kbl = 0; kbl < 4; ++kbl) acc[kbl][v - 9] = mfma_f16(pT[kbl], bop, acc[kbl][v - 9]);
        }
        if (v + 3 < 17) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // reads of operand v + 3
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // an MFMA of operand v
          if (v + 1 < 9) __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);   // a quarter of the conversion
          else if (v + 1 < 17) __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        }
        __builtin_amdgcn_sched_barrier(0);   // nothing crosses a step boundary
      }
    }

    wait_vmem();   // no copy may still land in a stage once the segment is over
    // Partial of this segment: acc[kbl][v] holds dK[16 kbl + 4 g + i][16 (wave + 4 v) + l16].
    float* dst = p.part + ((int64_t)u * 2 + ph) * kPartFloats;
#pragma unroll
    for (int kbl = 0; kbl < 4; ++kbl)
#pragma unroll
      for (int v = 0; v < 9; ++v)
        *reinterpret_cast<f32x4*>(dst + ((kbl * kCb + wave + 4 * v) * 64 + lane) * 4) = acc[kbl][v];
  }
}

// ---- 4. dQ = dS' K_lat ----------------------------------------------------------------------
// Workgroup = 8 waves on 128 rows x 576 dims; wave w owns column blocks w%4, w%4+4, .., +32 of
// the four row blocks of its row half w/4 (36 accumulators), so each 36 KB K^T tile staged in
// LDS serves 128 rows.  Per 32-key tile: dS' (A operand, row fixed per lane) from the stored
// C-order blocks through ds_read_b64_tr_b16, K^T (B operand) with b128 reads.  Tiles flow
// through a 3-slot ring: the copies of tile kt+2 go out between the MFMAs of tile kt, so the
// dS' blocks (read from HBM) have two tiles of time to land.
__device__ __forceinline__ void dk_reduce_unit(const BwdParams& p, int b, int kb, int kbl, int t);

__global__ void __launch_bounds__(kDqThreads, 1) bwd_dq_kernel(BwdParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[kDqLds];
  DMLA_LDS char* lds = (DMLA_LDS char*)smem;
  const int wave = uniform(threadIdx.x >> 6);
  const int lane = lane_id();
  // The chunk's 128-row tiles (its row groups), heaviest (latest) first.
  const int g_end = (p.rt_end + 3) / 4;
  const int n_dq = p.B * (g_end - p.rt_begin / 4);
  if ((int)blockIdx.x >= n_dq) {
    // Past the dQ tiles: the dK_lat reduction, two (b, key block, column quarter) units per
    // workgroup, one per 256 threads.  These workgroups start as the dQ tiles drain.
    const int u = 2 * ((int)blockIdx.x - n_dq) + (int)(threadIdx.x >> 8);
    if (u < 4 * p.n_kb * p.B) dk_reduce_unit(p, u / (4 * p.n_kb), (u / 4) % p.n_kb, u % 4, (int)(threadIdx.x & 255));
    return;
  }
  const int b = (int)blockIdx.x % p.B;
  const int t = g_end - 1 - (int)blockIdx.x / p.B;
  const int row0 = kDqRows * t;
  const int last_row = min(p.R, row0 + kDqRows) - 1;
  const int kmax = p.causal ? min(p.Sk - 1, last_row / p.H + (p.Sk - p.Sq)) : p.Sk - 1;
  const int n_kt = kmax >= 0 ? kmax / 32 + 1 : 0;
  const int l16 = lane & 15, g = lane >> 4;
  const int e = l16 >> 2, qq = l16 & 3;
  const int rh = wave >> 2, wc = wave & 3;   // row half (64 rows) and column phase of this wave
  const unsigned lds_base = lds_addr(lds);
  // Row blocks of 16 that exist in the dS' buffer (rows padded to 64).
  const int n_rb = 2 * p.n_rt;

  // Copies.  dS': wave w moves row block w of the group, key blocks 2 kt, 2 kt + 1 (1 KB contiguous).
  // K^T: 16 dims x 32 keys per copy (1 KB, contiguous in the tiled K^T: whole 128-byte lines
  // per copy, where rows of a dims x keys matrix gave 64-byte pieces of 16 lines), wave w copies
  // dim blocks w, w+8, .. (5 or 4 copies);
  // lane l -> dim row r = l/4 of block n, physical chunk l%4 = logical chunk (l%4) ^ kt_swz(r).
  // A ds_read_b128 is served 16 lanes at a time, the lanes with equal bit 5 and equal parity of
  // bits 2-4 of the lane index (a model that predicts the LDS bank-conflict counter for every
  // swizzle of the form parity(r & m0) | parity(r & m1) << 1 of this read).  In the read below
  // such a group holds rows r, r^12 of one column group g and rows r^4, r^8 of g^1, all on the
  // same 16 banks of the 64 (64-byte rows), so their four chunks must differ: kt_swz(r) = 2 *
  // bit 2 of r does that.  Swizzled by r >> 2, every K^T read was a two-way conflict.
  auto kt_swz = [](int r) { return 2 * ((r >> 2) & 1); };
  const unsigned kt_voff = (unsigned)(((lane >> 2) * 32 + 8 * ((lane & 3) ^ kt_swz(lane >> 2))) * 2);
  // Every wave issues exactly six copies per stage (so one vmcnt value waits for a stage):
  // a row block past the buffer copies row block 0 instead (its rows are not stored), and
  // waves 4-7 copy their dim block w + 24 a second time (same bytes to the same place).
  const int rblk = 8 * t + wave < n_rb ? wave : 0;
  const int64_t pair0 = (int64_t)b * p.chunk_pairs + p.goff[t] - p.goff[p.rt_begin / 4];
  auto copy = [&](int kt, int st, int m) {
    const unsigned dst = lds_base + st * kDqStageBytes;
    if (m == 0) {
      const _Float16* dsrc = p.ds + (((pair0 + (kt >> 1)) * 8 + rblk) * 4 + 2 * (kt & 1)) * 256;
      dma16(dsrc, 16u * lane, dst + wave * 1024);
    } else {
      const int n0 = wave + 8 * (m - 1);
      const int n = n0 < kDqk / 16 ? n0 : n0 - 8;
      const _Float16* ksrc = p.kt + (((int64_t)b * (p.kt_ld / 32) + kt) * kDqk + 16 * n) * 32;
      dma16(ksrc, kt_voff, dst + kDqDsBytes + n * 1024);
    }
  };
  auto stage = [&](int kt, int st) {
#pragma unroll
    for (int m = 0; m < 6; ++m) copy(kt, st, m);
  };
  // dS' A operand of row block rq, half h: lane 4e+q of group g reads C-order lane
  // 16 q + 8 (g & 1) + 4 h + e of key block g >> 1 (see the tr-read rule in dmla_common.h), at
  // its stored slot ds_slot().
  const int a_c = 16 * qq + 8 * (g & 1) + e;
  const int a_off0 = 4 * rh * 1024 + (g >> 1) * 512 + 8 * ds_slot(a_c);
  const int a_off1 = 4 * rh * 1024 + (g >> 1) * 512 + 8 * ds_slot(a_c + 4);
  // K^T B operand of column block wc + 4u: dim row 16 cb + l16, logical chunk g.
  const int b_off = kDqDsBytes + wc * 1024 + l16 * 64 + 16 * (g ^ kt_swz(l16));

  f32x4 acc[4][9];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int v = 0; v < 9; ++v) acc[a][v] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (n_kt > 0) stage(0, 0);
  if (n_kt > 1) stage(1, 1);
  int st = 0;
  for (int kt = 0; kt < n_kt; ++kt) {
    // stage kt has landed; stage kt+1 (six copies per wave) may still be in flight
    if (kt + 1 < n_kt) __builtin_amdgcn_s_waitcnt(0x0f76);   // vmcnt(6)
    else wait_vmem();
    __syncthreads();
    const bool more = kt + 2 < n_kt;
    const int st2 = st == 0 ? 2 : st - 1;   // (kt + 2) % 3
    const DMLA_LDS char* sb = lds + st * kDqStageBytes;
    f16x8 a[4];
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const DMLA_LDS char* ab = sb + rq * 1024;
      const f16x4 lo = lds_read_tr16_f16(reinterpret_cast<const DMLA_LDS f16x4*>(ab + a_off0));
      const f16x4 hi = lds_read_tr16_f16(reinterpret_cast<const DMLA_LDS f16x4*>(ab + a_off1));
      a[rq] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
#pragma unroll
    for (int v = 0; v < 9; ++v) {
      const f16x8 kb = *reinterpret_cast<const DMLA_LDS f16x8*>(sb + b_off + v * 4096);
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) acc[rq][v] = mfma_f16(a[rq], kb, acc[rq][v]);
      // copies of stage kt+2 into the slot step kt-1 read, between the MFMAs
      if (more && v < 6) copy(kt + 2, st2, v);
    }
    st = st == 2 ? 0 : st + 1;
  }

  // acc[rq][v] holds dQ[row0 + 64 rh + 16 rq + 4 g + i][16 (wc + 4 v) + l16] times 2^e.
  const float unscale = exp2i(-grad_exponent(p.gmax));
  if (p.dq_rows16) {
    // bf16 dQ leaves as whole-line pieces with 16-byte stores: the 128 x 576 tile is staged in
    // the (now free) stages in two column parts, columns 0-319 (the waves' column blocks v < 5)
    // and 320-575 (v >= 5), every wave staging its own blocks of both row halves at once; then
    // every thread stores its share of the part's 16-byte pieces.  Stored straight from the
    // accumulators (one 2-byte value per lane and instruction, 144 store instructions per lane)
    // the kernel took 168 us at the config-5 shapes, staged 161 us.  The row pitch (part width
    // + 16 bytes) puts the four row groups of a staging write on distinct banks.
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      const int v0 = part == 0 ? 0 : 5, v1 = part == 0 ? 5 : 9;
      const int c0 = 16 * 4 * v0;                 // first column of the part
      const int width = 16 * 4 * (v1 - v0);       // 320 or 256 columns
      const int pitch = 2 * width + 16;
      __syncthreads();   // the stages (first part) or the previous part's pieces are read out
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int v = v0; v < v1; ++v)
            *reinterpret_cast<DMLA_LDS bf16*>(lds + (64 * rh + 16 * rq + 4 * g + i) * pitch +
                                             (16 * (wc + 4 * v) - c0 + l16) * 2) = (bf16)(acc[rq][v][i] * unscale);
      __syncthreads();
      const int per_row = width / 8;              // 40 or 32 pieces
#pragma unroll
      for (int it = 0; it < 10; ++it) {
        const int j = it * kDqThreads + (int)threadIdx.x;
        if (j >= kDqRows * per_row) break;
        const int rl = j / per_row, c = j - rl * per_row;
        const int r = row0 + rl;
        if (r >= p.R) continue;
        const bf16x8 piece = *reinterpret_cast<const DMLA_LDS bf16x8*>(lds + rl * pitch + 16 * c);
        const int pos = fast_div(r, p.hdiv), h = r - pos * p.H;
        *reinterpret_cast<bf16x8*>(static_cast<bf16*>(p.dq) + b * p.dq_sb + h * p.dq_sh + pos * p.dq_ss + c0 + 8 * c) = piece;
      }
    }
    return;
  }
#pragma unroll
  for (int rq = 0; rq < 4; ++rq) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = row0 + 64 * rh + 16 * rq + 4 * g + i;
      if (r >= p.R) continue;
      const int pos = fast_div(r, p.hdiv), h = r - pos * p.H;
      const int64_t base = b * p.dq_sb + h * p.dq_sh + pos * p.dq_ss + l16;
#pragma unroll
      for (int v = 0; v < 9; ++v) {
        const int col = 16 * (wc + 4 * v);
        const float x = acc[rq][v][i] * unscale;
        if (p.dq_fp32) static_cast<float*>(p.dq)[base + col] = x;
        else static_cast<bf16*>(p.dq)[base + col] = (bf16)x;
      }
    }
  }
}

// ---- 5. dK_lat = sum of the segment partials ------------------------------------------------
// One unit per (batch, 64-key block, 16-key block), run by 256 threads of a workgroup past the
// dQ tiles of bwd_dq_kernel (they start as those tiles drain; a launch of its own measured
// 20 us, the shared launch ~5 us less in the traced sum).  The segments of the block are added
// in part order, so the result does not depend on scheduling.  Thread t owns the 9 (column block,
// lane) slots t + 256 r of the 16 keys and loads all 9 of a part together (a wave reads 1 KB per
// slot), so each wave keeps 9 KB in flight instead of one dependent load per slot (33 -> 19 us
// at config 5; two parts at a time measured no faster).
constexpr int kReduceSlots = kCb * 64 / 256;
static_assert(kReduceSlots * 256 == kCb * 64, "the reduction's slots cover the partial evenly");

__device__ __forceinline__ void dk_reduce_unit(const BwdParams& p, int b, int kb, int kbl, int t) {
  const int pi = min(kb, p.n_kb - 1 - kb);
  const int ph = kb == pi ? 0 : 1;
  const PairPlan pp = pair_plan(p.causal, p.Sq, p.Sk, p.H, p.rt_begin, p.rt_end, p.n_kb, pi);
  const int iv_lo = ph == 0 ? 0 : pp.steps_a;
  const int iv_hi = ph == 0 ? pp.steps_a : pp.total;
  const int ln = t & 63;
  f32x4 s[kReduceSlots];
#pragma unroll
  for (int r = 0; r < kReduceSlots; ++r) s[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < p.parts; ++j) {
    const int lo = part_begin(pp.total, p.parts, j), hi = part_begin(pp.total, p.parts, j + 1);
    if (max(lo, iv_lo) >= min(hi, iv_hi)) continue;   // no partial stored for this phase
    const int u = (b * p.parts + j) * p.n_pairs + pi;
    const f32x4* src = reinterpret_cast<const f32x4*>(p.part + ((int64_t)u * 2 + ph) * kPartFloats) +
                       kbl * kCb * 64 + t;
    f32x4 v[kReduceSlots];
#pragma unroll
    for (int r = 0; r < kReduceSlots; ++r) v[r] = src[256 * r];
#pragma unroll
    for (int r = 0; r < kReduceSlots; ++r) s[r] += v[r];
  }
  const float unscale = exp2i(-grad_exponent(p.gmax));   // the partials carry 2^e
#pragma unroll
  for (int r = 0; r < kReduceSlots; ++r) {
    const int cb = (t >> 6) + 4 * r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = kb * kKeys + 16 * kbl + 4 * (ln >> 4) + i;
      if (key >= p.Sk) continue;
      const int col = 16 * cb + (ln & 15);
      const int64_t o = b * p.dk_sb + key * p.dk_ss + col;
      // Chunks after the first add to the fp32 sum of the earlier ones; the last writes dK_lat.
      const int64_t oa = p.dk_fp32 ? o : ((int64_t)b * p.Sk + key) * kDqk + col;
      float v = s[r][i] * unscale;
      if (p.chunk > 0) v += p.dk_acc[oa];
      if (!p.last_chunk) p.dk_acc[oa] = v;
      else if (p.dk_fp32) static_cast<float*>(p.dk)[o] = v;
      else static_cast<bf16*>(p.dk)[o] = (bf16)v;
    }
  }
}

// ---- host-side planning ----------------------------------------------------------------------
// dS' bytes of one (128-row group, 64-key block) pair: 8 row blocks x 4 key blocks x 256 fp16.
constexpr int64_t kPairBytes = 8 * 4 * 256 * 2;

// The cap on a chunk's dS' storage: DMLA_BWD_DS_CAP_BYTES, or the environment variable of that
// name when set (tests use it to force several chunks at small sizes).  Read once per plan: the
// plan keeps it, and both the workspace sizing and the chunk loop of a call use that copy.
// Like any environment variable it must not be changed while another thread calls in.
int64_t ds_cap_bytes() {
  const char* e = getenv("DMLA_BWD_DS_CAP_BYTES");
  if (e != nullptr && *e) {
    const long long v = atoll(e);
    if (v > 0) return v;
  }
  return DMLA_BWD_DS_CAP_BYTES;
}

struct BwdChunk {
  int g0, g1;      // row groups [g0, g1)
  int pairs;       // (group, key block) pairs: dS' blocks per batch element
  int parts, n_items;
};

struct BwdPlan {
  int R, n_rt, n_kb, n_pairs, kt_ld, n_groups;
  int n_chunks, max_pairs, max_items;
  int64_t cap;     // dS' bytes per chunk, read once (ds_cap_bytes)
  int64_t off_rstat, off_roff, off_kt, off_goff, off_bmax, off_gmax, off_ds, off_part, off_acc, bytes;
};

int64_t round256(int64_t x) { return (x + 255) & ~(int64_t)255; }

// The chunk starting at group g0: whole groups while their dS' fits the cap (at least one).
BwdChunk next_chunk(const BwdPlan& pl, int64_t B, int64_t H, int64_t Sq, int64_t Sk, int causal, int cus, int g0,
                    int64_t cap) {
  BwdChunk c = {};
  c.g0 = g0;
  c.g1 = g0;
  int64_t pairs = 0;
  while (c.g1 < pl.n_groups) {
    const int nk = group_key_blocks(causal, (int)Sq, (int)Sk, (int)H, pl.n_kb, c.g1);
    if (c.g1 > g0 && (pairs + nk) * B * kPairBytes > cap) break;
    pairs += nk;
    ++c.g1;
  }
  c.pairs = (int)pairs;
  const int rt0 = 4 * c.g0, rt1 = min(pl.n_rt, 4 * c.g1);
  int max_total = 1;
  for (int i = 0; i < pl.n_pairs; ++i)
    max_total = max(max_total, pair_plan(causal, (int)Sq, (int)Sk, (int)H, rt0, rt1, pl.n_kb, i).total);
  const int64_t base = B * pl.n_pairs;
  int parts = (int)((cus + base - 1) / base);
  c.parts = max(1, min(parts, min(kMaxParts, max_total)));
  c.n_items = (int)(base * c.parts);
  return c;
}

BwdPlan make_plan(int64_t B, int64_t H, int64_t Sq, int64_t Sk, int causal, int cus) {
  BwdPlan pl = {};
  pl.R = (int)(H * Sq);
  pl.n_rt = 2 * (int)((pl.R + 63) / 64);
  pl.n_kb = (int)((Sk + kKeys - 1) / kKeys);
  pl.n_pairs = (pl.n_kb + 1) / 2;
  pl.kt_ld = kKeys * pl.n_kb;
  pl.n_groups = (pl.n_rt + 3) / 4;
  pl.cap = ds_cap_bytes();
  for (int g0 = 0; g0 < pl.n_groups;) {
    const BwdChunk c = next_chunk(pl, B, H, Sq, Sk, causal, cus, g0, pl.cap);
    ++pl.n_chunks;
    pl.max_pairs = max(pl.max_pairs, c.pairs);
    pl.max_items = max(pl.max_items, c.n_items);
    g0 = c.g1;
  }
  int64_t o = 0;
  pl.off_rstat = o; o += round256(B * pl.n_rt * kRows * 16);
  pl.off_roff = o; o += round256(B * pl.n_rt * kRows * 16);
  pl.off_kt = o;   o += round256(B * kDqk * (int64_t)pl.kt_ld * 2);
  pl.off_goff = o; o += round256(((int64_t)pl.n_groups + 1) * 4);
  pl.off_bmax = o; o += round256(B * pl.n_rt * 4);
  pl.off_gmax = o; o += 256;
  pl.off_ds = o;   o += round256(B * (int64_t)pl.max_pairs * kPairBytes);
  pl.off_part = o; o += round256((int64_t)pl.max_items * 2 * kPartFloats * 4);
  pl.off_acc = o;  o += pl.n_chunks > 1 ? round256(B * Sk * kDqk * 4) : 0;
  pl.bytes = o;
  return pl;
}

}  // namespace
}  // namespace dmla

using namespace dmla;

extern "C" int64_t dmla_bwd_workspace_bytes(int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t d_qk,
                                            int64_t d_v, int causal) {
  if (B <= 0 || H <= 0 || Sq <= 0 || Sk <= 0 || d_qk != kDqk || d_v != kDv) return 0;
  if (H * Sq > ((int64_t)1 << 30) || Sk > ((int64_t)1 << 30)) return 0;
  return make_plan(B, H, Sq, Sk, causal ? 1 : 0, device_cu_count()).bytes;
}

extern "C" int dmla_bwd_cache_latent(const void* q, const void* k_lat, const void* o, const void* dout,
                                     const float* m, const float* l, void* dq, void* dk_lat, int64_t B,
                                     int64_t H, int64_t Sq, int64_t Sk, int64_t d_qk, int64_t d_v,
                                     int64_t q_sb, int64_t q_sh, int64_t q_ss, int64_t k_sb, int64_t k_ss,
                                     int64_t o_sb, int64_t o_sh, int64_t o_ss, int64_t do_sb,
                                     int64_t do_sh, int64_t do_ss, int64_t dq_sb, int64_t dq_sh,
                                     int64_t dq_ss, int64_t dk_sb, int64_t dk_ss, int dq_fp32,
                                     int dk_fp32, float softmax_scale, int causal, void* workspace,
                                     int64_t workspace_bytes, dmla_stream_t stream) {
  clear_error();
  if (!q || !k_lat || !o || !dout || !m || !l || !dq || !dk_lat)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_bwd_cache_latent: null pointer argument");
  if (B < 0 || H < 0 || Sq < 0 || Sk < 0)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_bwd_cache_latent: negative size");
  if (d_qk != kDqk || d_v != kDv)
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_bwd_cache_latent: only d_qk=576, d_v=512 is compiled (got %lld, %lld)",
                (long long)d_qk, (long long)d_v);
  if (!(softmax_scale > 0.f) || !__builtin_isfinite(softmax_scale))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_bwd_cache_latent: softmax_scale must be finite and > 0");
  if (!aligned16(q) || !aligned16(k_lat) || !aligned16(o) || !aligned16(dout) || !aligned16(m) ||
      !aligned16(l) || !aligned16(dq) || !aligned16(dk_lat))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_bwd_cache_latent: tensors must be 16-byte aligned");
  if (!mult8(q_sb) || !mult8(q_sh) || !mult8(q_ss) || !mult8(k_sb) || !mult8(k_ss) || !mult8(o_sb) ||
      !mult8(o_sh) || !mult8(o_ss) || !mult8(do_sb) || !mult8(do_sh) || !mult8(do_ss))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_bwd_cache_latent: input strides must be multiples of 8 elements");
  if (H * Sq > ((int64_t)1 << 30) || Sk > ((int64_t)1 << 30))
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_bwd_cache_latent: size too large");
  if (B == 0 || H == 0 || Sq == 0) return DMLA_OK;
  if (Sk == 0) return fail(DMLA_ERR_INVALID_ARG, "dmla_bwd_cache_latent: Sk must be > 0");

  const BwdPlan pl = make_plan(B, H, Sq, Sk, causal ? 1 : 0, device_cu_count());
  if (workspace_bytes < pl.bytes || (!workspace && pl.bytes > 0))
    return fail(DMLA_ERR_WORKSPACE, "dmla_bwd_cache_latent: workspace of %lld bytes needed, got %lld",
                (long long)pl.bytes, (long long)workspace_bytes);
  if (!aligned16(workspace))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_bwd_cache_latent: workspace must be 16-byte aligned");

  BwdParams p = {};
  p.q = static_cast<const bf16*>(q);
  p.k = static_cast<const bf16*>(k_lat);
  p.o = static_cast<const bf16*>(o);
  p.dout = static_cast<const bf16*>(dout);
  p.m = m;
  p.l = l;
  p.dq = dq;
  p.dk = dk_lat;
  p.dq_fp32 = dq_fp32 ? 1 : 0;
  p.dq_rows16 = !dq_fp32 && mult8(dq_sb) && mult8(dq_sh) && mult8(dq_ss);
  p.dk_fp32 = dk_fp32 ? 1 : 0;
  p.q_sb = q_sb; p.q_sh = q_sh; p.q_ss = q_ss;
  p.k_sb = k_sb; p.k_ss = k_ss;
  p.o_sb = o_sb; p.o_sh = o_sh; p.o_ss = o_ss;
  p.do_sb = do_sb; p.do_sh = do_sh; p.do_ss = do_ss;
  p.dq_sb = dq_sb; p.dq_sh = dq_sh; p.dq_ss = dq_ss;
  p.dk_sb = dk_sb; p.dk_ss = dk_ss;
  p.B = (int)B; p.H = (int)H; p.Sq = (int)Sq; p.Sk = (int)Sk;
  p.causal = causal ? 1 : 0;
  p.hdiv = make_fastdiv((unsigned)H);
  p.scale = softmax_scale;
  p.scale_log2 = softmax_scale * kLog2e;
  p.R = pl.R; p.n_rt = pl.n_rt; p.n_kb = pl.n_kb; p.n_pairs = pl.n_pairs;
  p.kt_ld = pl.kt_ld; p.n_groups = pl.n_groups;
  char* ws = static_cast<char*>(workspace);
  p.rstat = reinterpret_cast<float4*>(ws + pl.off_rstat);
  p.roff = reinterpret_cast<int64_t*>(ws + pl.off_roff);
  p.kt = reinterpret_cast<_Float16*>(ws + pl.off_kt);
  p.goff = reinterpret_cast<int32_t*>(ws + pl.off_goff);
  p.bmax = reinterpret_cast<float*>(ws + pl.off_bmax);
  p.gmax = reinterpret_cast<unsigned*>(ws + pl.off_gmax);
  p.ds = reinterpret_cast<_Float16*>(ws + pl.off_ds);
  p.part = reinterpret_cast<float*>(ws + pl.off_part);
  p.dk_acc = dk_fp32 ? static_cast<float*>(dk_lat) : reinterpret_cast<float*>(ws + pl.off_acc);
  // The dQ launch holds a chunk's row groups plus the reduction's units, two per workgroup; a
  // dispatch counts its work-items in 32 bits.
  if ((B * (int64_t)pl.n_groups + 2 * (int64_t)pl.n_kb * B) * kDqThreads > 0xffffffffll)
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_bwd_cache_latent: grid too large");

  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(bwd_prep_kernel, dim3((unsigned)pl.n_rt, (unsigned)B), dim3(256), 0, s, p);
  hipLaunchKernelGGL(bwd_kt_kernel, dim3(kDqk / 64, (unsigned)pl.n_kb, (unsigned)B), dim3(256), 0, s, p);
  const int cus = device_cu_count();
  int chunk = 0;
  for (int g0 = 0; g0 < pl.n_groups; ++chunk) {
    // the plan's own cap: the chunks are the ones its workspace regions were sized for
    const BwdChunk c = next_chunk(pl, B, H, Sq, Sk, causal ? 1 : 0, cus, g0, pl.cap);
    p.rt_begin = 4 * c.g0;
    p.rt_end = min(pl.n_rt, 4 * c.g1);
    p.chunk_pairs = c.pairs;
    p.parts = c.parts;
    p.n_items = c.n_items;
    p.chunk = chunk;
    p.last_chunk = c.g1 >= pl.n_groups ? 1 : 0;
    const int64_t grid_kv = 8 * ((c.n_items + 7) / 8);
    hipLaunchKernelGGL(bwd_dkdv_kernel, dim3((unsigned)grid_kv), dim3(kBwdThreads), 0, s, p);
    // dQ tiles, then the dK_lat reduction's units two per workgroup (bwd_dq_kernel)
    const int64_t n_red = (int64_t)2 * pl.n_kb * B;
    hipLaunchKernelGGL(bwd_dq_kernel, dim3((unsigned)(B * (c.g1 - c.g0) + n_red)), dim3(kDqThreads), 0, s, p);
    g0 = c.g1;
  }
  return check_launch("dmla_bwd_cache_latent");
}
