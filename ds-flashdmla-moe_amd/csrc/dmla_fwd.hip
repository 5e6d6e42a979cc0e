// Flash-DMLA forward over a shared 576-wide latent cache: cache-latent prefill and paged decode.
//
// Semantics follow the reference's online-softmax forward (csrc/attention/fa2_fwd.cu:9-133 for
// the tile loop, csrc/attention/fa_fwd.cu:81-123 for the m/l/alpha recurrence and the 1/l guard)
// applied to the DMLA cache-latent mode of README.md:15: every head of a batch attends the same
// latent rows K_lat[b] (d_qk = 576 = 512 latent + 64 rope) and V_lat = K_lat[..., :512].
//
// MI355X design (one kernel family for both paths):
//  * A workgroup owns 64 query rows.  Rows are (position, head) pairs with the head fastest, so
//    all heads of a position share one causal limit and the workgroup streams ONE latent key
//    sequence: prefill is multi-query attention with M = 64 rows per key tile, decode puts 64
//    heads of one sequence in M.
//  * Key tiles of 32 rows x 576 (36 KB) are copied global -> LDS with 16-byte direct loads
//    (no VGPR staging) into a 3-slot ring.
//  * 8 waves, two per SIMD.  Wave w = 4p + 2h + k computes partial scores
//    S^T = K . Q^T for rows 32p..32p+31 (its pair), keys 16k..16k+15 (its key half) over dims
//    288h..288h+287 (its dims half; Q half in 72 VGPRs), on v_mfma_f32_16x16x32_bf16 whose
//    output leaves each lane one row's scores for 4 keys -- the B-operand layout PV needs.
//    The partner wave w^2 holds the other dims half; the two swap halves through LDS and each
//    finalises the softmax of 16 rows x 16 keys.  P of all 64 rows is shared through LDS and
//    wave w accumulates O for all 64 rows over output columns 64w..64w+63 (64 fp32 VGPRs),
//    reading V^T with ds_read_b64_tr_b16 (the slow LDS path, ~62 B/clk/CU on MI355X) once per
//    workgroup.  ~210 live registers per lane, so two waves share each SIMD.
//  * Software pipeline with one barrier per tile: iteration t runs PV(t-1) and the partial
//    scores of tile t+1 on the matrix cores with softmax(t) in between, and each wave refills
//    the chunk group it alone reads in PV (plus a rope slice) of the ring slot it just drained.
//  * Softmax in the exp2 domain against a per-row reference max fixed at the first tile: p
//    stays below 2^kHeadroom, so O is never rescaled.  Scores climbing past that headroom
//    trigger a recomputation of the row tile from a higher reference.
#include <mutex>
#include <type_traits>

#include "dmla_common.h"
#include "dmla_host.h"

namespace dmla {
namespace {

constexpr int kDqk = 576;
constexpr int kDv = 512;
constexpr int kPage = 64;                           // decode page size (tokens)
constexpr int kTileN = 32;                          // keys per LDS tile
constexpr int kGroups = kDqk / 64;                  // 9 chunk groups of 64 columns (128 B)
constexpr int kTileBytes = kGroups * kGroupBytes;   // 36 KB
constexpr int kRing = 3;                            // ring slots
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kRowsPerWG = 64;
constexpr int kKcHalf = kDqk / 32 / 2;              // 9 k-steps per dims half
constexpr int kDbWave = kDv / 16 / kWaves;          // 4 output column blocks (64 columns) per wave
constexpr int kXBytes = kWaves * 1024;              // partial-score exchange, one buffer
constexpr int kPBytes = 4 * 1024;                   // P of the 64 rows as MFMA B operands
constexpr int kMaxSegPages = 128;                   // page indices of a decode segment: two VGPRs
constexpr int kXOffset = kRing * kTileBytes;
constexpr int kPOffset = kXOffset + kRing * kXBytes;  // partial scores and P follow the ring's period
constexpr int kRowOffset = kPOffset + kRing * kPBytes;  // per-row exchange [3][2 key halves][64]
constexpr int kFlagOffset = kRowOffset + 3 * 2 * kRowsPerWG * 4;
constexpr int kPageOffset = kFlagOffset + 2 * kWaves * 4;
// Q staging at the start of a work item: the 64 rows (1152 B each, padded by one 16-byte chunk
// so that 16 consecutive rows fall into distinct LDS banks) from ring slot 1 on.  Slot 0 takes
// the first key tile meanwhile; the region reaches 1 KB into partial-score buffer 0, which is
// first written after Q has been read out.
constexpr int kQRowBytes = kDqk * 2 + 16;
constexpr int kQChunks = kRowsPerWG * kQRowBytes / 16;   // 4672 16-byte chunks, 73 per row
constexpr int kQOffset = kTileBytes;
static_assert(kQOffset + kRowsPerWG * kQRowBytes <= kXOffset + kXBytes, "Q staging fits before buffer 1");
constexpr int kLdsBytes = kPageOffset;
constexpr float kHeadroom = 32.0f;                  // log2 headroom of p over the reference max
static_assert(kLdsBytes <= 160 * 1024, "LDS budget");
static_assert(kPage % kTileN == 0, "a page holds whole tiles");
static_assert(kTileN == kTileRows, "key tiles use the shared 32-row tile layout");
static_assert(kGroups == kWaves + 1, "each wave copies its PV chunk group; the rope group is shared");

// Scheduling template of one pipelined tile iteration: 22 LDS operand reads (partials, P, V,
// K) feeding 34 MFMAs, with vector ALU work slotted between them.  A few reads run ahead; the
// rest are interleaved so in-flight operands stay within the register budget.
__device__ __forceinline__ void iteration_schedule() {
  __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
}

struct MqaParams {
  const bf16* q;
  const bf16* kv;
  bf16* o;
  float* m;        // prefill statistics (nullable)
  float* l;
  float* lse;      // decode log-sum-exp (nullable)
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_ss;  // prefill: batch/row strides of K_lat; decode: page/row strides
  int64_t o_sb, o_sh, o_ss;
  int B, H, Sq, Sk;
  FastDiv hdiv;        // division by H (prefill rows are (position, head) with the head fastest)
  float scale_log2;    // softmax_scale * log2(e)
  int causal;
  int n_row_tiles;     // prefill: ceil(H*Sq / 64)
  // decode
  const int32_t* block_table;
  const int32_t* seqlens;
  int64_t bt_sb;
  int num_pages;
  int max_pages;
  int head_groups;     // ceil(H / 64)
  int n_ranges;        // R of the decode plan
  const int32_t* plan; // decode plan (see decode_plan_kernel); unused when plan_inline
  int plan_inline;     // every workgroup builds the plan in LDS (B <= kInlinePlanB, R <= kInlinePlanR)
  int32_t* plan_out;   // with plan_inline: workgroup 0 stores the plan here (the combine reads it)
  bf16* part_o;        // [slots, H, 512] normalised partial outputs, rounded to bf16
  float* part_lse;     // [slots, H]
};

struct Work {
  int b, row0, tile_begin, tile_end, split, nsplit, ctx, page_begin, slot;
};

// ---- decode plan --------------------------------------------------------------------------
// The key tiles (32 tokens) of all sequences, in order, are cut into R ranges; range r is
// processed by head_groups workgroups on one XCD, one per group of 64 heads.  Every piece of
// a sequence in a range is one split of that sequence (a segment of the workgroup's work);
// sequences with more than one split are merged by the LSE combine.  A segment costs a fixed
// prologue and epilogue (loading Q and the first tile, writing the output) of about
// kSegCost tiles, so the ranges are equal in the weighted space where each nonempty sequence
// is preceded by kSegCost virtual tiles: range r starts at weighted position r W with
// W = ceil(weighted total / R), moved to the sequence's first tile when it falls among the
// virtual ones.  The work per workgroup is then about the same whatever the context lengths.
// Layout (int32): header[8] = {B, R, W, total tiles, total splits, kSegCost, 0, 0}, then
// tile_prefix[B + 1], split_base[B + 1] (first partial slot of each sequence), num_splits[B],
// first_range[B], range_start[R + 1] (first tile of each range, in the concatenated tile
// space), range_first_b[R] (the sequence holding the range's first tile).
constexpr int kPlanHeader = 8;
constexpr int kSegCost = 10;   // per-segment cost in tiles: a launch timeline fits 0.92 us per tile + 9.2 us per segment
constexpr int kMaxSegTiles = 2 * kMaxSegPages - 2;   // a segment's pages fit its page registers
__host__ __device__ inline int64_t plan_ints(int64_t B, int64_t R) { return kPlanHeader + 4 * B + 2 + 2 * R + 1; }
// Inline plan: the decode kernel builds the plan itself, in LDS past the pipeline's area, when
// the batch and the range count fit (the common serving case); the standalone plan kernel and
// its global round trips are then skipped.
constexpr int kInlinePlanB = kThreads;   // one sequence per thread
constexpr int kInlinePlanR = kThreads;
struct InlinePlan {
  int tp[kInlinePlanB + 1];    // tile prefix
  int rfb[kInlinePlanR];       // first sequence of each range
  int ns[kInlinePlanB];        // split count
  int fr[kInlinePlanB];        // first range
  int sb[kInlinePlanB + 1];    // first partial slot
  int ctx[kInlinePlanB];       // context length, clamped to the block table
  int rs[kInlinePlanR + 1];    // range starts
  int tmp[kWaves];             // scan scratch
};
constexpr int kDecodeLdsBytes = kLdsBytes + (int)sizeof(InlinePlan);
static_assert(kDecodeLdsBytes <= 160 * 1024, "LDS budget (decode)");

template <bool kDecode, int kHalf>
__device__ __noinline__ void mqa_fwd_exact(const MqaParams* params, Work wk, DMLA_LDS char* lds, int wave, int lane);

// kExact = false: the fast path, reference max = the row max of the first tile; on overflow it
// hands the whole row tile to the kExact = true path, which first computes every row's exact
// max in a scores-only pass and then runs the same pipeline against it.  The fast path never
// contains the (register-hungry) retry code.
template <bool kDecode, int kHalf, bool kExact>
__device__ __forceinline__ void mqa_fwd_body(const MqaParams& p, const MqaParams* params, const Work& wk,
                                             DMLA_LDS char* lds, const int wave, const int lane_arg) {
  // Per-lane values are derived here, per work item, rather than once per kernel: kept live
  // across every item's tile loop they would be spilled, and each reload's vmcnt wait would
  // drain the copies and stores in flight.
  (void)lane_arg;
  const int lane = fresh_lane_id();
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int pair = wave >> 2;          // rows 32 pair .. +31 for the partial scores
  const int kh = wave & 1;             // key half of the tile: keys 16 kh .. +15
  const int rb = wave >> 1;            // own softmax rows 16 rb .. +15 (= 2 pair + kHalf)
  const int b = wk.b, row0 = wk.row0, tile_begin = wk.tile_begin, tile_end = wk.tile_end;
  DMLA_LDS char* pbuf = lds + kPOffset;
  DMLA_LDS float* rowx = reinterpret_cast<DMLA_LDS float*>(lds + kRowOffset);
  DMLA_LDS int* flags = reinterpret_cast<DMLA_LDS int*>(lds + kFlagOffset);

  const int nrows = kDecode ? p.H : p.H * p.Sq;
  const int own_row = row0 + 16 * rb + l16;
  auto limit_of = [&](int r) -> int {
    if constexpr (!kDecode) {
      const int pos = fast_div(r, p.hdiv);
      return p.causal ? min(pos + (p.Sk - p.Sq), p.Sk - 1) : p.Sk - 1;
    } else {
      return wk.ctx - 1;
    }
  };
  // Rows past the last one (the tail of the last item) compute the item's first row again: its
  // Q, its limit (the smallest of the item), output discarded; so no tile below that limit needs
  // a mask for any row of the item.
  const int own_lim = limit_of(own_row < nrows ? own_row : row0);
  // First tile holding a key past some row's limit (the item's first row has the smallest).
  const int first_mask_tile = max(limit_of(row0) + 1, 0) / kTileN;

  // ---- Q: the pair's 32 rows, this wave's dims half, as MFMA B operand --------------------
  // lane holds Q[row 32 pair + 16 qg + l16][288 kHalf + 32 c + 8 g .. +7]; loaded through LDS
  // below (one copy per workgroup, whole rows per copy instruction).
  bf16x8 qreg[2][kKcHalf];

  // ---- tile staging ----------------------------------------------------------------------
  // Wave w copies chunk group w -- the output columns it alone reads in PV -- in 4 copies of 8
  // rows, and waves 0..3 also copy rows 8w..8w+7 of the rope group 8, which only QK reads.
  // A ring slot can therefore be refilled by each wave as soon as its own PV reads of it are
  // done, without a barrier.  Lane l covers row 8r + l/8 at physical chunk l%8, i.e. logical
  // chunk (l%8) ^ swz(row); the group's 128-byte column offset goes into the scalar base (an
  // instruction offset would also move the LDS address).
  bool bad_page = false;
  int seg_pages[2] = {0, 0};
  if constexpr (kDecode) {
    const int npg = (tile_end + (kPage / kTileN) - 1) / (kPage / kTileN) - wk.page_begin;
    // The plan keeps segments within the two page registers (decode_ranges); a segment past
    // them would read wrapped (valid but wrong) pages, so its output is poisoned instead.
    bad_page = npg > kMaxSegPages;
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (64 * h + lane < npg) seg_pages[h] = p.block_table[b * p.bt_sb + wk.page_begin + 64 * h + lane];
  }
  const int row_stride_bytes = (int)(p.k_ss * 2);
  // Row 8r + l/8 of a copy has swizzle swz(8 (r & 1) + l/8): two column variants per lane.
  const int dma_lrow = lane >> 3;
  // (Two scalars and an xor, not a two-element array: an array indexed by the runtime rope row
  // would be placed in LDS by the compiler, one ds_read and a full lgkmcnt wait per copy.)
  const unsigned dma_col0 = 16u * ((lane & 7) ^ swz(dma_lrow));
  const unsigned dma_col_x = dma_col0 ^ (16u * ((lane & 7) ^ swz(8 + dma_lrow)));
  const unsigned dma_lane = (unsigned)(dma_lrow * row_stride_bytes);
  const int dma_rope_r = wave & 3;   // rope copy of waves 0..3: rows 8w .. 8w+7
  const int ncopies = wave < 4 ? 5 : 4;
  const unsigned lds_base = lds_addr(lds);
  // Scalar base of tile `tile` (clamped into the work item, so copies past the end re-read the
  // last tile: finite data in a slot nobody reads) and its count of valid rows.
  auto tile_src = [&](int tile, int& valid_rows) -> const char* {
    tile = min(tile, tile_end - 1);
    if constexpr (!kDecode) {
      valid_rows = p.Sk - tile * kTileN;
      return reinterpret_cast<const char*>(p.kv + b * p.k_sb + (int64_t)tile * kTileN * p.k_ss);
    } else {
      // The segment's page indices sit in two VGPRs, lane i holding pages i and 64 + i of it:
      // a lane read gives the index in an SGPR, with no memory access or wait.
      // Branch-free (selects on scalars), so the pipelined iteration stays one basic block.
      const int idx = tile / (kPage / kTileN) - wk.page_begin;
      const int pa = __builtin_amdgcn_readlane(seg_pages[0], idx & 63);
      const int pb = __builtin_amdgcn_readlane(seg_pages[1], idx & 63);
      int page = idx < 64 ? pa : pb;
      const bool bad = page < 0 || page >= p.num_pages;
      bad_page = bad_page || bad;
      page = bad ? 0 : page;
      valid_rows = wk.ctx - tile * kTileN;
      return reinterpret_cast<const char*>(p.kv + (int64_t)page * p.k_sb +
                                           (int64_t)(tile % (kPage / kTileN)) * kTileN * p.k_ss);
    }
  };
  // Ring slot of tile t, relative to the item's first tile (t >= tile_begin - 1); the partial
  // scores and P of tile t use exchange buffer slot_idx(t) of three as well.  The bulk of the
  // loop passes these indices as compile-time constants.
  auto slot_idx = [&](int t) { return (t - tile_begin + 2 * kRing) % kRing; };
  auto slot_addr = [&](int tile) { return lds_base + slot_idx(tile) * kTileBytes; };
  // Copy k (0..ncopies-1) of this wave; rows past the valid range re-read row 0 of the tile
  // (finite data, masked later).
  f32x4 oacc[kDbWave][4];   // O^T[64 wave + 16 d + 4 g + i][16 qg + l16]
  bf16x8 vpre[kDbWave];     // V operands of the next PV (read one iteration ahead)
  // Lane offsets of a full tile's copies (the copy's 8 r rows go into the scalar base): two
  // column variants, rows 8r + l/8 with r even / odd.
  const unsigned dma_off_even = dma_lane + dma_col0;
  const unsigned dma_off_odd = dma_lane + (dma_col0 ^ dma_col_x);
  // check_tag: the tile may end early (the last tile of a sequence); rows past the valid range
  // then re-read row 0 of the tile (finite data, masked later).  after_tag: the copy refills
  // this wave's chunk group of the slot whose V operands it read last iteration into vpre;
  // vpre as asm operands orders the copy after those reads.
  auto copy_part = [&](int k, const char* src, int valid_rows, unsigned dst, auto after_tag, auto check_tag) {
    const int r = k < 4 ? k : dma_rope_r;
    const char* gbase = k < 4 ? src + wave * 128 : src + 8 * 128;
    unsigned off;
    if constexpr (decltype(check_tag)::value) {
      const unsigned col = dma_col0 ^ ((r & 1) ? dma_col_x : 0u);
      off = 8 * r + dma_lrow < valid_rows ? dma_lane + (unsigned)(8 * r * row_stride_bytes) + col : col;
    } else {
      gbase += (int64_t)(8 * r) * row_stride_bytes;
      off = (r & 1) ? dma_off_odd : dma_off_even;
    }
    const unsigned ldst = k < 4 ? dst + wave * kGroupBytes + k * 1024 : dst + 8 * kGroupBytes + dma_rope_r * 1024;
    if constexpr (decltype(after_tag)::value) dma16_after_v(gbase, off, ldst, vpre[0], vpre[1], vpre[2], vpre[3]);
    else dma16(gbase, off, ldst);
  };
  using Plain = std::integral_constant<bool, false>;
  using Checked = std::integral_constant<bool, true>;
  auto stage = [&](int tile, int slot_tile) {
    int valid_rows;
    const char* src = tile_src(tile, valid_rows);
    const unsigned dst = slot_addr(slot_tile);
#pragma unroll
    for (int k = 0; k < 4; ++k) copy_part(k, src, valid_rows, dst, Plain{}, Checked{});
    if (ncopies > 4) copy_part(4, src, valid_rows, dst, Plain{}, Checked{});
  };

  // ---- per-lane LDS byte offsets -----------------------------------------------------------
  // K operand (A of S^T) for global k-step c: row 16 kh + l16, logical chunk 4c + g = chunk
  // group c/2, in-group position 4(c&1) + g.
  const int ksw = swz(l16);
  const int kh_off = kh * 16 * 128;
  const int k_off[2] = {kh_off + l16 * 128 + 16 * (g ^ ksw), kh_off + l16 * 128 + 16 * ((4 + g) ^ ksw)};
  // V operand (A of O^T) through transpose reads: lane 4e+q of group g reads row 4g+e (and
  // 16+4g+e), columns 16db + 4q .. +3 = chunk group db/4, in-group chunk 2(db%4) + (q>>1),
  // byte 8(q&1) inside the chunk.  This wave's output columns 64w.. are chunk group w.
  const int e = l16 >> 2, qq = l16 & 3;
  const int vsw = swz(4 * g + e);
  int v_off[kDbWave];
#pragma unroll
  for (int d = 0; d < kDbWave; ++d)
    v_off[d] = wave * kGroupBytes + (4 * g + e) * 128 + 16 * ((2 * d + (qq >> 1)) ^ vsw) + 8 * (qq & 1);
  // Exchange slots: partial scores [buffer][wave][lane] x 16 B; P [buffer][row block][lane] x
  // 16 B with the key-half owner writing bytes 8 kh .. 8 kh + 7.
  const int x_post = wave * 1024 + lane * 16;
  const int x_take = (wave ^ 2) * 1024 + lane * 16;
  const int p_post = rb * 1024 + lane * 16 + kh * 8;
  // LDS address lane_off + add as one register, opaque to the compiler: the accesses through it
  // then carry their constant parts as instruction offsets (one add per operand stream and
  // iteration, instead of an add per access of a runtime ring slot).
  auto lds_at = [&](int lane_off, int add) {
    unsigned r;
    asm("v_add_u32 %0, %1, %2" : "=v"(r) : "v"(lane_off), "s"(add));
    return reinterpret_cast<DMLA_LDS char*>(static_cast<uintptr_t>(r));
  };
  const int lds0 = (int)lds_base;


  float mref;               // max the accumulators of the own rows are relative to
  float mtrue;              // exact running max of this lane's keys of its own row
  float lsum;               // this lane's partial row sum relative to mref
  float mref_init = kNegInf;
  const float scale_log2 = p.scale_log2;

  // PV of tile tp for this wave's 64 columns and all 64 rows.
  // The V operands of a tile are read one iteration ahead of its PV (vload), off the burst
  // of P reads that follows each barrier; a slot's data is complete from the barrier after
  // its copies landed until this wave's next copies into it.
  auto vload = [&](int slot) {
#pragma unroll
    for (int d = 0; d < kDbWave; ++d) {
      const DMLA_LDS char* vb = lds_at(v_off[d], lds0 + slot * kTileBytes);
      const bf16x4 v0 = lds_read_tr16(reinterpret_cast<const DMLA_LDS bf16x4*>(vb));
      const bf16x4 v1 = lds_read_tr16(reinterpret_cast<const DMLA_LDS bf16x4*>(vb + 16 * 128));
      vpre[d] = concat(v0, v1);
    }
  };
  auto pv = [&](int buf) {
    const DMLA_LDS char* pb = lds_at(lane * 16, lds0 + kPOffset + buf * kPBytes);
    bf16x8 pall[4];
#pragma unroll
    for (int qg = 0; qg < 4; ++qg) pall[qg] = *reinterpret_cast<const DMLA_LDS bf16x8*>(pb + qg * 1024);
#pragma unroll
    for (int d = 0; d < kDbWave; ++d)
#pragma unroll
      for (int qg = 0; qg < 4; ++qg) oacc[d][qg] = mfma_bf16(vpre[d], pall[qg], oacc[d][qg]);
  };
  // Partial S^T[key 16 kh + 4g + i][pair row 16 qg + l16] of the tile in ring slot q_slot over
  // this wave's dims half; the copies of tile `ctile` into slot c_slot are issued between the
  // k-steps.  kCopy: 0 when there is no tile to fetch; 1 copies into a slot nobody has read
  // since the last barrier; 2 refills this wave's chunk group of the slot whose V operands it
  // has just read into vpre (ordered after those reads by register dependences, so the K reads
  // can run ahead of it).
  auto qk = [&](int q_slot, f32x4 (&sacc)[2], int ctile, int c_slot, auto copy_tag, auto check_tag) {
    constexpr int kCopy = decltype(copy_tag)::value;
    const DMLA_LDS char* kb0 = lds_at(k_off[0], lds0 + q_slot * kTileBytes);
    const DMLA_LDS char* kb1 = lds_at(k_off[1], lds0 + q_slot * kTileBytes);
    int valid_rows = 0;
    const char* src = nullptr;
    unsigned dst = 0;
    if constexpr (kCopy) {
      src = tile_src(ctile, valid_rows);
      dst = lds_base + c_slot * kTileBytes;
    }
    sacc[0] = sacc[1] = f32x4{0.f, 0.f, 0.f, 0.f};
    // K operands are read two k-steps ahead of their MFMAs.
    auto kread = [&](int c) {
      const int cc = kHalf * kKcHalf + c;
      return lds_read_b128(reinterpret_cast<const DMLA_LDS bf16x8*>(((cc & 1) ? kb1 : kb0) + (cc >> 1) * kGroupBytes));
    };
    bf16x8 kb[3];
    kb[0] = kread(0);
    kb[1] = kread(1);
#pragma unroll
    for (int c = 0; c < kKcHalf; ++c) {
      if (c + 2 < kKcHalf) kb[(c + 2) % 3] = kread(c + 2);
      const bf16x8 a = kb[c % 3];
      sacc[0] = mfma_bf16(a, qreg[0][c], sacc[0]);
      sacc[1] = mfma_bf16(a, qreg[1][c], sacc[1]);
      if constexpr (kCopy != 0) {
        using Tag = std::integral_constant<bool, kCopy == 2>;
        if (c < 4) copy_part(c, src, valid_rows, dst, Tag{}, check_tag);
        if (c == 4 && ncopies > 4) copy_part(4, src, valid_rows, dst, Tag{}, check_tag);
      }
    }
  };
  using CopyOn = std::integral_constant<int, 1>;
  using CopyOff = std::integral_constant<int, 0>;
  // Copy distance.  Decode streams its tiles from HBM, so its copies run three tiles ahead:
  // iteration t refills this wave's part of slot(t) with tile t+3 between the k-steps of
  // QK(t+1), once its V operands of tile t are read (the other waves read that part of no slot,
  // and every wave's K reads of tile t were done an iteration earlier); a tile's copies then
  // have two iterations to land.  The prefill's tiles come from L2: its copies run two tiles
  // ahead, into slot(t-1) during QK(t+1), which it runs before PV(t-1).  At the start of
  // iteration t a wave waits for its copies of tile t+1; in decode those of tile t+2, its newest
  // batch of ncopies instructions, stay in flight when they exist.
  constexpr int kAhead = kDecode ? 3 : 2;
  auto wait_tile = [&](bool newer_batch) {
    if (!newer_batch) wait_vmem();
    else if (ncopies > 4) wait_vmem_le<5>();
    else wait_vmem_le<4>();
  };
  using CopyAfterV = std::integral_constant<int, 2>;
  auto post_partial = [&](int buf, const f32x4 (&sacc)[2]) {
    *reinterpret_cast<DMLA_LDS f32x4*>(lds_at(x_post, lds0 + kXOffset + buf * kXBytes)) = sacc[1 - kHalf];
  };
  auto take_scores = [&](int buf, const f32x4 (&sacc)[2]) {
    return sacc[kHalf] + *reinterpret_cast<const DMLA_LDS f32x4*>(lds_at(x_take, lds0 + kXOffset + buf * kXBytes));
  };
  auto masked = [&](int tq, const f32x4& s, float (&sr)[4]) {
    const int key0 = tq * kTileN + 16 * kh + 4 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) sr[i] = key0 + i > own_lim ? kNegInf : s[i];
  };
  // Max over both key halves of a per-row value (one LDS round trip; `slot` picks the buffer).
  auto row_max_both_halves = [&](float v, int slot) {
    rowx[(slot * 2 + kh) * kRowsPerWG + 16 * rb + l16] = v;
    __syncthreads();
    return fmaxf(v, rowx[(slot * 2 + (kh ^ 1)) * kRowsPerWG + 16 * rb + l16]);
  };

  // This wave's row statistics over its key half (l and the exact max of its own 16 rows),
  // posted for the partner wave before the last barrier of the loop.
  float lhalf = 0.f, mhalf = kNegInf;
  auto post_row_stats = [&]() {
    lhalf = group_sum(lsum);
    mhalf = group_max(mtrue);
    rowx[(2 * 2 + kh) * kRowsPerWG + 16 * rb + l16] = lhalf;
    rowx[(0 * 2 + kh) * kRowsPerWG + 16 * rb + l16] = mhalf;
  };

  f32x4 sacc[2];
#pragma unroll
  for (int d = 0; d < kDbWave; ++d)
#pragma unroll
    for (int qg = 0; qg < 4; ++qg) oacc[d][qg] = f32x4{0.f, 0.f, 0.f, 0.f};
  mtrue = kNegInf;
  lsum = 0.f;
  mref = kNegInf;
  bool overflow = false;

  // ---- Q through LDS, with the first key tile in flight beside it ---------------------------
  // Chunk k of the staging area is 16-byte chunk k % 73 of row k / 73 (chunk 72 is the row's
  // padding and re-reads chunk 0); rows past the last one re-read row 0 of the item.
  auto stage_q = [&]() {
    const unsigned qbase = lds_base + kQOffset;
    for (int i = wave; i * 64 < kQChunks; i += kWaves) {
      const int k = i * 64 + lane;
      const int rl = k / (kQRowBytes / 16), ch = k - rl * (kQRowBytes / 16);
      const int rq = row0 + rl;
      const int r = rq < nrows ? rq : row0;
      const bf16* qrow;
      if constexpr (!kDecode) {
        const int pos = fast_div(r, p.hdiv), head = r - pos * p.H;
        qrow = p.q + b * p.q_sb + head * p.q_sh + pos * p.q_ss;
      } else {
        qrow = p.q + b * p.q_sb + r * p.q_sh;
      }
      dma16_addr(qrow + 8 * (ch < kDqk / 8 ? ch : 0), qbase + i * 1024);
    }
  };
  if constexpr (!kDecode) {
    if (tile_begin < tile_end) stage(tile_begin, tile_begin);
    stage_q();
  } else {
    // The Q copies go out first; the first tile's page index then comes through the scalar
    // cache (lgkmcnt), so the Q copies and the page-index vector loads above stay in flight
    // while it is fetched: the first tile's copies wait for one lookup instead of for the vector
    // loads and everything issued with them.
    stage_q();
    int page0 = 0;
    if (tile_begin < tile_end) {
      const uint64_t ba = reinterpret_cast<uint64_t>(p.block_table + b * p.bt_sb + tile_begin / (kPage / kTileN));
      const uint64_t bu = ((uint64_t)__builtin_amdgcn_readfirstlane((unsigned)(ba >> 32)) << 32) |
                          (unsigned)__builtin_amdgcn_readfirstlane((unsigned)ba);
      asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(page0) : "s"(bu) : "memory");
      const bool bad = page0 < 0 || page0 >= p.num_pages;
      bad_page = bad_page || bad;
      const int pg = bad ? 0 : page0;
      const char* src = reinterpret_cast<const char*>(p.kv + (int64_t)pg * p.k_sb +
                                                      (int64_t)(tile_begin % (kPage / kTileN)) * kTileN * p.k_ss);
      const unsigned dst = slot_addr(tile_begin);
      const int valid_rows = wk.ctx - tile_begin * kTileN;
#pragma unroll
      for (int k = 0; k < 4; ++k) copy_part(k, src, valid_rows, dst, Plain{}, Checked{});
      if (ncopies > 4) copy_part(4, src, valid_rows, dst, Plain{}, Checked{});
    }
  }
  wait_vmem();
  __syncthreads();
#pragma unroll
  for (int qg = 0; qg < 2; ++qg)
#pragma unroll
    for (int c = 0; c < kKcHalf; ++c)
      qreg[qg][c] = lds_read_b128(reinterpret_cast<const DMLA_LDS bf16x8*>(
          lds + kQOffset + (32 * pair + 16 * qg + l16) * kQRowBytes + (kHalf * (kDqk / 2) + 32 * c + 8 * g) * 2));
  __syncthreads();   // Q is read out before the tile copies below reuse its LDS

  if (tile_begin < tile_end) {
    if constexpr (kExact) {
      // Scores-only pass for the exact row max (rows without any key keep -inf); slot(t0)
      // already holds tile t0.
      float mx = kNegInf;
      for (int t = tile_begin; t < tile_end; ++t) {
        wait_vmem();
        __syncthreads();
        if (t + 1 < tile_end) qk(slot_idx(t), sacc, t + 1, slot_idx(t + 1), CopyOn{}, Checked{});
        else qk(slot_idx(t), sacc, t + 1, slot_idx(t + 1), CopyOff{}, Checked{});
        post_partial(slot_idx(t), sacc);
        __syncthreads();
        float sr[4];
        masked(t, take_scores(slot_idx(t), sacc), sr);
        mx = fmaxf(mx, fmaxf(fmaxf(sr[0], sr[1]), fmaxf(sr[2], sr[3])) * scale_log2);
      }
      wait_vmem();
      mref_init = row_max_both_halves(group_max(mx), 1);
      __syncthreads();
    }

    // Prologue: the V operands of a tile t0-1 are zero and P(t0-1) = 0, so the PV of the first
    // iteration adds nothing; slot(t0) holds t0 (restaged after the exact path's scores pass);
    // its partial scores are posted and the copies of t0+1 and t0+2 are in flight.  The fast path's
    // reference max of each row is its max over tile t0 (every row with any key has one in
    // the first tile of its work item).
#pragma unroll
    for (int d = 0; d < kDbWave; ++d) vpre[d] = bf16x8{};
    *reinterpret_cast<DMLA_LDS bf16x4*>(pbuf + slot_idx(tile_begin - 1) * kPBytes + p_post) = bf16x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (kExact) {
      stage(tile_begin, tile_begin);
      wait_vmem();
      __syncthreads();
    }
    if (tile_begin + 1 < tile_end) qk(0, sacc, tile_begin + 1, 1, CopyOn{}, Checked{});
    else qk(0, sacc, tile_begin + 1, 1, CopyOff{}, Checked{});
    if (kAhead == 3 && tile_begin + 2 < tile_end) stage(tile_begin + 2, tile_begin + 2);
    post_partial(0, sacc);
    if constexpr (!kExact) {
      __syncthreads();
      float sr[4];
      masked(tile_begin, take_scores(0, sacc), sr);
      const float mhalf = group_max(fmaxf(fmaxf(sr[0], sr[1]), fmaxf(sr[2], sr[3])) * scale_log2);
      mref = row_max_both_halves(mhalf, 0);
    } else {
      mref = mref_init;
    }

    // Iteration t: PV(t-1) and the partial scores of tile t+1 on the matrix cores with softmax(t)
    // in between, then P(t) and the partials of t+1 are posted.  One barrier per tile.  Ring:
    // PV(t-1) uses the V operands read last iteration, slot(t) is read for the next PV, QK(t+1)
    // reads slot(t+1), and the copies of tile t+kAhead go into slot(t+kAhead) (see kAhead).
    // kKind 0 is the steady state; kKind 1 (t+kAhead past the end) copies nothing and kKind 2
    // (the last tile) computes no scores for a tile t+1.  kPh >= 0 would pass t's ring phase as
    // a constant (the loop below passes it at run time); kMask: some row's causal or length
    // limit falls inside tile t; kCheck: tile t+kAhead may be the item's partial last tile.  An
    // overflow of the reference max is only recorded per lane here and acted on once, after the
    // last tile: inputs that trigger it are rare, and a per-tile exchange of flags would cost
    // every tile LDS traffic.
    auto iteration = [&](int t, auto kind_tag, auto phase_tag, auto mask_tag, auto check_tag) {
      constexpr int kKind = decltype(kind_tag)::value;
      constexpr int kPh = decltype(phase_tag)::value;
      const int s_cur = kPh >= 0 ? kPh : (t - tile_begin) % kRing;
      const int s_next = s_cur == kRing - 1 ? 0 : s_cur + 1, s_prev = s_cur == 0 ? kRing - 1 : s_cur - 1;
      wait_tile(kAhead == 3 && t + 2 < tile_end);   // this wave's copies of tile t+1 have landed
      __syncthreads();   // partials(t) and P(t-1) posted; tile t+1 complete
      const f32x4 s = take_scores(s_cur, sacc);
      if constexpr (kAhead == 3) {
        pv(s_prev);
        vload(s_cur);
        if constexpr (kKind == 0) qk(s_next, sacc, t + 3, s_cur, CopyAfterV{}, check_tag);
        if constexpr (kKind == 1) qk(s_next, sacc, 0, 0, CopyOff{}, check_tag);
      } else {
        // QK first, so that its partials are ready long before they are posted (vpre still
        // holds the V operands of slot(t-1), the slot refilled here)
        if constexpr (kKind == 0) qk(s_next, sacc, t + 2, s_prev, CopyAfterV{}, check_tag);
        if constexpr (kKind == 1) qk(s_next, sacc, 0, 0, CopyOff{}, check_tag);
        pv(s_prev);
        vload(s_cur);
      }

      // ---- softmax of the own 16 rows x 16 keys (exp2 domain) ------------------------------
      float sr[4];
      if constexpr (decltype(mask_tag)::value) {
        masked(t, s, sr);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) sr[i] = s[i];
      }
      const float mloc = fmaxf(fmaxf(sr[0], sr[1]), fmaxf(sr[2], sr[3])) * scale_log2;  // scale > 0
      mtrue = fmaxf(mtrue, mloc);
      overflow = overflow || mloc > mref + kHeadroom;
      const float ms = mref == kNegInf ? 0.f : mref;
      bf16x4 pk;  // keys 16 kh + 4g .. +3 of the own row
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float pj = fast_exp2(__builtin_fmaf(sr[j], scale_log2, -ms));
        lsum += pj;
        pk[j] = (bf16)pj;
      }
      *reinterpret_cast<DMLA_LDS bf16x4*>(lds_at(p_post, lds0 + kPOffset + s_cur * kPBytes)) = pk;
      if constexpr (kKind != 2) {
        post_partial(s_next, sacc);
        iteration_schedule();
      }
    };
    using K0 = std::integral_constant<int, 0>;
    using K1 = std::integral_constant<int, 1>;
    using K2 = std::integral_constant<int, 2>;
    using PhRt = std::integral_constant<int, -1>;
    using Mask = std::true_type;
    using NoMask = std::false_type;
    int t = tile_begin;
    if constexpr (!kExact) {
      // The bulk: tiles below every row's limit, whose copies fetch full tiles.  The remaining
      // tiles take the general iteration.
      const int fast_end = min(first_mask_tile, tile_end - kAhead - 1);
      for (; t < fast_end; ++t) iteration(t, K0{}, PhRt{}, NoMask{}, Plain{});
    }
    for (; t + kAhead < tile_end; ++t) iteration(t, K0{}, PhRt{}, Mask{}, Checked{});
    for (; t + 1 < tile_end; ++t) iteration(t, K1{}, PhRt{}, Mask{}, Checked{});
    iteration(t, K2{}, PhRt{}, Mask{}, Checked{});
    post_row_stats();
    if constexpr (!kExact) flags[wave] = __any(overflow) ? 1 : 0;
    wait_vmem();
    // lgkmcnt(0): this wave's reads of the ring are done before any wave stages its output there
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __syncthreads();     // P(end-1), the row statistics and the overflow flags posted
    if constexpr (!kExact) {
      const i32x4 f0 = *reinterpret_cast<const DMLA_LDS i32x4*>(flags);
      const i32x4 f1 = *reinterpret_cast<const DMLA_LDS i32x4*>(flags + 4);
      if (((f0[0] | f0[1] | f0[2] | f0[3]) | (f1[0] | f1[1] | f1[2] | f1[3])) != 0) {
        mqa_fwd_exact<kDecode, kHalf>(params, wk, lds, wave, lane);
        return;
      }
    }
    pv(slot_idx(tile_end - 1));
  } else {
    post_row_stats();
    __syncthreads();
  }

  // ---- epilogue ---------------------------------------------------------------------------
  // Row statistics over both key halves, and 1/l of the 64 rows this wave scales (rows
  // 16 qg + l16), read from the statistics both key-half waves posted.
  const bool poison = kDecode && __any(bad_page);
  const float nanv = __builtin_nanf("");
  const float ltot = lhalf + rowx[(2 * 2 + (kh ^ 1)) * kRowsPerWG + 16 * rb + l16];
  const float mt = fmaxf(mhalf, rowx[(0 * 2 + (kh ^ 1)) * kRowsPerWG + 16 * rb + l16]);
  float inv_l[4];
#pragma unroll
  for (int qg = 0; qg < 4; ++qg) {
    const float lr = rowx[(2 * 2 + 0) * kRowsPerWG + 16 * qg + l16] + rowx[(2 * 2 + 1) * kRowsPerWG + 16 * qg + l16];
    inv_l[qg] = lr > 0.f ? 1.f / lr : 0.f;
  }
  if (kh == 0 && g == 0 && own_row < nrows) {
    if constexpr (!kDecode) {
      if (p.m != nullptr) {
        const int pos = fast_div(own_row, p.hdiv), head = own_row - pos * p.H;
        const int si = (b * p.H + head) * p.Sq + pos;
        p.m[si] = mt == kNegInf ? kNegInf : mt * kLn2;
        p.l[si] = mt == kNegInf ? 0.f : ltot * fast_exp2(mref - mt);
      }
    } else {
      const float lse = poison ? nanv : (ltot > 0.f ? (mref + __log2f(ltot)) * kLn2 : kNegInf);
      if (wk.nsplit == 1) {
        if (p.lse != nullptr) p.lse[b * p.H + own_row] = lse;
      } else {
        p.part_lse[(int64_t)wk.slot * p.H + own_row] = lse;
      }
    }
  }
  const int col = 64 * wave + 4 * g;
  if constexpr (!kDecode) {
    // O goes out as whole 1 KB rows: each wave writes its 64 x 64 block (scaled, bf16) into
    // the free ring slots as [row][512] with the 16-byte chunks of row r xor-swizzled by r % 16
    // (two-way bank conflicts at most), then stores 8 rows with 16 contiguous bytes per lane.
    // (Decode keeps direct stores: measured faster there.)
    DMLA_LDS char* ost = lds;
#pragma unroll
    for (int qg = 0; qg < 4; ++qg) {
      const int rl = 16 * qg + l16;
      const float inv = inv_l[qg];
#pragma unroll
      for (int d = 0; d < kDbWave; ++d) {
        const f32x4 v = oacc[d][qg] * inv;
        bf16x4 w;
        w[0] = (bf16)v[0]; w[1] = (bf16)v[1]; w[2] = (bf16)v[2]; w[3] = (bf16)v[3];
        const int chunk = (8 * wave + 2 * d + (g >> 1)) ^ (rl & 15);
        *reinterpret_cast<DMLA_LDS bf16x4*>(ost + rl * 1024 + chunk * 16 + (g & 1) * 8) = w;
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int rl = 8 * wave + k;
      const int r = row0 + rl;
      if (r >= nrows) break;
      const bf16x8 v = *reinterpret_cast<const DMLA_LDS bf16x8*>(ost + rl * 1024 + (lane ^ (rl & 15)) * 16);
      const int pos = fast_div(r, p.hdiv), head = r - pos * p.H;
      // non-temporal: O is not read again by this kernel, and lines streamed out during the grid
      // leave less dirty L2 for the end-of-kernel write-back (measured 313 -> 308 us at cfg 2)
      __builtin_nontemporal_store(v, reinterpret_cast<bf16x8*>(p.o + b * p.o_sb + head * p.o_sh + pos * p.o_ss + 8 * lane));
    }
    return;
  }
#pragma unroll
  for (int qg = 0; qg < 4; ++qg) {
    const int r = row0 + 16 * qg + l16;
    if (r >= nrows) continue;
    const float inv = inv_l[qg];
    if (wk.nsplit == 1) {
      bf16* orp = p.o + b * p.o_sb + r * p.o_sh + col;
#pragma unroll
      for (int d = 0; d < kDbWave; ++d) {
        f32x4 v = oacc[d][qg] * inv;
        if (poison) v = f32x4{nanv, nanv, nanv, nanv};
        bf16x4 w;
        w[0] = (bf16)v[0]; w[1] = (bf16)v[1]; w[2] = (bf16)v[2]; w[3] = (bf16)v[3];
        *reinterpret_cast<bf16x4*>(orp + 16 * d) = w;
      }
    } else {
      // bf16 partials: the end-of-segment stores of all workgroups come in one burst that the
      // HBM write bandwidth paces; the combine rescales and sums them in fp32.
      bf16* pp = p.part_o + ((int64_t)wk.slot * p.H + r) * kDv + col;
#pragma unroll
      for (int d = 0; d < kDbWave; ++d) {
        f32x4 v = oacc[d][qg] * inv;
        if (poison) v = f32x4{nanv, nanv, nanv, nanv};
        bf16x4 w;
        w[0] = (bf16)v[0]; w[1] = (bf16)v[1]; w[2] = (bf16)v[2]; w[3] = (bf16)v[3];
        *reinterpret_cast<bf16x4*>(pp + 16 * d) = w;
      }
    }
  }
}

// Out-of-line so the fast path carries none of its registers.  `params` is the kernel's
// argument segment (MqaParams is the kernel's only argument), taken in the kernel itself: the
// segment pointer is only defined inside kernels, and passing the parameters by reference
// would copy them to scratch memory in every workgroup.
template <bool kDecode, int kHalf>
__device__ __noinline__ void mqa_fwd_exact(const MqaParams* params, Work wk, DMLA_LDS char* lds, int wave, int lane) {
  // Call arguments arrive in VGPRs; the staging code needs the wave-uniform values in SGPRs.
  const uint64_t pa = reinterpret_cast<uint64_t>(params);
  const MqaParams& p = *reinterpret_cast<const MqaParams*>(
      ((uint64_t)__builtin_amdgcn_readfirstlane((unsigned)(pa >> 32)) << 32) |
      (unsigned)__builtin_amdgcn_readfirstlane((unsigned)pa));
  wave = uniform(wave);
  wk.b = uniform(wk.b); wk.row0 = uniform(wk.row0); wk.tile_begin = uniform(wk.tile_begin);
  wk.tile_end = uniform(wk.tile_end); wk.split = uniform(wk.split); wk.nsplit = uniform(wk.nsplit);
  wk.ctx = uniform(wk.ctx); wk.page_begin = uniform(wk.page_begin); wk.slot = uniform(wk.slot);
  lds = reinterpret_cast<DMLA_LDS char*>(static_cast<uintptr_t>(uniform((int)lds_addr(lds))));
  __syncthreads();
  mqa_fwd_body<kDecode, kHalf, true>(p, &p, wk, lds, wave, lane);
}

// Exclusive prefix of one value per thread over the workgroup; `total` gets the sum.
__device__ __forceinline__ int wg_exclusive_scan(int v, DMLA_LDS int* tmp, int& total) {
  const int lane = lane_id(), wave = uniform(threadIdx.x >> 6);
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) tmp[wave] = x;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int v2 = tmp[w];
    before += w < wave ? v2 : 0;
    tot += v2;
  }
  __syncthreads();   // tmp is free again
  total = tot;
  return before + x - v;
}

// The decode plan built by a workgroup in LDS: the arithmetic of decode_plan_kernel with one
// sequence and one range per thread.  Workgroup 0 also stores it in the plan layout, where
// the combine reads the split counts and bases.
__device__ __forceinline__ void build_inline_plan(const MqaParams& p, DMLA_LDS InlinePlan* ip) {
  const int tid = threadIdx.x;
  const int B = p.B, R = p.n_ranges;
  int nt = 0;
  int ctx = 0;
  if (tid < B) {
    ctx = min(max(p.seqlens[tid], 0), p.max_pages * kPage);
    nt = (ctx + kTileN - 1) / kTileN;
  }
  int total, nonempty;
  const int tpb = wg_exclusive_scan(nt, ip->tmp, total);
  const int nb = wg_exclusive_scan(nt > 0 ? 1 : 0, ip->tmp, nonempty);
  const int64_t weighted = (int64_t)total + (int64_t)kSegCost * nonempty;
  const int W = (int)max<int64_t>(1, (weighted + R - 1) / R);
  // Each nonempty sequence owns the weighted positions [ws, ws + kSegCost + nt): its kSegCost
  // virtual tiles, then its tiles.  The ranges starting there (r W in that span) start at its
  // first tile or at the tile under r W -- the value the plan kernel's search over sequences
  // finds -- and a tile t of it lies in range floor((t + kSegCost (nb + 1)) / W), the last range
  // starting at or before t.  So every thread places its sequence's ranges and splits itself,
  // with no searches.
  int ns = 0, fr = 0;
  if (tid < B) {
    ip->tp[tid] = tpb;
    if (nt > 0) {
      const int64_t ws = (int64_t)tpb + (int64_t)kSegCost * nb;
      const int64_t we = ws + kSegCost + nt;
      const int r0 = (int)((ws + W - 1) / W), r1 = (int)min<int64_t>((we + W - 1) / W, R);
      for (int r = r0; r < r1; ++r) {
        ip->rs[r] = tpb + (int)max<int64_t>(0, (int64_t)r * W - ws - kSegCost);
        ip->rfb[r] = tid;
      }
      const int64_t w1 = (int64_t)kSegCost * (nb + 1);
      fr = (int)(((int64_t)tpb + w1) / W);
      ns = (int)(((int64_t)tpb + nt - 1 + w1) / W) - fr + 1;
    }
  }
  if (tid == 0) ip->tp[B] = total;
  // Ranges past the weighted total are empty.
  for (int rr = (int)((weighted + W - 1) / W) + tid; rr <= R; rr += kThreads) {
    ip->rs[rr] = total;
    if (rr < R) ip->rfb[rr] = B - 1;
  }
  int nsplits;
  const int sbb = wg_exclusive_scan(ns, ip->tmp, nsplits);
  if (tid < B) {
    ip->ns[tid] = ns;
    ip->ctx[tid] = ctx;
    ip->fr[tid] = fr;
    ip->sb[tid] = sbb;
  }
  if (tid == 0) ip->sb[B] = nsplits;
  __syncthreads();
  if (blockIdx.x == 0 && p.plan_out != nullptr) {
    int32_t* plan = p.plan_out;
    int32_t* tile_prefix = plan + kPlanHeader;
    int32_t* split_base = tile_prefix + B + 1;
    int32_t* num_splits = split_base + B + 1;
    int32_t* first_range = num_splits + B;
    int32_t* range_start = first_range + B;
    int32_t* range_first_b = range_start + R + 1;
    for (int i = tid; i <= B; i += kThreads) {
      tile_prefix[i] = ip->tp[i];
      split_base[i] = ip->sb[i];
    }
    for (int i = tid; i < B; i += kThreads) {
      num_splits[i] = ip->ns[i];
      first_range[i] = ip->fr[i];
    }
    for (int i = tid; i <= R; i += kThreads) range_start[i] = ip->rs[i];
    for (int i = tid; i < R; i += kThreads) range_first_b[i] = ip->rfb[i];
    if (tid == 0) {
      plan[0] = B; plan[1] = R; plan[2] = W; plan[3] = total; plan[4] = nsplits; plan[5] = kSegCost;
      plan[6] = plan[7] = 0;
    }
  }
}

template <bool kDecode>
__global__ __launch_bounds__(kThreads, 1) void mqa_fwd_kernel(MqaParams p) {
  __shared__ __attribute__((aligned(1024))) char smem[kDecode ? kDecodeLdsBytes : kLdsBytes];
  DMLA_LDS char* lds = (DMLA_LDS char*)smem;
  const int lane = lane_id();
  const int wave = uniform(threadIdx.x >> 6);

  Work wk = {};
  if constexpr (!kDecode) {
    // Heaviest (latest) row tiles first; consecutive ids alternate batches so each XCD's L2
    // sees few distinct K_lat sequences.
    const int id = blockIdx.x;
    wk.b = id % p.B;
    const int rt = p.n_row_tiles - 1 - id / p.B;
    wk.row0 = rt * kRowsPerWG;
    const int last_row = min(wk.row0 + kRowsPerWG, p.H * p.Sq) - 1;
    const int last_pos = fast_div(last_row, p.hdiv);
    int kend = p.causal ? min(p.Sk, last_pos + 1 + (p.Sk - p.Sq)) : p.Sk;
    kend = max(kend, 0);
    wk.tile_begin = 0;
    wk.tile_end = (kend + kTileN - 1) / kTileN;
    wk.nsplit = 1;
    const MqaParams* params = (const MqaParams*)(__builtin_amdgcn_kernarg_segment_ptr());
    if (((wave >> 1) & 1) == 0) mqa_fwd_body<kDecode, 0, false>(p, params, wk, lds, wave, lane);
    else mqa_fwd_body<kDecode, 1, false>(p, params, wk, lds, wave, lane);
  } else {
    // Workgroup -> (range r, head group k) with the head groups of a range 8 ids apart, so
    // they run on the same XCD and the second read of the range's pages hits that XCD's L2.
    const int id = blockIdx.x;
    const int k = (id / 8) % p.head_groups;
    const int r = (id / (8 * p.head_groups)) * 8 + id % 8;
    const bool inl = p.plan_inline != 0;
    DMLA_LDS InlinePlan* ip = reinterpret_cast<DMLA_LDS InlinePlan*>(lds + kLdsBytes);
    if (inl) build_inline_plan(p, ip);   // every workgroup, before any early exit
    if (r >= p.n_ranges) return;
    const int32_t* plan = p.plan;
    const int32_t* tile_prefix = plan + kPlanHeader;
    const int32_t* split_base = tile_prefix + p.B + 1;
    const int32_t* num_splits = split_base + p.B + 1;
    const int32_t* first_range = num_splits + p.B;
    const int32_t* range_start = first_range + p.B;
    const int32_t* range_first_b = range_start + p.n_ranges + 1;
    auto tp_of = [&](int i) { return inl ? ip->tp[i] : tile_prefix[i]; };
    const int t0 = inl ? ip->rs[r] : range_start[r];
    const int t1 = inl ? ip->rs[r + 1] : range_start[r + 1];
    if (t0 >= t1) return;
    const int first_b = inl ? ip->rfb[r] : range_first_b[r];
    const MqaParams* params = (const MqaParams*)(__builtin_amdgcn_kernarg_segment_ptr());
    for (int bseq = first_b; bseq < p.B; ++bseq) {
      const int tb = tp_of(bseq);
      if (tb >= t1) break;
      const int seg0 = max(t0, tb), seg1 = min(t1, tp_of(bseq + 1));
      if (seg0 >= seg1) continue;   // an empty sequence (its output comes from the combine)
      wk.b = bseq;
      wk.row0 = k * kRowsPerWG;
      // From the inline plan when there is one: a global load here would also wait for the
      // previous segment's output stores (loads and stores share one counter).
      wk.ctx = inl ? ip->ctx[bseq] : min(max(p.seqlens[bseq], 0), p.max_pages * kPage);
      wk.tile_begin = seg0 - tb;
      wk.tile_end = seg1 - tb;
      wk.page_begin = wk.tile_begin / (kPage / kTileN);
      wk.nsplit = inl ? ip->ns[bseq] : num_splits[bseq];
      wk.split = r - (inl ? ip->fr[bseq] : first_range[bseq]);
      wk.slot = (inl ? ip->sb[bseq] : split_base[bseq]) + wk.split;
      if (((wave >> 1) & 1) == 0) mqa_fwd_body<kDecode, 0, false>(p, params, wk, lds, wave, lane);
      else mqa_fwd_body<kDecode, 1, false>(p, params, wk, lds, wave, lane);
      __syncthreads();   // every LDS read of this segment is done before the next one's copies
    }
  }
}

// One workgroup computes the decode plan (layout above) from the context lengths.  The arrays
// the binary searches read are mirrored in LDS when they fit (the common case), so every
// dependent step is an LDS access rather than a global memory round trip.
constexpr int kPlanLds = 4096;
constexpr int kPlanThreads = 256;   // four waves: the scans and barriers stay short
constexpr int kPlanWaves = kPlanThreads / 64;
__global__ __launch_bounds__(kPlanThreads) void decode_plan_kernel(const int32_t* seqlens, int B, int R, int max_pages,
                                                           int32_t* plan) {
  __shared__ int scan[kPlanThreads];
  __shared__ int l_tp[kPlanLds], l_ne[kPlanLds], l_rs[kPlanLds];
  int32_t* tile_prefix = plan + kPlanHeader;
  int32_t* split_base = tile_prefix + B + 1;
  int32_t* num_splits = split_base + B + 1;
  int32_t* first_range = num_splits + B;
  int32_t* range_start = first_range + B;
  int32_t* range_first_b = range_start + R + 1;
  const bool lds_b = B + 1 <= kPlanLds, lds_r = R + 1 <= kPlanLds;
  // nonempty_before[b] lives in num_splits until the split counts replace it
  const int* tp = lds_b ? l_tp : tile_prefix;
  const int* ne = lds_b ? l_ne : num_splits;
  const int* rs = lds_r ? l_rs : range_start;
  const int tid = threadIdx.x;
  // Prefix over kPlanThreads-element chunks: a shuffle scan within each wave, the wave totals
  // scanned by wave 0 through LDS, three barriers per chunk.  Returns the inclusive scan;
  // scan[kPlanThreads - 1] is the chunk total afterwards.
  auto chunk_scan = [&](int v) -> int {
    const int ln = tid & 63, wv = tid >> 6;
#pragma unroll
    for (int off = 1; off < 64; off *= 2) {
      const int up = __shfl_up(v, off, 64);
      if (ln >= off) v += up;
    }
    if (ln == 63) scan[wv] = v;
    __syncthreads();
    if (wv == 0) {
      int t = ln < kPlanWaves ? scan[ln] : 0;
#pragma unroll
      for (int off = 1; off < kPlanWaves; off *= 2) {
        const int up = __shfl_up(t, off, 64);
        if (ln >= off) t += up;
      }
      if (ln < kPlanWaves) scan[32 + ln] = t;   // inclusive wave-total prefix
    }
    __syncthreads();
    const int incl = v + (wv > 0 ? scan[32 + wv - 1] : 0);
    if (tid == kPlanThreads - 1) scan[kPlanThreads - 1] = incl;
    __syncthreads();
    return incl;
  };
  int carry = 0, ncarry = 0;
  for (int base = 0; base < B; base += kPlanThreads) {
    const int b = base + tid;
    int nt = 0;
    if (b < B) nt = (min(max(seqlens[b], 0), max_pages * kPage) + kTileN - 1) / kTileN;
    const int incl = chunk_scan(nt);
    const int tpb = carry + incl - nt;
    carry += scan[kPlanThreads - 1];
    __syncthreads();
    const int nz = nt > 0 ? 1 : 0;
    const int incl2 = chunk_scan(nz);
    const int neb = ncarry + incl2 - nz;
    ncarry += scan[kPlanThreads - 1];
    if (b < B) {
      tile_prefix[b] = tpb; num_splits[b] = neb;
      if (lds_b) { l_tp[b] = tpb; l_ne[b] = neb; }
    }
    __syncthreads();
  }
  const int total = carry;
  if (tid == 0) { tile_prefix[B] = total; if (lds_b) l_tp[B] = total; }
  const int64_t weighted = (int64_t)total + (int64_t)kSegCost * ncarry;
  const int W = (int)max<int64_t>(1, (weighted + R - 1) / R);
  __threadfence_block();
  __syncthreads();
  // Range starts: weighted position r W -> the sequence holding it (last b whose weighted start
  // is <= it) -> its tile, or the sequence's first tile when among its virtual tiles.
  for (int r = tid; r <= R; r += kPlanThreads) {
    int t = total;
    if (r < R && (int64_t)r * W < weighted) {
      const int64_t pos = (int64_t)r * W;
      int lo = 0, hi = B - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if ((int64_t)tp[mid] + (int64_t)kSegCost * ne[mid] <= pos) lo = mid; else hi = mid - 1;
      }
      const int64_t off = pos - ((int64_t)tp[lo] + (int64_t)kSegCost * ne[lo]);
      t = tp[lo] + (int)max<int64_t>(0, off - kSegCost);
      t = min(t, tp[lo + 1]);
    }
    range_start[r] = t;
    if (lds_r) l_rs[r] = t;
  }
  __threadfence_block();
  __syncthreads();
  // first_range[b] / last range: the last range starting at or before the sequence's first /
  // last tile; num_splits and split_base follow.
  auto range_of = [&](int t) {
    int lo = 0, hi = R - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) / 2;
      if (rs[mid] <= t) lo = mid; else hi = mid - 1;
    }
    return lo;
  };
  int scarry = 0;
  for (int base = 0; base < B; base += kPlanThreads) {
    const int b = base + tid;
    int ns = 0, fr = 0;
    if (b < B) {
      const int tb = tp[b], te = tp[b + 1];
      if (te > tb) {
        fr = range_of(tb);
        ns = range_of(te - 1) - fr + 1;
      }
    }
    __syncthreads();   // every thread is past its reads of the nonempty counts
    if (b < B) { num_splits[b] = ns; first_range[b] = fr; }
    const int incl = chunk_scan(ns);
    if (b < B) split_base[b] = scarry + incl - ns;
    scarry += scan[kPlanThreads - 1];
    __syncthreads();
  }
  if (tid == 0) {
    split_base[B] = scarry;
    plan[0] = B; plan[1] = R; plan[2] = W; plan[3] = total; plan[4] = scarry; plan[5] = kSegCost;
    plan[6] = plan[7] = 0;
  }
  // range_first_b[r]: the sequence holding tile range_start[r] (last b with tile_prefix[b] <= it)
  for (int r = tid; r < R; r += kPlanThreads) {
    const int t = rs[r];
    int lo = 0, hi = B - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) / 2;
      if (tp[mid] <= t) lo = mid; else hi = mid - 1;
    }
    range_first_b[r] = lo;
  }
}

// Ranges of a decode plan: one workgroup per range and head group fills the CUs; more ranges
// when the widest batch would overflow a segment's page cache.  A segment spans at most W
// tiles, W = ceil(weighted / R), and the weighted total is at most B max_pages 2 + kSegCost B
// (every sequence full and nonempty), so R >= that bound / kMaxSegTiles keeps W <= kMaxSegTiles
// and every segment within kMaxSegPages pages (a segment may start on the second tile of a page).
int64_t decode_ranges(int64_t B, int64_t H, int64_t max_pages) {
  const int64_t hg = (H + kRowsPerWG - 1) / kRowsPerWG;
  int64_t r = device_cu_count() / hg;
  if (r >= 8) r -= r % 8;
  const int64_t weighted_max = B * max_pages * (kPage / kTileN) + (int64_t)kSegCost * B;
  const int64_t cap = (weighted_max + kMaxSegTiles - 1) / kMaxSegTiles;
  return std::max<int64_t>(std::max<int64_t>(r, cap), 1);
}

}  // namespace
}  // namespace dmla

using namespace dmla;

extern "C" int dmla_fwd_cache_latent(const void* q, const void* k_lat, void* o, float* m, float* l,
                                     int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t d_qk,
                                     int64_t d_v, int64_t q_sb, int64_t q_sh, int64_t q_ss,
                                     int64_t k_sb, int64_t k_ss, int64_t o_sb, int64_t o_sh,
                                     int64_t o_ss, float softmax_scale, int causal,
                                     dmla_stream_t stream) {
  clear_error();
  if (!q || !k_lat || !o) return fail(DMLA_ERR_INVALID_ARG, "dmla_fwd_cache_latent: null q/k_lat/o");
  if ((m == nullptr) != (l == nullptr))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_fwd_cache_latent: m and l must both be set or both be NULL");
  if (B < 0 || H < 0 || Sq < 0 || Sk < 0)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_fwd_cache_latent: negative size");
  if (d_qk != kDqk || d_v != kDv)
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_fwd_cache_latent: only d_qk=576, d_v=512 is compiled (got %lld, %lld)",
                (long long)d_qk, (long long)d_v);
  if (!(softmax_scale > 0.f) || !__builtin_isfinite(softmax_scale))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_fwd_cache_latent: softmax_scale must be finite and > 0");
  if (!aligned16(q) || !aligned16(k_lat) || !aligned16(o))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_fwd_cache_latent: q/k_lat/o must be 16-byte aligned");
  if (!mult8(q_sb) || !mult8(q_sh) || !mult8(q_ss) || !mult8(k_sb) || !mult8(k_ss) || !mult8(o_sb) ||
      !mult8(o_sh) || !mult8(o_ss))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_fwd_cache_latent: strides must be multiples of 8 elements");
  if (k_ss < kDqk || k_ss * 2 * kTileN >= ((int64_t)1 << 31))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_fwd_cache_latent: k_lat row stride out of range");
  const int64_t rows = H * Sq;
  if (rows > ((int64_t)1 << 30) || Sk > ((int64_t)1 << 30))
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_fwd_cache_latent: size too large");
  if (B == 0 || rows == 0) return DMLA_OK;

  MqaParams p = {};
  p.q = static_cast<const bf16*>(q);
  p.kv = static_cast<const bf16*>(k_lat);
  p.o = static_cast<bf16*>(o);
  p.m = m;
  p.l = l;
  p.q_sb = q_sb; p.q_sh = q_sh; p.q_ss = q_ss;
  p.k_sb = k_sb; p.k_ss = k_ss;
  p.o_sb = o_sb; p.o_sh = o_sh; p.o_ss = o_ss;
  p.B = (int)B; p.H = (int)H; p.Sq = (int)Sq; p.Sk = (int)Sk;
  p.hdiv = make_fastdiv((unsigned)H);
  p.scale_log2 = softmax_scale * kLog2e;
  p.causal = causal ? 1 : 0;
  p.n_row_tiles = (int)((rows + kRowsPerWG - 1) / kRowsPerWG);
  const int64_t grid = (int64_t)p.n_row_tiles * B;
  if (grid > 0x7fffffff) return fail(DMLA_ERR_UNSUPPORTED, "dmla_fwd_cache_latent: grid too large");
  hipLaunchKernelGGL(mqa_fwd_kernel<false>, dim3((unsigned)grid), dim3(kThreads), 0,
                     (hipStream_t)stream, p);
  return check_launch("dmla_fwd_cache_latent");
}

// Bytes of a decode plan for this batch on the current device (a multiple of 256).
extern "C" int64_t dmla_decode_plan_bytes(int64_t B, int64_t H, int64_t max_pages_per_seq) {
  if (B <= 0 || H <= 0 || max_pages_per_seq <= 0) return 0;
  const int64_t R = decode_ranges(B, H, max_pages_per_seq);
  return (plan_ints(B, R) * 4 + 255) / 256 * 256;
}

static int64_t decode_slots(int64_t B, int64_t H, int64_t max_pages_per_seq) {
  return decode_ranges(B, H, max_pages_per_seq) + B;   // sum over sequences of their splits
}

extern "C" int64_t dmla_decode_workspace_bytes(int64_t B, int64_t H, int64_t d_v, int64_t max_pages_per_seq) {
  if (B <= 0 || H <= 0 || d_v != kDv || max_pages_per_seq <= 0) return 0;
  return dmla_decode_plan_bytes(B, H, max_pages_per_seq) +
         decode_slots(B, H, max_pages_per_seq) * H * (int64_t)(kDv * 2 + 4);
}

extern "C" int dmla_decode_plan(const int32_t* cache_seqlens, int64_t B, int64_t H, int64_t max_pages_per_seq,
                                int32_t* plan, int64_t plan_bytes, dmla_stream_t stream) {
  clear_error();
  if (!cache_seqlens || !plan) return fail(DMLA_ERR_INVALID_ARG, "dmla_decode_plan: null pointer argument");
  if (B <= 0 || H <= 0 || max_pages_per_seq <= 0)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_decode_plan: sizes must be positive");
  if (H > ((int64_t)1 << 16) || B > ((int64_t)1 << 20) || max_pages_per_seq > ((int64_t)1 << 24) ||
      B * max_pages_per_seq * (kPage / kTileN) > 0x7fffffff)
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_decode_plan: size too large");
  const int64_t need = dmla_decode_plan_bytes(B, H, max_pages_per_seq);
  if (plan_bytes < need)
    return fail(DMLA_ERR_WORKSPACE, "dmla_decode_plan: %lld bytes needed (got %lld)", (long long)need,
                (long long)plan_bytes);
  const int64_t R = decode_ranges(B, H, max_pages_per_seq);
  hipLaunchKernelGGL(decode_plan_kernel, dim3(1), dim3(kPlanThreads), 0, (hipStream_t)stream, cache_seqlens, (int)B, (int)R,
                     (int)max_pages_per_seq, plan);
  return check_launch("dmla_decode_plan");
}

// Argument checks shared by the decode entry points (before any workspace check).
static int decode_validate(const void* q, const void* kv_pool, const int32_t* block_table,
                           const int32_t* cache_seqlens, const void* o, int64_t B, int64_t H, int64_t d_qk,
                           int64_t d_v, int64_t page_size, int64_t num_pages, int64_t max_pages_per_seq,
                           int64_t q_sb, int64_t q_sh, int64_t kv_sp, int64_t kv_ss, int64_t bt_sb, int64_t o_sb,
                           int64_t o_sh, float softmax_scale) {
  if (!q || !kv_pool || !block_table || !cache_seqlens || !o)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_decode_paged: null pointer argument");
  if (B < 0 || H < 0 || num_pages < 0 || max_pages_per_seq < 0)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_decode_paged: negative size");
  if (d_qk != kDqk || d_v != kDv || page_size != kPage)
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_decode_paged: only d_qk=576, d_v=512, page_size=64 is compiled (got %lld, %lld, %lld)",
                (long long)d_qk, (long long)d_v, (long long)page_size);
  if (!(softmax_scale > 0.f) || !__builtin_isfinite(softmax_scale))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_decode_paged: softmax_scale must be finite and > 0");
  if (!aligned16(q) || !aligned16(kv_pool) || !aligned16(o))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_decode_paged: q/kv_pool/o must be 16-byte aligned");
  if (!mult8(q_sb) || !mult8(q_sh) || !mult8(kv_sp) || !mult8(kv_ss) || !mult8(o_sb) || !mult8(o_sh))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_decode_paged: strides must be multiples of 8 elements");
  if (kv_ss < kDqk || kv_sp < kv_ss * kPage || kv_ss * 2 * kPage >= ((int64_t)1 << 31))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_decode_paged: kv_pool strides out of range");
  if (bt_sb < max_pages_per_seq)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_decode_paged: block_table row stride %lld < max_pages_per_seq %lld",
                (long long)bt_sb, (long long)max_pages_per_seq);
  if (H > ((int64_t)1 << 16) || B > ((int64_t)1 << 20) || max_pages_per_seq > ((int64_t)1 << 24) ||
      num_pages > 0x7fffffff || B * max_pages_per_seq * (kPage / kTileN) > 0x7fffffff)
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_decode_paged: size too large");
  if (B == 0 || H == 0) return DMLA_OK;
  if (num_pages == 0 || max_pages_per_seq == 0)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_decode_paged: empty page pool or block table");
  return DMLA_OK;
}

namespace dmla {
namespace {

// Launches the decode kernel and the combine on partial buffers of `part_bytes` bytes.  With
// plan_out set, the decode kernel builds the plan itself and stores it there for the combine;
// otherwise it reads `plan`.
int decode_launch(const void* q, const void* kv_pool, const int32_t* block_table, const int32_t* cache_seqlens,
                  void* o, float* lse, int64_t B, int64_t H, int64_t num_pages, int64_t max_pages_per_seq,
                  int64_t q_sb, int64_t q_sh, int64_t kv_sp, int64_t kv_ss, int64_t bt_sb, int64_t o_sb,
                  int64_t o_sh, float softmax_scale, const int32_t* plan, int32_t* plan_out, void* workspace,
                  int64_t workspace_bytes, hipStream_t stream) {
  const int64_t slots = decode_slots(B, H, max_pages_per_seq);
  const int64_t need = slots * H * (int64_t)(kDv * 2 + 4);   // bf16 partial rows, then fp32 lse
  if (workspace == nullptr || workspace_bytes < need)
    return fail(DMLA_ERR_WORKSPACE, "dmla_decode_paged: workspace of %lld bytes needed (got %lld)",
                (long long)need, (long long)workspace_bytes);
  if (!aligned16(workspace)) return fail(DMLA_ERR_INVALID_ARG, "dmla_decode_paged: workspace must be 16-byte aligned");

  MqaParams p = {};
  p.q = static_cast<const bf16*>(q);
  p.kv = static_cast<const bf16*>(kv_pool);
  p.o = static_cast<bf16*>(o);
  p.lse = lse;
  p.q_sb = q_sb; p.q_sh = q_sh;
  p.k_sb = kv_sp; p.k_ss = kv_ss;
  p.o_sb = o_sb; p.o_sh = o_sh;
  p.B = (int)B; p.H = (int)H; p.Sq = 1; p.Sk = 0;
  p.hdiv = make_fastdiv((unsigned)H);
  p.scale_log2 = softmax_scale * kLog2e;
  p.block_table = block_table;
  p.seqlens = cache_seqlens;
  p.bt_sb = bt_sb;
  p.num_pages = (int)num_pages;
  p.max_pages = (int)max_pages_per_seq;
  p.head_groups = (int)((H + kRowsPerWG - 1) / kRowsPerWG);
  p.n_ranges = (int)decode_ranges(B, H, max_pages_per_seq);
  p.plan = plan_out != nullptr ? nullptr : plan;
  p.plan_inline = plan_out != nullptr ? 1 : 0;
  p.plan_out = plan_out;
  p.part_o = static_cast<bf16*>(workspace);
  p.part_lse = reinterpret_cast<float*>(p.part_o + slots * H * kDv);
  const int64_t grid = ((int64_t)(p.n_ranges + 7) / 8) * 8 * p.head_groups;
  if (grid > 0x7fffffff) return fail(DMLA_ERR_UNSUPPORTED, "dmla_decode_paged: grid too large");
  hipLaunchKernelGGL(mqa_fwd_kernel<true>, dim3((unsigned)grid), dim3(kThreads), 0, stream, p);
  int rc = check_launch("dmla_decode_paged");
  if (rc != DMLA_OK) return rc;
  // Sequences with one split were written by the decode kernel; the others (and the empty
  // ones: zeros, lse -inf) come from the combine.
  const int32_t* tile_prefix = (plan_out != nullptr ? plan_out : plan) + kPlanHeader;
  CombineArgs c = {};
  c.part_o16 = p.part_o;
  c.part_lse = p.part_lse;
  c.split_base = tile_prefix + B + 1;
  c.num_splits = tile_prefix + 2 * (B + 1);
  c.o = p.o;
  c.lse = lse;
  c.B = (int)B; c.H = (int)H; c.max_splits = p.n_ranges + 1; c.d = kDv;
  c.skip_single = 1;
  c.po_ss = H * kDv; c.po_sh = kDv;
  c.lse_ss = H; c.lse_sh = 1;
  c.o_sb = o_sb; c.o_sh = o_sh;
  return launch_lse_combine(c, stream, "dmla_decode_paged(combine)");
}


}  // namespace
}  // namespace dmla

extern "C" int dmla_decode_paged_planned(const void* q, const void* kv_pool, const int32_t* block_table,
                                         const int32_t* cache_seqlens, void* o, float* lse, int64_t B,
                                         int64_t H, int64_t d_qk, int64_t d_v, int64_t page_size,
                                         int64_t num_pages, int64_t max_pages_per_seq, int64_t q_sb,
                                         int64_t q_sh, int64_t kv_sp, int64_t kv_ss, int64_t bt_sb,
                                         int64_t o_sb, int64_t o_sh, float softmax_scale, const int32_t* plan,
                                         void* workspace, int64_t workspace_bytes, dmla_stream_t stream) {
  clear_error();
  if (!plan) return fail(DMLA_ERR_INVALID_ARG, "dmla_decode_paged: null plan");
  int rc0 = decode_validate(q, kv_pool, block_table, cache_seqlens, o, B, H, d_qk, d_v, page_size, num_pages,
                            max_pages_per_seq, q_sb, q_sh, kv_sp, kv_ss, bt_sb, o_sb, o_sh, softmax_scale);
  if (rc0 != DMLA_OK || B == 0 || H == 0) return rc0;
  return decode_launch(q, kv_pool, block_table, cache_seqlens, o, lse, B, H, num_pages, max_pages_per_seq, q_sb,
                       q_sh, kv_sp, kv_ss, bt_sb, o_sb, o_sh, softmax_scale, plan, nullptr, workspace,
                       workspace_bytes, (hipStream_t)stream);
}

namespace dmla {
namespace {

// The body of dmla_decode_paged on a workspace the caller vouches for (16-byte aligned, at
// least dmla_decode_workspace_bytes): the plan at its head, the split partials after it.
int decode_paged_on(const void* q, const void* kv_pool, const int32_t* block_table, const int32_t* cache_seqlens,
                    void* o, float* lse, int64_t B, int64_t H, int64_t d_v, int64_t num_pages,
                    int64_t max_pages_per_seq, int64_t q_sb, int64_t q_sh, int64_t kv_sp, int64_t kv_ss,
                    int64_t bt_sb, int64_t o_sb, int64_t o_sh, float softmax_scale, void* workspace,
                    int64_t workspace_bytes, hipStream_t stream) {
  const int64_t pb = dmla_decode_plan_bytes(B, H, max_pages_per_seq);
  int32_t* plan = static_cast<int32_t*>(workspace);
  void* parts = static_cast<char*>(workspace) + pb;
  // Small batches (the serving case): the decode kernel builds the plan itself and stores it in
  // the workspace; otherwise the plan kernel runs first.
  if (B <= kInlinePlanB && decode_ranges(B, H, max_pages_per_seq) <= kInlinePlanR)
    return decode_launch(q, kv_pool, block_table, cache_seqlens, o, lse, B, H, num_pages, max_pages_per_seq, q_sb,
                         q_sh, kv_sp, kv_ss, bt_sb, o_sb, o_sh, softmax_scale, nullptr, plan, parts,
                         workspace_bytes - pb, stream);
  int rc = dmla_decode_plan(cache_seqlens, B, H, max_pages_per_seq, plan, pb, stream);
  if (rc != DMLA_OK) return rc;
  return decode_launch(q, kv_pool, block_table, cache_seqlens, o, lse, B, H, num_pages, max_pages_per_seq, q_sb,
                       q_sh, kv_sp, kv_ss, bt_sb, o_sb, o_sh, softmax_scale, plan, nullptr, parts,
                       workspace_bytes - pb, stream);
}

// Scratch of dmla_decode_paged_noalloc: a file-scope device array, one copy per GPU, held until
// the process ends.  Host code never uses the array's name as an address (on the host it is a
// stand-in for the symbol); the device address comes from hipGetSymbolAddress, looked up once
// per device with that device current.
static __device__ __align__(256) char scratch[DMLA_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_on_current_device(void** out, const char* what) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(DMLA_ERR_HIP, "%s: hipGetDevice failed: %s", what, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(DMLA_ERR_UNSUPPORTED, "%s: device %d out of range", what, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(DMLA_ERR_HIP, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return DMLA_OK;
}

}  // namespace
}  // namespace dmla

extern "C" int dmla_decode_paged(const void* q, const void* kv_pool, const int32_t* block_table,
                                 const int32_t* cache_seqlens, void* o, float* lse, int64_t B,
                                 int64_t H, int64_t d_qk, int64_t d_v, int64_t page_size,
                                 int64_t num_pages, int64_t max_pages_per_seq, int64_t q_sb,
                                 int64_t q_sh, int64_t kv_sp, int64_t kv_ss, int64_t bt_sb,
                                 int64_t o_sb, int64_t o_sh, float softmax_scale, void* workspace,
                                 int64_t workspace_bytes, dmla_stream_t stream) {
  clear_error();
  int rc0 = decode_validate(q, kv_pool, block_table, cache_seqlens, o, B, H, d_qk, d_v, page_size, num_pages,
                            max_pages_per_seq, q_sb, q_sh, kv_sp, kv_ss, bt_sb, o_sb, o_sh, softmax_scale);
  if (rc0 != DMLA_OK || B == 0 || H == 0) return rc0;
  const int64_t need = dmla_decode_workspace_bytes(B, H, d_v, max_pages_per_seq);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(DMLA_ERR_WORKSPACE, "dmla_decode_paged: workspace of %lld bytes needed (got %lld)",
                (long long)need, (long long)workspace_bytes);
  if (!aligned16(workspace)) return fail(DMLA_ERR_INVALID_ARG, "dmla_decode_paged: workspace must be 16-byte aligned");
  return decode_paged_on(q, kv_pool, block_table, cache_seqlens, o, lse, B, H, d_v, num_pages, max_pages_per_seq,
                         q_sb, q_sh, kv_sp, kv_ss, bt_sb, o_sb, o_sh, softmax_scale, workspace, workspace_bytes,
                         (hipStream_t)stream);
}

extern "C" int dmla_decode_paged_noalloc(const void* q, const void* kv_pool, const int32_t* block_table,
                                         const int32_t* cache_seqlens, void* o, float* lse, int64_t B,
                                         int64_t H, int64_t d_qk, int64_t d_v, int64_t page_size,
                                         int64_t num_pages, int64_t max_pages_per_seq, int64_t q_sb,
                                         int64_t q_sh, int64_t kv_sp, int64_t kv_ss, int64_t bt_sb,
                                         int64_t o_sb, int64_t o_sh, float softmax_scale, dmla_stream_t stream) {
  clear_error();
  int rc0 = decode_validate(q, kv_pool, block_table, cache_seqlens, o, B, H, d_qk, d_v, page_size, num_pages,
                            max_pages_per_seq, q_sb, q_sh, kv_sp, kv_ss, bt_sb, o_sb, o_sh, softmax_scale);
  if (rc0 != DMLA_OK || B == 0 || H == 0) return rc0;
  const int64_t need = dmla_decode_workspace_bytes(B, H, d_v, max_pages_per_seq);
  if (need > DMLA_NOALLOC_SCRATCH_BYTES)
    return fail(DMLA_ERR_WORKSPACE,
                "dmla_decode_paged_noalloc: this batch needs %lld bytes of scratch, more than the %lld of the "
                "static scratch; use dmla_decode_paged with a workspace",
                (long long)need, (long long)DMLA_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  int rc = scratch_on_current_device(&ws, "dmla_decode_paged_noalloc");
  if (rc != DMLA_OK) return rc;
  return decode_paged_on(q, kv_pool, block_table, cache_seqlens, o, lse, B, H, d_v, num_pages, max_pages_per_seq,
                         q_sb, q_sh, kv_sp, kv_ss, bt_sb, o_sb, o_sh, softmax_scale, ws, DMLA_NOALLOC_SCRATCH_BYTES,
                         (hipStream_t)stream);
}
