// The two ends of paged split-KV decoding that are not attention:
//   * the paged latent-cache append (the producer of the [num_pages, 64, 576] pages that
//     dmla_decode_paged reads through the block table);
//   * the split-KV log-sum-exp combine, also usable on its own (e.g. to merge partials that
//     several devices computed over disjoint page ranges of one context).
// Neither has a reference counterpart: the reference has no paged decode (benchmark config 3).
#include <type_traits>

#include "dmla_common.h"
#include "dmla_host.h"

namespace dmla {

// ---- split-KV combine --------------------------------------------------------------------
// One wave per (sequence, head), four per 256-thread block; lane l covers columns 4l + 256i.
//   o = sum_s w_s o_s / sum_s w_s, w_s = exp(lse_s - max_s lse_s), lse = max + log(sum w)
// over the first n_b splits; no finite lse leaves o = 0 and lse = -inf (max of the inputs);
// a NaN lse makes o and lse NaN.  A split with lse = -inf is skipped whatever its o slot holds.
// The weights are summed and applied in split order.  The common decode shape (at most 4
// splits, d <= 512) issues every partial load before the first weight is known, so a wave
// waits for one memory round trip instead of one per phase.
constexpr int kCombineFast = 4;   // splits held in registers by the one-round-trip path

template <typename T>
__device__ __forceinline__ f32x4 load_part4(const T* p) {
  if constexpr (std::is_same<T, float>::value) {
    return *reinterpret_cast<const f32x4*>(p);
  } else {
    const bf16x4 x = *reinterpret_cast<const bf16x4*>(p);
    return f32x4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
  }
}

template <typename T>
__device__ __forceinline__ void combine_pair(const CombineArgs& a, const T* part, int b, int h, int n, int64_t s0,
                                             int lane) {
  const int64_t lbase = (a.split_base != nullptr ? s0 * a.lse_ss : (int64_t)b * a.lse_sb) + (int64_t)h * a.lse_sh;
  const int64_t obase = (a.split_base != nullptr ? s0 * a.po_ss : (int64_t)b * a.po_sb) + (int64_t)h * a.po_sh;
  bf16* orow = a.o + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh;
  // lse of split s < 64 sits in lane s; later splits are read again from memory
  const float lv_lane = lane < n ? a.part_lse[lbase + (int64_t)lane * a.lse_ss] : kNegInf;
  auto lse_of = [&](int s) -> float {
    if (s < 64) return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lv_lane), s));
    return a.part_lse[lbase + (int64_t)s * a.lse_ss];
  };
  const bool fast = n >= 1 && n <= kCombineFast && a.d <= 512;
  f32x4 pre[kCombineFast][2];
  if (fast) {
    // Unconditional loads (split 0 and column 0 stand in for the ones that do not exist), so
    // that all of them are in flight together; the extra values are never used.
#pragma unroll
    for (int s = 0; s < kCombineFast; ++s)
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int col = 4 * lane + 256 * i;
        pre[s][i] = load_part4(part + obase + (int64_t)(s < n ? s : 0) * a.po_ss + (col < a.d ? col : 0));
      }
  }
  float mx = kNegInf;
  bool bad = false;   // a NaN lse (e.g. a split that met an invalid page) poisons the sequence
  for (int s = 0; s < n; ++s) {
    const float lv = lse_of(s);
    bad = bad || lv != lv;
    mx = fmaxf(mx, lv);
  }
  if (bad) {
    const bf16 nb = (bf16)__builtin_nanf("");
    for (int col = 4 * lane; col < a.d; col += 256) *reinterpret_cast<bf16x4*>(orow + col) = bf16x4{nb, nb, nb, nb};
    if (lane == 0 && a.lse != nullptr) a.lse[(int64_t)b * a.H + h] = __builtin_nanf("");
    return;
  }
  const float mref = mx == kNegInf ? 0.f : mx;
  float wsum = 0.f;
  for (int s = 0; s < n; ++s) wsum += __expf(lse_of(s) - mref);
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  auto store = [&](int col, f32x4 acc) {
    acc *= inv;
    bf16x4 w4;
    w4[0] = (bf16)acc[0]; w4[1] = (bf16)acc[1]; w4[2] = (bf16)acc[2]; w4[3] = (bf16)acc[3];
    *reinterpret_cast<bf16x4*>(orow + col) = w4;
  };
  if (fast) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int col = 4 * lane + 256 * i;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < kCombineFast; ++s) {
        const float lv = lse_of(s);
        if (s < n && lv != kNegInf) acc += __expf(lv - mref) * pre[s][i];
      }
      if (col < a.d) store(col, acc);
    }
  } else {
    for (int col = 4 * lane; col < a.d; col += 256) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int s = 0; s < n; ++s) {
        const float lv = lse_of(s);
        if (lv == kNegInf) continue;
        acc += __expf(lv - mref) * load_part4(part + obase + (int64_t)s * a.po_ss + col);
      }
      store(col, acc);
    }
  }
  if (lane == 0 && a.lse != nullptr) a.lse[(int64_t)b * a.H + h] = wsum > 0.f ? mref + __logf(wsum) : mx;
}

// kPlan: the decode case, split_base and num_splits both given, so that both loads go out
// together (one round trip before the partials' loads, not one per null check).
template <bool kPlan>
__global__ void __launch_bounds__(256) lse_combine_kernel(CombineArgs a) {
  const int lane = threadIdx.x & 63;
  // 32-bit index math: the launcher checks B * H < 2^31
  const unsigned pair = blockIdx.x * 4u + (unsigned)uniform(threadIdx.x >> 6);
  if (pair >= (unsigned)(a.B * a.H)) return;
  const int b = (int)(pair / (unsigned)a.H), h = (int)(pair - (unsigned)b * (unsigned)a.H);
  int n = a.max_splits;
  int64_t s0 = 0;
  if constexpr (kPlan) {
    int sb = a.split_base[b], ns = a.num_splits[b];
    asm volatile("" : "+s"(sb), "+s"(ns));   // both loads issued before anything waits on either
    s0 = sb;
    n = min(max(ns, 0), a.max_splits);
  } else {
    if (a.split_base != nullptr) s0 = a.split_base[b];
    if (a.num_splits != nullptr) {
      n = min(max(a.num_splits[b], 0), a.max_splits);
    } else if (a.seqlens != nullptr) {
      const int ctx = min(max(a.seqlens[b], 0), a.max_pages * a.page_size);
      const int npages = (ctx + a.page_size - 1) / a.page_size;
      n = max(1, (npages + a.pages_per_split - 1) / a.pages_per_split);
    }
  }
  if (a.skip_single && n == 1) return;   // the decode kernel already wrote such rows itself
  if (a.part_o16 != nullptr) combine_pair(a, a.part_o16, b, h, n, s0, lane);
  else combine_pair(a, a.part_o, b, h, n, s0, lane);
}

int launch_lse_combine(const CombineArgs& a, hipStream_t stream, const char* what) {
  if (a.B == 0 || a.H == 0) return DMLA_OK;
  if ((int64_t)a.B * a.H >= ((int64_t)1 << 31)) return fail(DMLA_ERR_UNSUPPORTED, "%s: B * H must be below 2^31", what);
  const dim3 grid((unsigned)(((int64_t)a.B * a.H + 3) / 4));
  if (a.split_base != nullptr && a.num_splits != nullptr)
    hipLaunchKernelGGL(lse_combine_kernel<true>, grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(lse_combine_kernel<false>, grid, dim3(256), 0, stream, a);
  return check_launch(what);
}

namespace {

// ---- paged append ------------------------------------------------------------------------
struct AppendArgs {
  bf16* pool;
  const int32_t* block_table;
  const int32_t* seqlens;
  const int32_t* new_lens;   // nullable: every sequence appends n_new rows
  const bf16* new_kv;
  int32_t* bad;              // nullable: set to 1 when a row's page slot or index is out of range
  int64_t pool_sp, pool_ss, bt_sb, nk_sb, nk_ss;
  int B, n_new, chunks;      // chunks = d / 8 (16-byte pieces per row)
  int page_size, num_pages, max_pages;
};

// One 16-byte piece per thread and step, consecutive threads on consecutive pieces of a row.
__global__ void __launch_bounds__(256) kv_append_kernel(AppendArgs a) {
  const int64_t total = (int64_t)a.B * a.n_new * a.chunks;
  for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < total; u += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(u % a.chunks);
    const int64_t bt = u / a.chunks;
    const int t = (int)(bt % a.n_new);
    const int b = (int)(bt / a.n_new);
    const int n = a.new_lens ? min(max(a.new_lens[b], 0), a.n_new) : a.n_new;
    if (t >= n) continue;
    const int64_t pos = (int64_t)max(a.seqlens[b], 0) + t;
    const int64_t slot = pos / a.page_size;
    const int page = slot < a.max_pages ? a.block_table[b * a.bt_sb + slot] : -1;
    if (page < 0 || page >= a.num_pages) {
      if (a.bad != nullptr) a.bad[0] = 1;
      continue;
    }
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(a.new_kv + b * a.nk_sb + t * a.nk_ss + 8 * c);
    *reinterpret_cast<bf16x8*>(a.pool + page * a.pool_sp + (pos % a.page_size) * a.pool_ss + 8 * c) = v;
  }
}

}  // namespace
}  // namespace dmla

using namespace dmla;

extern "C" int dmla_kv_append(void* kv_pool, const int32_t* block_table, const int32_t* cache_seqlens,
                              const int32_t* new_lens, const void* new_kv, int32_t* bad_index_flag, int64_t B,
                              int64_t n_new, int64_t d, int64_t page_size, int64_t num_pages,
                              int64_t max_pages_per_seq, int64_t kv_sp, int64_t kv_ss, int64_t bt_sb,
                              int64_t nk_sb, int64_t nk_ss, dmla_stream_t stream) {
  clear_error();
  if (!kv_pool || !block_table || !cache_seqlens || !new_kv)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_kv_append: null pointer argument");
  if (B < 0 || n_new < 0 || d <= 0 || page_size <= 0 || num_pages < 0 || max_pages_per_seq < 0)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_kv_append: negative or zero size");
  if (d % 8 != 0) return fail(DMLA_ERR_UNSUPPORTED, "dmla_kv_append: d must be a multiple of 8 (got %lld)", (long long)d);
  if (!aligned16(kv_pool) || !aligned16(new_kv))
    return fail(DMLA_ERR_INVALID_ARG, "dmla_kv_append: kv_pool and new_kv must be 16-byte aligned");
  if (!mult8(kv_sp) || !mult8(kv_ss) || !mult8(nk_sb) || !mult8(nk_ss) || kv_ss < d || kv_sp < page_size * kv_ss)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_kv_append: strides must be multiples of 8 and cover a row / page");
  if (bt_sb < max_pages_per_seq)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_kv_append: block_table row stride < max_pages_per_seq");
  if (B > ((int64_t)1 << 24) || n_new > ((int64_t)1 << 24) || num_pages > 0x7fffffff ||
      max_pages_per_seq > ((int64_t)1 << 24) || d / 8 > 0x7fffffff)
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_kv_append: size too large");
  if (B == 0 || n_new == 0) return DMLA_OK;
  AppendArgs a = {};
  a.pool = static_cast<bf16*>(kv_pool);
  a.block_table = block_table;
  a.seqlens = cache_seqlens;
  a.new_lens = new_lens;
  a.new_kv = static_cast<const bf16*>(new_kv);
  a.bad = bad_index_flag;
  a.pool_sp = kv_sp; a.pool_ss = kv_ss; a.bt_sb = bt_sb; a.nk_sb = nk_sb; a.nk_ss = nk_ss;
  a.B = (int)B; a.n_new = (int)n_new; a.chunks = (int)(d / 8);
  a.page_size = (int)page_size; a.num_pages = (int)num_pages; a.max_pages = (int)max_pages_per_seq;
  const int64_t total = B * n_new * (d / 8);
  const int64_t blocks = std::min<int64_t>((total + 255) / 256, (int64_t)device_cu_count() * 16);
  hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, a);
  return check_launch("dmla_kv_append");
}

extern "C" int dmla_lse_combine(const float* part_o, const float* part_lse, const int32_t* num_splits, void* o,
                                float* lse, int64_t B, int64_t H, int64_t max_splits, int64_t d, int64_t po_sb,
                                int64_t po_ss, int64_t po_sh, int64_t lse_sb, int64_t lse_ss, int64_t lse_sh,
                                int64_t o_sb, int64_t o_sh, dmla_stream_t stream) {
  clear_error();
  if (!part_o || !part_lse || !o) return fail(DMLA_ERR_INVALID_ARG, "dmla_lse_combine: null pointer argument");
  if (B < 0 || H < 0 || max_splits <= 0 || d <= 0)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_lse_combine: bad size");
  if (d % 4 != 0) return fail(DMLA_ERR_UNSUPPORTED, "dmla_lse_combine: d must be a multiple of 4");
  if (!aligned16(part_o) || (reinterpret_cast<uintptr_t>(o) & 7u) != 0)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_lse_combine: part_o must be 16-byte and o 8-byte aligned");
  if (po_sb % 4 || po_ss % 4 || po_sh % 4 || o_sb % 4 || o_sh % 4)
    return fail(DMLA_ERR_INVALID_ARG, "dmla_lse_combine: part_o / o strides must be multiples of 4 elements");
  if (B * H > 0x7fffffff || max_splits > 0x7fffffff || d > 0x7fffffff)
    return fail(DMLA_ERR_UNSUPPORTED, "dmla_lse_combine: size too large");
  CombineArgs a = {};
  a.part_o = part_o;
  a.part_lse = part_lse;
  a.num_splits = num_splits;
  a.o = static_cast<bf16*>(o);
  a.lse = lse;
  a.B = (int)B; a.H = (int)H; a.max_splits = (int)max_splits; a.d = (int)d;
  a.po_sb = po_sb; a.po_ss = po_ss; a.po_sh = po_sh;
  a.lse_sb = lse_sb; a.lse_ss = lse_ss; a.lse_sh = lse_sh;
  a.o_sb = o_sb; a.o_sh = o_sh;
  return launch_lse_combine(a, (hipStream_t)stream, "dmla_lse_combine");
}
