// EXL3 MoE per-launch stages on gfx950: the launches of the reference's unfused MoE path
// (cuda/csrc/exl3_marlin_moe.cu:376-618; run order cuda/src/sglang_exl3/kernels/marlin_moe.py:272-294), for callers
// that drive the stages themselves.  exl3_moe_forward (exl3_moe.hip) computes the same arithmetic in three launches.
//   exl3_moe_align       routing in the layout of vLLM's moe_align_block_size (the reference's moe_align_decode for
//                        one block size): experts' slot runs padded to the block size, the expert of every block
//   exl3_moe_had_in      the rotated inputs fp16(Had(fp16(x) * suh)) per (shard, slot)
//   exl3_moe_gemm        grouped expert GEMV/GEMM over the align blocks, fp32 accumulation, optional in-launch output
//                        transform fp16(Had(fp16(acc)) * svh)
//   exl3_moe_glu_had_in  a = fp16(silu(g) * u) in fp32, the rotated down inputs fp16(Had(fp16(a * suh_down)))
//   exl3_moe_combine     (exl3_moe.hip) weighted fp32 sum over a token's slots
// The weights stay in their stored layout, [E][k/16][n/16][16K] per projection: the reference's moe_gemm reads its
// repacked Marlin stack instead.
//
// exl3_moe_gemm: grid (shards * n / 128 column blocks, align blocks, k-splits), 8 waves; wave w decodes tile column
// 8 * block + w of the block's expert on the dense GEMV's streaming core (TileStream, 16 tile rows per chunk) and
// feeds every decoded tile to P 16-row MFMAs (the block's rows, P = block / 16 rounded up).  A block's rows are its
// sorted slot ids; padding entries (ids >= rows) stage zeros and are never stored.  Each k-split stores fp32 partials
// [split][row][column] with device-scope coherence; the last split of a (block, column block) to arrive sums them in
// split order (deterministic), rounds once to fp16, applies the output transform when asked, and stores the rows.
#include <stdlib.h>

#include <algorithm>

#include "exl3_api.hpp"
#include "exl3_device.hpp"
#include "exl3_stream.hpp"

namespace exl3 {

constexpr int kStageWaves = 8, kStageThreads = kStageWaves * 64;
constexpr int kStageNT = 16;                     // tile rows per chunk: NB = 2 blocks of 128 input rows
constexpr int kStageMStride = a_mstride(kStageNT);  // staged activation row stride (halves)
constexpr int kAlignThreads = 1024, kAlignMaxExperts = 1024;

struct StageStacks {
  const uint32_t* tr[2];   // per shard: [E][k/16][n/16][16K]
  const uint16_t* svh[2];  // per shard: [E][n], or null (no output transform)
  const uint16_t* suh[2];  // per shard: [E][k] (had_in)
};

template <int K, int P>
__host__ __device__ constexpr int stage_lds_bytes() {
  return 16 * P * kStageMStride * 2 + kStageWaves * stream_lds_bytes(K);
}

// ---- routing (one workgroup): per-expert counts (LDS atomics), then for each expert class (one class, or the K
// classes of a mixed layer: each its own expert map and block size) the padded runs of its experts by an exclusive
// scan, the block experts, and every slot of the class into its expert's run.  Slots keep no particular order inside
// a run (rows of a block are independent).
struct AlignClass {
  const int* emap;  // global id -> local id, -1: not in this class; null: every id in [0, E), local = global
  int block, cap, mblk;
  int* sorted;
  int* eids;
  int* post;
};
struct AlignClasses {
  AlignClass c[EXL3_MOE_MAX_CLASSES];
  int n;
};

__global__ __launch_bounds__(kAlignThreads) void moe_align_kernel(const int* __restrict__ ids, int slots, int E,
                                                                  AlignClasses ac) {
  __shared__ int cnt[kAlignMaxExperts], start[kAlignMaxExperts], fill[kAlignMaxExperts];
  __shared__ int scan[kAlignThreads];
  const int t = threadIdx.x;
  for (int e = t; e < kAlignMaxExperts; e += kAlignThreads) cnt[e] = 0;
  __syncthreads();
  for (int s = t; s < slots; s += kAlignThreads) {
    const int e = ids[s];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  for (int ci = 0; ci < ac.n; ci++) {
    const AlignClass c = ac.c[ci];
    for (int e = t; e < kAlignMaxExperts; e += kAlignThreads) fill[e] = 0;
    __syncthreads();  // counts complete; the previous class's fills done
    auto mine = [&](int e) { return e >= 0 && e < E && (c.emap == nullptr || c.emap[e] >= 0); };
    const int padded = mine(t) ? (cnt[t] + c.block - 1) / c.block * c.block : 0;
    scan[t] = padded;
    __syncthreads();
    for (int d = 1; d < kAlignThreads; d <<= 1) {  // inclusive Hillis-Steele scan
      const int v = t >= d ? scan[t - d] : 0;
      __syncthreads();
      scan[t] += v;
      __syncthreads();
    }
    const int total = scan[kAlignThreads - 1];
    if (t < E) start[t] = scan[t] - padded;
    // sentinels first (padding inside the runs and past the end), then the blocks' experts and the slots
    for (int i = t; i < c.cap; i += kAlignThreads) c.sorted[i] = slots;
    for (int i = t; i < c.mblk; i += kAlignThreads) c.eids[i] = -1;
    __syncthreads();
    if (padded > 0)
      for (int i = start[t]; i < start[t] + padded; i += c.block) c.eids[i / c.block] = c.emap ? c.emap[t] : t;
    for (int s = t; s < slots; s += kAlignThreads) {
      const int e = ids[s];
      if (mine(e)) c.sorted[start[e] + atomicAdd(&fill[e], 1)] = s;
    }
    if (t == 0) *c.post = total;
    __syncthreads();  // scan and start are rewritten by the next class
  }
}

// ---- rotated expert inputs: one half-wave per (shard, slot, 128-block); rows of unrouted slots are left alone
template <bool X_BF16>
__global__ __launch_bounds__(256) void moe_had_in_kernel(const void* __restrict__ x, int k, const int* __restrict__ ids,
                                                         int top_k, int slots, int E, StageStacks st, int shards,
                                                         uint16_t* __restrict__ xh) {
  const int kb = k >> 7;
  const int unit = blockIdx.x * 8 + (threadIdx.x >> 5);
  if (unit >= shards * slots * kb) return;
  const int t = threadIdx.x & 31;
  const int sh = unit / (slots * kb), rem = unit - sh * slots * kb, slot = rem / kb, b = rem - slot * kb;
  const int e = ids[slot];
  if (e < 0 || e >= E) return;
  const int kk = b * 128 + 4 * t;
  const uint16_t* xr = static_cast<const uint16_t*>(x) + (size_t)(slot / top_k) * k + kk;
  _Float16 v[4];
  if constexpr (X_BF16) {
    const uint2_t raw = *reinterpret_cast<const uint2_t*>(xr);
    v[0] = (_Float16)bf16_to_f32((uint16_t)(raw.x & 0xFFFF));
    v[1] = (_Float16)bf16_to_f32((uint16_t)(raw.x >> 16));
    v[2] = (_Float16)bf16_to_f32((uint16_t)(raw.y & 0xFFFF));
    v[3] = (_Float16)bf16_to_f32((uint16_t)(raw.y >> 16));
  } else {
    const half4_t raw = *reinterpret_cast<const half4_t*>(xr);
    v[0] = raw.x; v[1] = raw.y; v[2] = raw.z; v[3] = raw.w;
  }
  const half4_t su = *reinterpret_cast<const half4_t*>((sh ? st.suh[1] : st.suh[0]) + (size_t)e * k + kk);
  float f0 = (float)(_Float16)(v[0] * su.x), f1 = (float)(_Float16)(v[1] * su.y);
  float f2 = (float)(_Float16)(v[2] * su.z), f3 = (float)(_Float16)(v[3] * su.w);
  had128_x4(f0, f1, f2, f3);
  *reinterpret_cast<half4_t*>(xh + ((size_t)sh * slots + slot) * k + kk) =
      half4_t{had_scale_f16(f0), had_scale_f16(f1), had_scale_f16(f2), had_scale_f16(f3)};
}

// ---- GLU and the rotated down inputs: one half-wave per (slot, 128-block of the intermediate)
__global__ __launch_bounds__(256) void moe_glu_had_in_kernel(const uint16_t* __restrict__ gu, int slots, int inter,
                                                             const int* __restrict__ ids, int E,
                                                             const uint16_t* __restrict__ suh,
                                                             uint16_t* __restrict__ act, uint16_t* __restrict__ xd) {
  const int kb = inter >> 7;
  const int unit = blockIdx.x * 8 + (threadIdx.x >> 5);
  if (unit >= slots * kb) return;
  const int t = threadIdx.x & 31;
  const int slot = unit / kb, b = unit - slot * kb;
  const int e = ids[slot];
  if (e < 0 || e >= E) return;
  const int kk = b * 128 + 4 * t;
  const half4_t gv = *reinterpret_cast<const half4_t*>(gu + (size_t)slot * 2 * inter + kk);
  const half4_t uv = *reinterpret_cast<const half4_t*>(gu + (size_t)slot * 2 * inter + inter + kk);
  const half4_t su = *reinterpret_cast<const half4_t*>(suh + (size_t)e * inter + kk);
  const _Float16 a[4] = {f16_of_f32(silu32((float)gv.x) * (float)uv.x), f16_of_f32(silu32((float)gv.y) * (float)uv.y),
                         f16_of_f32(silu32((float)gv.z) * (float)uv.z), f16_of_f32(silu32((float)gv.w) * (float)uv.w)};
  if (act) *reinterpret_cast<half4_t*>(act + (size_t)slot * inter + kk) = half4_t{a[0], a[1], a[2], a[3]};
  float f0 = (float)(_Float16)(a[0] * su.x), f1 = (float)(_Float16)(a[1] * su.y);
  float f2 = (float)(_Float16)(a[2] * su.z), f3 = (float)(_Float16)(a[3] * su.w);
  had128_x4(f0, f1, f2, f3);
  *reinterpret_cast<half4_t*>(xd + (size_t)slot * inter + kk) =
      half4_t{had_scale_f16(f0), had_scale_f16(f1), had_scale_f16(f2), had_scale_f16(f3)};
}

// ---- grouped expert GEMV/GEMM over align blocks (see the header comment)
template <int K, int CB, int P>
__global__ __launch_bounds__(kStageThreads) void moe_block_gemm_kernel(
    StageStacks st, const uint16_t* __restrict__ a, int rows, int k, int n, int shards, const int* __restrict__ sorted,
    const int* __restrict__ eids, const int* __restrict__ post, int block, int E, uint16_t* __restrict__ c,
    float* partial, int* counters, int splits, int chunks, int bi0) {
  typedef TileStream<K, CB, kStageNT> Stream;
  constexpr int NB = Stream::NB;
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ int last_flag;
  _Float16* xs = reinterpret_cast<_Float16*>(lds);
  const int bi = bi0 + blockIdx.y;  // align block; this launch covers blocks bi0 .. bi0 + gridDim.y - 1
  if (bi * block >= *post) return;
  const int e = eids[bi];
  if (e < 0 || e >= E) return;
  const int* ids = sorted + (size_t)bi * block;
  const int ncb = n >> 7, n_total = shards * n;
  const int cb = blockIdx.x, sh = cb / ncb, cbl = cb - sh * ncb, sp = blockIdx.z;
  const int tn = n / 16;
  const int mat_bytes = (k >> 4) * tn * 32 * K;
  const uint32_t* trellis = (sh ? st.tr[1] : st.tr[0]) + (size_t)e * (mat_bytes / 4);
  const uint16_t* svh = sh ? st.svh[1] : st.svh[0];
  const uint16_t* arows = a + (size_t)sh * rows * k;
  const int kblocks = k >> 7;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, cl = l & 15, j = l >> 4;
  const int hw = threadIdx.x >> 5, t = threadIdx.x & 31;
  uint8_t* stage = lds + 16 * P * kStageMStride * 2 + w * Stream::LDS_BYTES;
  const int groups = (block + 15) / 16;

  float4_t acc[P];
#pragma unroll
  for (int p = 0; p < P; p++) acc[p] = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int ch = 0; ch < chunks; ch++) {
    const int kb0 = (sp * chunks + ch) * NB;
    if (kb0 >= kblocks) break;
    const int nb = min(kblocks, kb0 + NB) - kb0;
    Stream stream;
    stream.init(trellis, mat_bytes, tn, cbl * kStageWaves + w, kb0, nb, stage, l);
    stream.start();
    // every staged row of the P groups: the block's rows, zeros for padding entries and past the block
    for (int u = hw; u < 16 * P * NB; u += 2 * kStageWaves) {
      const int m = u / NB, b = u - m * NB;
      half4_t v = {0, 0, 0, 0};
      if (m < block && b < nb) {
        const int r = ids[m];
        if (r < rows) v = *reinterpret_cast<const half4_t*>(arows + (size_t)r * k + (kb0 + b) * 128 + 4 * t);
      }
      // a_slot keeps each even-odd pair of positions adjacent: two 4-byte writes
      *reinterpret_cast<half2_t*>(xs + a_slot(b * 128 + 4 * t, m, kStageMStride)) = half2_t{v[0], v[1]};
      *reinterpret_cast<half2_t*>(xs + a_slot(b * 128 + 4 * t + 2, m, kStageMStride)) = half2_t{v[2], v[3]};
    }
    __syncthreads();
    stream.template run_groups<P>(reinterpret_cast<const half8_t*>(xs + cl * kStageMStride) + j,
                                  16 * kStageMStride / 8, groups, acc);
    __syncthreads();  // the next chunk restages LDS
  }
  // this split's partial rows (lane: rows 16 p + 4 j + r, column cl of the wave's 16), device-coherent: read by the
  // last split, possibly on another XCD
  float* pdst = partial + (size_t)sp * rows * n_total + cb * 128 + w * 16 + cl;
#pragma unroll
  for (int p = 0; p < P; p++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int m = 16 * p + 4 * j + r;
      if (m < block) {
        const int row = ids[m];
        if (row < rows) __hip_atomic_store(pdst + (size_t)row * n_total, acc[p][r], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  const int ctr = blockIdx.y * (shards * ncb) + cb;  // counters are per launch: launches are ordered on the stream
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&counters[ctr], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev == splits - 1;
  }
  __syncthreads();
  if (!last_flag) return;
  // last split: one row per half-wave, 4 columns per lane, splits summed in order, one rounding
  const int col = cb * 128 + 4 * t;
  for (int m = hw; m < block; m += 2 * kStageWaves) {
    const int row = ids[m];
    if (row >= rows) continue;
    float4_t s4 = {0.f, 0.f, 0.f, 0.f};
    for (int q = 0; q < splits; q++) {
      const uint64_t* src = reinterpret_cast<const uint64_t*>(partial + ((size_t)q * rows + row) * n_total + col);
      const uint64_t lo = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint64_t hi = __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s4 += float4_t{__builtin_bit_cast(float, (uint32_t)lo), __builtin_bit_cast(float, (uint32_t)(lo >> 32)),
                     __builtin_bit_cast(float, (uint32_t)hi), __builtin_bit_cast(float, (uint32_t)(hi >> 32))};
    }
    _Float16 h[4] = {(_Float16)s4.x, (_Float16)s4.y, (_Float16)s4.z, (_Float16)s4.w};
    if (svh) {
      float f0 = (float)h[0], f1 = (float)h[1], f2 = (float)h[2], f3 = (float)h[3];
      had128_x4(f0, f1, f2, f3);
      const half4_t sv = *reinterpret_cast<const half4_t*>(svh + (size_t)e * n + cbl * 128 + 4 * t);
      h[0] = (_Float16)(had_scale_f16(f0) * sv.x);
      h[1] = (_Float16)(had_scale_f16(f1) * sv.y);
      h[2] = (_Float16)(had_scale_f16(f2) * sv.z);
      h[3] = (_Float16)(had_scale_f16(f3) * sv.w);
    }
    *reinterpret_cast<half4_t*>(c + (size_t)row * n_total + col) = half4_t{h[0], h[1], h[2], h[3]};
  }
  if (threadIdx.x == 0) __hip_atomic_store(&counters[ctr], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---- host ----------------------------------------------------------------------------------------------------------

// k-splits of exl3_moe_gemm: chunks of 2 blocks of 128 input rows dealt to `splits` workgroups, enough splits for
// about 2048 workgroups over the blocks that can hold rows (at most min(max_blocks, rows)), at most 8
struct StagePlan {
  int splits, chunks;
  size_t partial_off, total;
};

static StagePlan stage_plan(int rows, int k, int n, int shards, int max_blocks) {
  StagePlan p{};
  const int C = (k / 128 + 1) / 2;
  const int grid_xy = std::max(1, std::min(max_blocks, rows)) * shards * (n / 128);
  const int want = std::max(1, (2048 + grid_xy - 1) / grid_xy);
  const int s = std::max(1, std::min(C, std::min(8, want)));
  p.chunks = (C + s - 1) / s;
  p.splits = (C + p.chunks - 1) / p.chunks;
  p.partial_off = kCounterBytes;
  p.total = p.partial_off + (((size_t)p.splits * rows * shards * n * 4 + 255) & ~(size_t)255);
  return p;
}

#define EXL3_STAGE_DISPATCH(K_, CB_, ...)                                 \
  [&]() -> bool {                                                         \
    switch (K_ * 4 + CB_) {                                               \
      EXL3_SCASE(2, __VA_ARGS__) EXL3_SCASE(3, __VA_ARGS__)               \
      EXL3_SCASE(4, __VA_ARGS__) EXL3_SCASE(5, __VA_ARGS__)               \
      EXL3_SCASE(6, __VA_ARGS__) EXL3_SCASE(8, __VA_ARGS__)               \
      default: return false;                                              \
    }                                                                     \
  }()
#define EXL3_SCASE(KV, ...)                                                            \
  case KV * 4 + 0: { constexpr int kK = KV, kCB = 0; __VA_ARGS__; return true; }      \
  case KV * 4 + 1: { constexpr int kK = KV, kCB = 1; __VA_ARGS__; return true; }      \
  case KV * 4 + 2: { constexpr int kK = KV, kCB = 2; __VA_ARGS__; return true; }

}  // namespace exl3

using namespace exl3;

static int check_align_class(const char* what, int slots, int num_experts, int block, int cap, int max_blocks,
                             const int* sorted_ids, const int* expert_ids, const int* num_post_padded) {
  EXL3_CHECK_ARG(sorted_ids && expert_ids && num_post_padded, "%s: null output pointer", what);
  EXL3_CHECK_ARG(block >= 1 && block <= 64, "%s: block = %d (1..64)", what, block);
  EXL3_CHECK_ARG((int64_t)cap >= (int64_t)slots + (int64_t)num_experts * (block - 1),
                 "%s: sorted_ids holds %d entries, the padded runs may need %lld", what, cap,
                 (long long)slots + (long long)num_experts * (block - 1));
  EXL3_CHECK_ARG((int64_t)max_blocks * block >= cap, "%s: expert_ids holds %d blocks of %d, fewer than %d", what,
                 max_blocks, block, cap);
  return EXL3_OK;
}

extern "C" int exl3_moe_align(const int* topk_ids, int slots, int num_experts, const int* expert_map, int block,
                              int* sorted_ids, int cap, int* expert_ids, int max_blocks, int* num_post_padded,
                              void* stream) {
  return exl3_moe_align_classes(topk_ids, slots, num_experts, 1, &expert_map, &block, &sorted_ids, &cap, &expert_ids,
                                &max_blocks, &num_post_padded, stream);
}

extern "C" int exl3_moe_align_classes(const int* topk_ids, int slots, int num_experts, int nclasses,
                                      const int* const* expert_maps_host, const int* blocks_host,
                                      int* const* sorted_ids_host, const int* caps_host,
                                      int* const* expert_ids_host, const int* max_blocks_host,
                                      int* const* num_post_padded_host, void* stream) {
  const char* what = nclasses == 1 ? "exl3_moe_align" : "exl3_moe_align_classes";
  EXL3_CHECK_ARG(slots == 0 || topk_ids, "%s: null pointer", what);
  EXL3_CHECK_ARG(nclasses >= 1 && nclasses <= EXL3_MOE_MAX_CLASSES, "%s: nclasses = %d (1..%d)", what, nclasses,
                 EXL3_MOE_MAX_CLASSES);
  EXL3_CHECK_ARG(expert_maps_host && blocks_host && sorted_ids_host && caps_host && expert_ids_host &&
                     max_blocks_host && num_post_padded_host,
                 "%s: null pointer", what);
  EXL3_CHECK_ARG(slots >= 0 && slots <= (1 << 24), "%s: slots = %d", what, slots);
  EXL3_CHECK_ARG(num_experts >= 1 && num_experts <= kAlignMaxExperts, "%s: num_experts = %d (1..%d)", what,
                 num_experts, kAlignMaxExperts);
  EXL3_CHECK_ARG(nclasses == 1 || (expert_maps_host[0] && expert_maps_host[1]),
                 "%s: every class of a mixed layer needs its expert map", what);
  AlignClasses ac{};
  ac.n = nclasses;
  for (int c = 0; c < nclasses; c++) {
    if (int rc = check_align_class(what, slots, num_experts, blocks_host[c], caps_host[c], max_blocks_host[c],
                                   sorted_ids_host[c], expert_ids_host[c], num_post_padded_host[c]))
      return rc;
    ac.c[c] = AlignClass{expert_maps_host[c], blocks_host[c], caps_host[c], max_blocks_host[c], sorted_ids_host[c],
                         expert_ids_host[c], num_post_padded_host[c]};
  }
  moe_align_kernel<<<1, kAlignThreads, 0, as_stream(stream)>>>(topk_ids, slots, num_experts, ac);
  EXL3_CHECK_LAUNCH();
  return EXL3_OK;
}

extern "C" int exl3_moe_had_in(const void* x, int x_bf16, int tokens, int k, const int* topk_ids, int top_k,
                               int num_experts, const void* const* suh, int shards, void* xh, void* stream) {
  EXL3_CHECK_ARG((tokens == 0 || (x && topk_ids && xh)) && suh, "exl3_moe_had_in: null pointer");
  EXL3_CHECK_ARG(shards == 1 || shards == 2, "exl3_moe_had_in: shards = %d (1 or 2)", shards);
  EXL3_CHECK_ARG(suh[0] && (shards == 1 || suh[1]), "exl3_moe_had_in: null suh");
  EXL3_CHECK_ARG(tokens >= 0 && top_k >= 1 && k > 0 && k % 128 == 0 && num_experts >= 1,
                 "exl3_moe_had_in: tokens = %d, top_k = %d, k = %d, num_experts = %d", tokens, top_k, k, num_experts);
  const int64_t slots = (int64_t)tokens * top_k;
  EXL3_CHECK_ARG(slots * shards * k <= INT32_MAX, "exl3_moe_had_in: too many rows");
  if (slots == 0) return EXL3_OK;
  StageStacks st{};
  st.suh[0] = static_cast<const uint16_t*>(suh[0]);
  st.suh[1] = shards > 1 ? static_cast<const uint16_t*>(suh[1]) : nullptr;
  const dim3 grid((unsigned)((slots * shards * (k / 128) + 7) / 8));
  if (x_bf16)
    moe_had_in_kernel<true><<<grid, 256, 0, as_stream(stream)>>>(x, k, topk_ids, top_k, (int)slots, num_experts, st,
                                                                 shards, static_cast<uint16_t*>(xh));
  else
    moe_had_in_kernel<false><<<grid, 256, 0, as_stream(stream)>>>(x, k, topk_ids, top_k, (int)slots, num_experts, st,
                                                                  shards, static_cast<uint16_t*>(xh));
  EXL3_CHECK_LAUNCH();
  return EXL3_OK;
}

extern "C" size_t exl3_moe_gemm_workspace_bytes(int rows, int k, int n, int shards, int max_blocks) {
  if (rows <= 0 || k <= 0 || k % 128 || n <= 0 || n % 128 || shards < 1 || shards > 2 || max_blocks <= 0) return 0;
  if (shards * (n / 128) > kMaxCounters) return 0;
  return stage_plan(rows, k, n, shards, max_blocks).total;
}

extern "C" int exl3_moe_gemm(const void* a, int rows, int k, const void* const* trellis, const void* const* svh,
                             int shards, int n, const int* sorted_ids, const int* expert_ids,
                             const int* num_post_padded, int max_blocks, int block, int num_experts, int K,
                             int codebook, void* c, void* workspace, size_t workspace_bytes, void* stream) {
  EXL3_CHECK_ARG((rows == 0 || (a && sorted_ids && expert_ids && num_post_padded && c)) && trellis,
                 "exl3_moe_gemm: null pointer");
  EXL3_CHECK_ARG(shards == 1 || shards == 2, "exl3_moe_gemm: shards = %d (1 or 2)", shards);
  EXL3_CHECK_ARG(trellis[0] && (shards == 1 || trellis[1]), "exl3_moe_gemm: null trellis");
  EXL3_CHECK_ARG(!svh || (svh[0] && (shards == 1 || svh[1])), "exl3_moe_gemm: svh given with a null shard");
  EXL3_CHECK_ARG(valid_bits(K) && valid_cb(codebook), "exl3_moe_gemm: K = %d / codebook = %d", K, codebook);
  EXL3_CHECK_ARG(rows >= 0 && k > 0 && k % 128 == 0 && n > 0 && n % 128 == 0,
                 "exl3_moe_gemm: rows = %d, k = %d, n = %d (k, n multiples of 128)", rows, k, n);
  EXL3_CHECK_ARG(block >= 1 && block <= 64 && max_blocks >= 1 && num_experts >= 1,
                 "exl3_moe_gemm: block = %d (1..64), max_blocks = %d, num_experts = %d", block, max_blocks,
                 num_experts);
  EXL3_CHECK_ARG((int64_t)k * n * K / 8 <= INT32_MAX, "exl3_moe_gemm: expert matrix exceeds the 2 GiB buffer range");
  EXL3_CHECK_ARG(shards * (n / 128) <= kMaxCounters, "exl3_moe_gemm: %d column blocks exceed the counter region",
                 shards * (n / 128));
  EXL3_CHECK_ARG((int64_t)rows * shards * n <= INT32_MAX / 8, "exl3_moe_gemm: too many rows");
  if (rows == 0) return EXL3_OK;
  const StagePlan p = stage_plan(rows, k, n, shards, max_blocks);
  EXL3_CHECK_ARG(workspace && workspace_bytes >= p.total, "exl3_moe_gemm: workspace %zu bytes, need %zu",
                 workspace_bytes, p.total);
  StageStacks st{};
  st.tr[0] = static_cast<const uint32_t*>(trellis[0]);
  st.tr[1] = shards > 1 ? static_cast<const uint32_t*>(trellis[1]) : nullptr;
  st.svh[0] = svh ? static_cast<const uint16_t*>(svh[0]) : nullptr;
  st.svh[1] = svh && shards > 1 ? static_cast<const uint16_t*>(svh[1]) : nullptr;
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  float* partial = reinterpret_cast<float*>(ws + p.partial_off);
  int* counters = reinterpret_cast<int*>(ws);
  hipStream_t s = as_stream(stream);
  const uint16_t* av = static_cast<const uint16_t*>(a);
  uint16_t* cv = static_cast<uint16_t*>(c);
  // One counter per (align block, column block) of a launch: align blocks go out in launches of at most
  // kMaxCounters / column blocks each (one launch up to 65536 / 32 = 2048 blocks at H = 4096, two column shards).
  // Launches are ordered on the stream and every launch leaves its counters at zero, so the next reuses them; a row
  // belongs to one block, so launches never share partial rows.
  const int per_launch = kMaxCounters / (shards * (n / 128));
  for (int b0 = 0; b0 < max_blocks; b0 += per_launch) {
    const dim3 grid((unsigned)(shards * (n / 128)), (unsigned)std::min(per_launch, max_blocks - b0),
                    (unsigned)p.splits);
    const bool ok = EXL3_STAGE_DISPATCH(K, codebook, {
      if (block <= 16)
        moe_block_gemm_kernel<kK, kCB, 1><<<grid, kStageThreads, stage_lds_bytes<kK, 1>(), s>>>(
            st, av, rows, k, n, shards, sorted_ids, expert_ids, num_post_padded, block, num_experts, cv, partial,
            counters, p.splits, p.chunks, b0);
      else if (block <= 32)
        moe_block_gemm_kernel<kK, kCB, 2><<<grid, kStageThreads, stage_lds_bytes<kK, 2>(), s>>>(
            st, av, rows, k, n, shards, sorted_ids, expert_ids, num_post_padded, block, num_experts, cv, partial,
            counters, p.splits, p.chunks, b0);
      else
        moe_block_gemm_kernel<kK, kCB, 4><<<grid, kStageThreads, stage_lds_bytes<kK, 4>(), s>>>(
            st, av, rows, k, n, shards, sorted_ids, expert_ids, num_post_padded, block, num_experts, cv, partial,
            counters, p.splits, p.chunks, b0);
    });
    if (!ok) return set_error(EXL3_ERR_INVALID, "exl3_moe_gemm: unsupported K = %d / codebook = %d", K, codebook);
    EXL3_CHECK_LAUNCH();
  }
  return EXL3_OK;
}

extern "C" int exl3_moe_glu_had_in(const void* gu, int slots, int inter, const int* topk_ids, int num_experts,
                                   const void* suh_down, void* act, void* xd, void* stream) {
  EXL3_CHECK_ARG((slots == 0 || (gu && topk_ids && xd)) && suh_down, "exl3_moe_glu_had_in: null pointer");
  EXL3_CHECK_ARG(slots >= 0 && inter > 0 && inter % 128 == 0 && num_experts >= 1,
                 "exl3_moe_glu_had_in: slots = %d, inter = %d, num_experts = %d", slots, inter, num_experts);
  EXL3_CHECK_ARG(slots == 0 || (act != xd && act != gu), "exl3_moe_glu_had_in: act must not alias gu or xd");
  EXL3_CHECK_ARG((int64_t)slots * 2 * inter <= INT32_MAX, "exl3_moe_glu_had_in: too many rows");
  if (slots == 0) return EXL3_OK;
  const dim3 grid((unsigned)(((int64_t)slots * (inter / 128) + 7) / 8));
  moe_glu_had_in_kernel<<<grid, 256, 0, as_stream(stream)>>>(
      static_cast<const uint16_t*>(gu), slots, inter, topk_ids, num_experts, static_cast<const uint16_t*>(suh_down),
      static_cast<uint16_t*>(act), static_cast<uint16_t*>(xd));
  EXL3_CHECK_LAUNCH();
  return EXL3_OK;
}
