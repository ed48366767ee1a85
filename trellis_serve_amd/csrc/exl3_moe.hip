// EXL3 MoE layer on gfx950: routing, grouped decode-GEMV for gate/up and for down, weighted combine.
//
// Reference semantics (cuda/csrc/exl3_marlin_moe.cu:210-292, run order cuda/src/sglang_exl3/kernels/marlin_moe.py:
// 272-294): a slot is (token t, choice j), slot = t * top_k + j, with expert e = topk_ids[t, j];
//   g, u = fp16 outputs of the gate / up linears of expert e on x[t] (input rotation with suh, output rotation * svh)
//   a    = fp16_rn(silu(g) * u) in fp32 (exl3_marlin_moe.cu:228-258)
//   d    = fp16 output of the down linear of expert e on a
//   y[t] = sum_j w[t, j] * d[slot] in fp32, slot order, one rounding; slots whose expert id is outside [0, E) are
//          skipped (exl3_marlin_moe.cu:274)
//
// Launches (the reference uses five plus an align launch; a single token skips the routing launch and runs its top-k
// slots directly):
//   moe_route_kernel   one workgroup: per-expert slot counts and lists (LDS atomics), the active experts in
//                      ascending order.  The order of slots inside an expert's list does not change any result: the
//                      rows of an MFMA are independent and the combine sums in slot order.
//   moe_gemv_kernel<PHASE 0>  grid (2I/128 column blocks, active experts, k-splits): gate/up of every active expert
//                      for all its slots, 16 slots per pass (TileStream, the dense GEMV's streaming core), input
//                      rotation of x[token] with the shard's suh in the prologue, split-K reduce + output rotation
//                      * svh by the last split, fp16 g|u rows.
//   moe_gemv_kernel<PHASE 1>  same for down; the prologue computes a = fp16(silu(g) * u) and its rotation with
//                      suh_down (the reference's separate GLU launch, fused).
//   moe_combine_kernel weighted fp32 sum over the token's slots.
#include <stdlib.h>

#include <algorithm>

#include "exl3_api.hpp"
#include "exl3_device.hpp"
#include "exl3_stream.hpp"

namespace exl3 {

constexpr int kMoeWaves = 8, kMoeThreads = kMoeWaves * 64, kMoeNT = 16;
constexpr int kMoeRows = 16;

struct MoeArgs {
  const uint32_t* tr[3];   // gate, up: [E][H/16][I/16][16K]; down: [E][I/16][H/16][16K]
  const uint16_t* suh[3];  // gate, up: [E][H]; down: [E][I]
  const uint16_t* svh[3];  // gate, up: [E][I]; down: [E][H]
  int E, H, I, top_k, slots;
  const int* counts;       // [E]
  const int* n_active;     // [1]
  const int* active;       // [E]: active experts, ascending
  const int* lists;        // [E][slots]
  const int* topk_ids;     // [slots]: read directly in slot mode
  int slot_mode;           // 1: one workgroup row per slot, no routing launch (a single token: its top-k experts)
};

__global__ __launch_bounds__(1024) void moe_route_kernel(const int* __restrict__ topk_ids, int slots, int E,
                                                         int* __restrict__ counts, int* __restrict__ n_active,
                                                         int* __restrict__ active, int* __restrict__ lists) {
  __shared__ int cnt[1024];
  __shared__ int scan[1024];
  const int tid = threadIdx.x;
  cnt[tid] = 0;
  __syncthreads();
  for (int s = tid; s < slots; s += 1024) {
    const int e = topk_ids[s];
    if (e >= 0 && e < E) {
      const int pos = atomicAdd(&cnt[e], 1);
      lists[(size_t)e * slots + pos] = s;
    }
  }
  __syncthreads();
  const int flag = tid < E && cnt[tid] > 0;
  scan[tid] = flag;
  __syncthreads();
  for (int d = 1; d < 1024; d <<= 1) {  // inclusive Hillis-Steele scan
    const int v = tid >= d ? scan[tid - d] : 0;
    __syncthreads();
    scan[tid] += v;
    __syncthreads();
  }
  if (tid < E) {
    counts[tid] = cnt[tid];
    if (flag) active[scan[tid] - 1] = tid;
  }
  if (tid == 1023) *n_active = scan[1023];
}

// LDS: staged activations [16 rows][NT*16 + 4 halves], then per wave the stream stages; the epilogue reduce reuses it
template <int K>
__host__ __device__ constexpr int moe_lds_bytes() {
  return kMoeRows * (kMoeNT * 16 + 4) * 2 + kMoeWaves * TileStream<K, 0, kMoeNT>::LDS_BYTES > kMoeThreads * 16
             ? kMoeRows * (kMoeNT * 16 + 4) * 2 + kMoeWaves * TileStream<K, 0, kMoeNT>::LDS_BYTES
             : kMoeThreads * 16;
}

__device__ __forceinline__ float silu32(float v) { return v / (1.0f + __expf(-v)); }

template <int K, int CB, int PHASE>
__global__ __launch_bounds__(kMoeThreads) void moe_gemv_kernel(MoeArgs a, const void* __restrict__ x, int x_bf16,
                                                                uint16_t* __restrict__ gu, uint16_t* __restrict__ dn,
                                                                float* __restrict__ partial,
                                                                int* __restrict__ counters, int splits) {
  typedef TileStream<K, CB, kMoeNT> Stream;
  constexpr int NB = Stream::NB;
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ int last_flag;
  _Float16* xs = reinterpret_cast<_Float16*>(lds);
  const int mstride = kMoeNT * 16 + 4;

  // expert and its slots: routed mode -- grid row = active expert, its slot list from the routing launch; slot mode
  // -- grid row = slot, one slot, its expert read from topk_ids (split counters then index slots, so repeated experts
  // in one token are still right)
  int e, n_e, ctr_row;
  const int* list;
  if (a.slot_mode) {
    e = a.topk_ids[blockIdx.y];
    if (e < 0 || e >= a.E) return;
    n_e = 1;
    list = nullptr;
    ctr_row = blockIdx.y;
  } else {
    if ((int)blockIdx.y >= *a.n_active) return;
    e = a.active[blockIdx.y];
    n_e = a.counts[e];
    list = a.lists + (size_t)e * a.slots;
    ctr_row = e;
  }
  auto slot_at = [&](int idx) { return a.slot_mode ? (int)blockIdx.y : list[idx]; };
  const int cb = blockIdx.x, sp = blockIdx.z;
  const int k = PHASE ? a.I : a.H;            // input width
  const int n_out = PHASE ? a.H : 2 * a.I;    // output row width (g|u for gate/up)
  const int sh = PHASE ? 2 : (cb < a.I / 128 ? 0 : 1);
  const int n_sh = PHASE ? a.H : a.I;         // output width of the shard
  const int cbl = PHASE ? cb : cb - (sh ? a.I / 128 : 0);  // column block inside the shard
  const int tn = n_sh / 16;
  const int mat_bytes = (k >> 4) * tn * 32 * K;
  const uint32_t* trellis = a.tr[sh] + (size_t)e * (mat_bytes / 4);
  const uint16_t* suh = a.suh[sh] + (size_t)e * k;
  const uint16_t* svh = a.svh[sh] + (size_t)e * n_sh;
  const int kb0 = sp * NB;
  const int nb = min(k >> 7, kb0 + NB) - kb0;

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, c = l & 15, j = l >> 4;
  const int hw = threadIdx.x >> 5, t = threadIdx.x & 31;
  uint8_t* stage = lds + kMoeRows * mstride * 2 + w * Stream::LDS_BYTES;

  for (int c0 = 0; c0 < n_e; c0 += kMoeRows) {
    const int M = min(kMoeRows, n_e - c0);
    Stream stream;
    stream.init(trellis, mat_bytes, tn, cbl * kMoeWaves + w, kb0, nb, stage, l);
    stream.start();
    for (int u = hw; u < M * NB; u += 2 * kMoeWaves) {
      const int m = u / NB, b = u - m * NB;
      const int kk = (kb0 + b) * 128 + 4 * t;
      const int slot = slot_at(c0 + m);
      _Float16 h[4] = {0, 0, 0, 0};
      if (b < nb) {
        float f[4];
        if constexpr (PHASE == 0) {
          const uint16_t* xr = static_cast<const uint16_t*>(x) + (size_t)(slot / a.top_k) * a.H + kk;
          _Float16 v[4];
          if (x_bf16) {
            const uint2_t raw = *reinterpret_cast<const uint2_t*>(xr);
            v[0] = (_Float16)bf16_to_f32((uint16_t)(raw.x & 0xFFFF));
            v[1] = (_Float16)bf16_to_f32((uint16_t)(raw.x >> 16));
            v[2] = (_Float16)bf16_to_f32((uint16_t)(raw.y & 0xFFFF));
            v[3] = (_Float16)bf16_to_f32((uint16_t)(raw.y >> 16));
          } else {
            const half4_t raw = *reinterpret_cast<const half4_t*>(xr);
            v[0] = raw.x; v[1] = raw.y; v[2] = raw.z; v[3] = raw.w;
          }
          const half4_t su = *reinterpret_cast<const half4_t*>(suh + kk);
          f[0] = (float)(_Float16)(v[0] * su.x); f[1] = (float)(_Float16)(v[1] * su.y);
          f[2] = (float)(_Float16)(v[2] * su.z); f[3] = (float)(_Float16)(v[3] * su.w);
        } else {
          const half4_t gv = *reinterpret_cast<const half4_t*>(gu + (size_t)slot * 2 * a.I + kk);
          const half4_t uv = *reinterpret_cast<const half4_t*>(gu + (size_t)slot * 2 * a.I + a.I + kk);
          const half4_t su = *reinterpret_cast<const half4_t*>(suh + kk);
          f[0] = (float)((_Float16)(silu32((float)gv.x) * (float)uv.x) * su.x);
          f[1] = (float)((_Float16)(silu32((float)gv.y) * (float)uv.y) * su.y);
          f[2] = (float)((_Float16)(silu32((float)gv.z) * (float)uv.z) * su.z);
          f[3] = (float)((_Float16)(silu32((float)gv.w) * (float)uv.w) * su.w);
        }
        had128_x4(f[0], f[1], f[2], f[3]);
#pragma unroll
        for (int i = 0; i < 4; i++) h[i] = (_Float16)(f[i] * kHadScale);
      }
#pragma unroll
      for (int i = 0; i < 4; i++) xs[a_slot(b * 128 + 4 * t + i, m, mstride)] = h[i];
    }
    __syncthreads();
    const float4_t acc = stream.run(reinterpret_cast<const half4_t*>(xs + min(c, M - 1) * mstride) + j);
    // this split's partial rows, device-coherent (read by the last split, possibly on another XCD)
    float* pdst = partial + (size_t)sp * a.slots * n_out + cb * 128 + w * 16 + c;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int m = 4 * j + r;
      if (m < M)
        __hip_atomic_store(pdst + (size_t)slot_at(c0 + m) * n_out, acc[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();  // the next pass restages LDS
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = __hip_atomic_fetch_add(&counters[ctr_row * (n_out / 128) + cb], 1, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev == splits - 1;
  }
  __syncthreads();
  if (!last_flag) return;

  // last split: every slot's 128 columns, splits summed in order, one rounding, output rotation * svh
  uint16_t* out = PHASE ? dn : gu;
  const int col = cb * 128 + 4 * t;
  for (int m = hw; m < n_e; m += 2 * kMoeWaves) {
    const int slot = slot_at(m);
    float4_t s4 = {0.f, 0.f, 0.f, 0.f};
    for (int p = 0; p < splits; p++) {
      const float* src = partial + ((size_t)p * a.slots + slot) * n_out + col;
      float4_t v;
      v.x = __hip_atomic_load(src + 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v.y = __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v.z = __hip_atomic_load(src + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      v.w = __hip_atomic_load(src + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s4 += v;
    }
    _Float16 h[4] = {(_Float16)s4.x, (_Float16)s4.y, (_Float16)s4.z, (_Float16)s4.w};
    float f0 = (float)h[0], f1 = (float)h[1], f2 = (float)h[2], f3 = (float)h[3];
    had128_x4(f0, f1, f2, f3);
    const half4_t sv = *reinterpret_cast<const half4_t*>(svh + cbl * 128 + 4 * t);
    const half4_t o = {(_Float16)((_Float16)(f0 * kHadScale) * sv.x), (_Float16)((_Float16)(f1 * kHadScale) * sv.y),
                       (_Float16)((_Float16)(f2 * kHadScale) * sv.z), (_Float16)((_Float16)(f3 * kHadScale) * sv.w)};
    *reinterpret_cast<half4_t*>(out + (size_t)slot * n_out + col) = o;
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(&counters[ctr_row * (n_out / 128) + cb], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <bool Y_BF16>
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t* __restrict__ dn,
                                                          const int* __restrict__ topk_ids,
                                                          const float* __restrict__ topk_w, int tokens, int top_k,
                                                          int E, int H, void* __restrict__ y) {
  const int nb = H >> 7;
  const int unit = blockIdx.x * 8 + (threadIdx.x >> 5);
  if (unit >= tokens * nb) return;
  const int t = threadIdx.x & 31;
  const int tok = unit / nb, b = unit - tok * nb;
  const int col = b * 128 + 4 * t;
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int jj = 0; jj < top_k; jj++) {
    const int slot = tok * top_k + jj;
    const int e = topk_ids[slot];
    if (e < 0 || e >= E) continue;
    const float wgt = topk_w[slot];
    const half4_t v = *reinterpret_cast<const half4_t*>(dn + (size_t)slot * H + col);
    acc.x += wgt * (float)v.x;
    acc.y += wgt * (float)v.y;
    acc.z += wgt * (float)v.z;
    acc.w += wgt * (float)v.w;
  }
  uint16_t* yr = static_cast<uint16_t*>(y) + (size_t)tok * H + col;
  if constexpr (Y_BF16) {
    uint2_t o;
    o.x = (uint32_t)f32_to_bf16(acc.x) | ((uint32_t)f32_to_bf16(acc.y) << 16);
    o.y = (uint32_t)f32_to_bf16(acc.z) | ((uint32_t)f32_to_bf16(acc.w) << 16);
    *reinterpret_cast<uint2_t*>(yr) = o;
  } else {
    *reinterpret_cast<half4_t*>(yr) = half4_t{(_Float16)acc.x, (_Float16)acc.y, (_Float16)acc.z, (_Float16)acc.w};
  }
}

// ---- host ----------------------------------------------------------------------------------------------------------

struct MoePlan {
  int splits_gu, splits_dn;
  size_t off_counts, off_nactive, off_active, off_lists, off_gu, off_dn, off_cnt_gu, off_cnt_dn, off_partial, total;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static int moe_splits(int slots, int E, int nblk, int k) {
  const int active = std::max(1, std::min(E, slots));
  const int want = (1536 + active * nblk - 1) / (active * nblk);
  const int maxs = (k / 128 + (kMoeNT / 8) - 1) / (kMoeNT / 8);
  return std::max(1, std::min(want, maxs));
}

static MoePlan moe_plan(int tokens, int top_k, int E, int H, int I) {
  MoePlan p{};
  const int slots = tokens * top_k;
  p.splits_gu = moe_splits(slots, E, 2 * I / 128, H);
  p.splits_dn = moe_splits(slots, E, H / 128, I);
  // the split counters first, in the fixed counter region (zero between calls whatever the shapes)
  p.off_cnt_gu = 0;
  p.off_cnt_dn = (size_t)E * (2 * I / 128) * 4;
  size_t o = kCounterBytes;
  p.off_counts = o; o = align256(o + (size_t)E * 4);
  p.off_nactive = o; o = align256(o + 4);
  p.off_active = o; o = align256(o + (size_t)E * 4);
  p.off_lists = o; o = align256(o + (size_t)E * slots * 4);
  p.off_gu = o; o = align256(o + (size_t)slots * 2 * I * 2);
  p.off_dn = o; o = align256(o + (size_t)slots * H * 2);
  p.off_partial = o;
  o = align256(o + std::max((size_t)p.splits_gu * slots * 2 * I, (size_t)p.splits_dn * slots * H) * 4);
  p.total = o;
  return p;
}

#define EXL3_MOE_DISPATCH(K_, CB_, ...)                                   \
  [&]() -> bool {                                                         \
    switch (K_ * 4 + CB_) {                                               \
      EXL3_MCASE(2, __VA_ARGS__) EXL3_MCASE(3, __VA_ARGS__)               \
      EXL3_MCASE(4, __VA_ARGS__) EXL3_MCASE(5, __VA_ARGS__)               \
      EXL3_MCASE(6, __VA_ARGS__) EXL3_MCASE(8, __VA_ARGS__)               \
      default: return false;                                              \
    }                                                                     \
  }()
#define EXL3_MCASE(KV, ...)                                                            \
  case KV * 4 + 0: { constexpr int kK = KV, kCB = 0; __VA_ARGS__; return true; }      \
  case KV * 4 + 1: { constexpr int kK = KV, kCB = 1; __VA_ARGS__; return true; }      \
  case KV * 4 + 2: { constexpr int kK = KV, kCB = 2; __VA_ARGS__; return true; }

}  // namespace exl3

using namespace exl3;

extern "C" size_t exl3_moe_workspace_bytes(int tokens, int top_k, int num_experts, int hidden, int inter, int K) {
  (void)K;
  if (tokens <= 0 || top_k <= 0 || num_experts <= 0 || hidden <= 0 || inter <= 0) return 0;
  if ((int64_t)num_experts * (2 * inter + hidden) / 128 > kMaxCounters) return 0;
  return moe_plan(tokens, top_k, num_experts, hidden, inter).total;
}

extern "C" int exl3_moe_forward(const void* x, int x_bf16, int tokens, int hidden, const void* topk_ids,
                                const void* topk_weights, int top_k, int num_experts, int inter,
                                const exl3_moe_weights* w, int K, int codebook, void* y, int y_bf16, void* workspace,
                                size_t workspace_bytes, void* stream) {
  EXL3_CHECK_ARG(x && y && topk_ids && topk_weights && w, "exl3_moe_forward: null pointer");
  EXL3_CHECK_ARG(valid_bits(K) && valid_cb(codebook), "exl3_moe_forward: K = %d / codebook = %d", K, codebook);
  EXL3_CHECK_ARG(tokens >= 0 && top_k >= 1 && top_k <= 64, "exl3_moe_forward: tokens = %d, top_k = %d", tokens, top_k);
  EXL3_CHECK_ARG(num_experts >= 1 && num_experts <= 1024, "exl3_moe_forward: num_experts = %d (1..1024)", num_experts);
  EXL3_CHECK_ARG(hidden > 0 && hidden % 128 == 0 && inter > 0 && inter % 128 == 0,
                 "exl3_moe_forward: hidden = %d, inter = %d (multiples of 128)", hidden, inter);
  EXL3_CHECK_ARG(w->gate_trellis && w->up_trellis && w->down_trellis && w->gate_suh && w->gate_svh && w->up_suh &&
                     w->up_svh && w->down_suh && w->down_svh,
                 "exl3_moe_forward: null expert tensor");
  EXL3_CHECK_ARG((int64_t)hidden * inter * K / 8 <= INT32_MAX, "exl3_moe_forward: expert matrix too large");
  EXL3_CHECK_ARG((int64_t)num_experts * (2 * inter + hidden) / 128 <= kMaxCounters,
                 "exl3_moe_forward: %d experts x (2 x %d + %d) / 128 split counters exceed %d", num_experts, inter,
                 hidden, kMaxCounters);
  if (tokens == 0) return EXL3_OK;
  const int slots = tokens * top_k;
  EXL3_CHECK_ARG((int64_t)slots * std::max(2 * inter, hidden) <= INT32_MAX / 4, "exl3_moe_forward: too many slots");
  const MoePlan p = moe_plan(tokens, top_k, num_experts, hidden, inter);
  EXL3_CHECK_ARG(workspace && workspace_bytes >= p.total, "exl3_moe_forward: workspace %zu bytes, need %zu",
                 workspace_bytes, p.total);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  MoeArgs a{};
  a.tr[0] = static_cast<const uint32_t*>(w->gate_trellis);
  a.tr[1] = static_cast<const uint32_t*>(w->up_trellis);
  a.tr[2] = static_cast<const uint32_t*>(w->down_trellis);
  a.suh[0] = static_cast<const uint16_t*>(w->gate_suh);
  a.suh[1] = static_cast<const uint16_t*>(w->up_suh);
  a.suh[2] = static_cast<const uint16_t*>(w->down_suh);
  a.svh[0] = static_cast<const uint16_t*>(w->gate_svh);
  a.svh[1] = static_cast<const uint16_t*>(w->up_svh);
  a.svh[2] = static_cast<const uint16_t*>(w->down_svh);
  a.E = num_experts;
  a.H = hidden;
  a.I = inter;
  a.top_k = top_k;
  a.slots = slots;
  int* counts = reinterpret_cast<int*>(ws + p.off_counts);
  int* nactive = reinterpret_cast<int*>(ws + p.off_nactive);
  int* active = reinterpret_cast<int*>(ws + p.off_active);
  int* lists = reinterpret_cast<int*>(ws + p.off_lists);
  a.counts = counts;
  a.n_active = nactive;
  a.active = active;
  a.lists = lists;
  a.topk_ids = static_cast<const int*>(topk_ids);
  // a single token: its top-k slots run directly (no routing launch); several tokens share experts, so they are routed
  a.slot_mode = tokens == 1 && slots <= num_experts;
  uint16_t* gu = reinterpret_cast<uint16_t*>(ws + p.off_gu);
  uint16_t* dn = reinterpret_cast<uint16_t*>(ws + p.off_dn);
  int* cnt_gu = reinterpret_cast<int*>(ws + p.off_cnt_gu);
  int* cnt_dn = reinterpret_cast<int*>(ws + p.off_cnt_dn);
  float* partial = reinterpret_cast<float*>(ws + p.off_partial);
  hipStream_t st = as_stream(stream);

  if (!a.slot_mode) {
    moe_route_kernel<<<1, 1024, 0, st>>>(static_cast<const int*>(topk_ids), slots, num_experts, counts, nactive,
                                         active, lists);
    EXL3_CHECK_LAUNCH();
  }
  const int max_active = a.slot_mode ? slots : std::min(num_experts, slots);
  bool ok = EXL3_MOE_DISPATCH(K, codebook, {
    moe_gemv_kernel<kK, kCB, 0><<<dim3(2 * inter / 128, max_active, p.splits_gu), kMoeThreads, moe_lds_bytes<kK>(),
                                  st>>>(a, x, x_bf16, gu, dn, partial, cnt_gu, p.splits_gu);
    moe_gemv_kernel<kK, kCB, 1><<<dim3(hidden / 128, max_active, p.splits_dn), kMoeThreads, moe_lds_bytes<kK>(),
                                  st>>>(a, x, x_bf16, gu, dn, partial, cnt_dn, p.splits_dn);
  });
  if (!ok) return set_error(EXL3_ERR_INVALID, "exl3_moe_forward: unsupported K/codebook");
  EXL3_CHECK_LAUNCH();
  const dim3 cgrid((unsigned)(((size_t)tokens * (hidden / 128) + 7) / 8));
  if (y_bf16)
    moe_combine_kernel<true><<<cgrid, 256, 0, st>>>(dn, static_cast<const int*>(topk_ids),
                                                    static_cast<const float*>(topk_weights), tokens, top_k,
                                                    num_experts, hidden, y);
  else
    moe_combine_kernel<false><<<cgrid, 256, 0, st>>>(dn, static_cast<const int*>(topk_ids),
                                                     static_cast<const float*>(topk_weights), tokens, top_k,
                                                     num_experts, hidden, y);
  EXL3_CHECK_LAUNCH();
  return EXL3_OK;
}
