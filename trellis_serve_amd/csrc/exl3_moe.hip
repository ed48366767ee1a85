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
// Launches (the reference uses five plus an align launch):
//   single token (slot mode): moe_gemv_kernel<PHASE 0> -> moe_gemv_kernel<PHASE 1> -> moe_combine_kernel; grid row =
//                      slot, its expert read from topk_ids; the gate/up reducers write fp16 g|u rows and the down
//                      workgroups compute the GLU and the input rotations in their prologues.
//   several tokens: moe_route_prep_kernel -> moe_gemv_kernel<PHASE 0> -> moe_gemv_kernel<PHASE 1> ->
//                      moe_combine_kernel; grid row = active expert.
//   moe_route_prep_kernel  the rotated gate/up inputs fp16(Had(x[token] * suh)) per (slot, shard), written once
//                      (the reference's moe_had_in); its first workgroup routes: per-expert slot counts and lists (LDS
//                      atomics), the active experts in ascending order.  The order of slots inside an expert's list
//                      does not change any result: the rows of an MFMA are independent and the combine sums in slot
//                      order.
//   moe_gemv_kernel<PHASE 0>  grid (2I/128 column blocks, experts or slots, k-splits): gate/up of every active expert
//                      for all its slots on the dense GEMV's streaming core (TileStream); up to 16 P slots share each
//                      decoded tile (P 16-row MFMAs).  The gate and up blocks of the same 128 columns count on one
//                      counter; the last of their splits sums both, applies the output rotations * svh (fp16 g, u),
//                      then a = fp16(silu(g) * u) (fp32 SiLU), * suh_down and its rotation -- the down inputs of those
//                      128 positions (the reference's moe_glu_had_in launch, folded in).
//   moe_gemv_kernel<PHASE 1>  the same for down, staging the prepared down inputs; fp16 d rows.
//   moe_combine_kernel weighted fp32 sum over the token's slots.
#include <stdlib.h>

#include <algorithm>
#include <cmath>

#include "exl3_api.hpp"
#include "exl3_device.hpp"
#include "exl3_stream.hpp"

namespace exl3 {

constexpr int kMoeWaves = 8, kMoeThreads = kMoeWaves * 64;
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
  const int* topk_ids;     // [slots]: read directly in slot mode and by the route+prep launch
  int slot_mode;           // 1: one workgroup row per slot, no routing launch (a single token: its top-k experts);
                           // the kernels take it from their PRE = false instance
  // rotated activations written once per slot, each 128-block in the staging order of a_slot: gate/up inputs
  // [2][slots][H] (moe_route_prep_kernel) and down inputs [slots][I] (the gate/up reducer), both for several tokens
  const uint16_t* pre_in;
  const uint16_t* pre_dn;
  // mixed-K layers: the launch serves one class, whose weights hold its experts at local ids (emap: global id ->
  // local id, -1 for other classes' experts; null when one class holds every expert)
  const int* emap;
  int E_local;
};

// The weights' row of global expert e in the launch's class, or -1 when e is unrouted or belongs to another class.
// Counters, routing lists and slot rows stay indexed by global ids and slots.
__device__ __forceinline__ int moe_local(const MoeArgs& a, int e) {
  if (e < 0 || e >= a.E) return -1;
  if (a.emap == nullptr) return e;
  const int el = a.emap[e];
  return el < a.E_local ? el : -1;
}


// Activation buffers of the prepared-row chunk pipeline: two (chunk c + 1 staged while chunk c decodes) where the
// LDS does not set the occupancy, one at P = 2 (the next chunk's rows wait in registers until every wave is done with
// the buffer: one more barrier per chunk, 4 workgroups per CU instead of 3 -- T = 256 down 62.2 -> 57.7 us)
template <int P, bool PRE>
__host__ __device__ constexpr int moe_act_buffers() { return PRE && P != 2 ? 2 : 1; }

// LDS: staged activations [16 P rows][a_mstride(NT) halves] x moe_act_buffers, then per wave the stream stages.  P
// groups of 16 slots share each decoded tile pair.
template <int K, int P, int NT, bool PRE>
__host__ __device__ constexpr int moe_lds_bytes() {
  return moe_act_buffers<P, PRE>() * kMoeRows * P * a_mstride(NT) * 2 + kMoeWaves * stream_lds_bytes(K, PRE);
}

static_assert(moe_lds_bytes<8, 4, 16, true>() <= 160 * 1024, "MoE LDS must fit a CU");
constexpr int kMoeMaxTopK = 64;


// The rotated fp16 gate/up inputs fp16(Had(x[token] * suh)) at positions kk .. kk+3 (kk = 128 b + 4 t, lane t of a
// half-wave); one 128-block per half-wave (had128_x4 spans 32 lanes).
__device__ __forceinline__ void moe_in4(const MoeArgs& a, const void* x, int x_bf16, const uint16_t* suh, int slot,
                                        int kk, _Float16 h[4]) {
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
  float f[4];
  f[0] = (float)(_Float16)(v[0] * su.x); f[1] = (float)(_Float16)(v[1] * su.y);
  f[2] = (float)(_Float16)(v[2] * su.z); f[3] = (float)(_Float16)(v[3] * su.w);
  had128_x4(f[0], f[1], f[2], f[3]);
#pragma unroll
  for (int i = 0; i < 4; i++) h[i] = had_scale_f16(f[i]);
}

// The rotated down inputs at positions kk .. kk+3 from the fp16 g|u row of a slot: a = fp16(silu(g) * u) in fp32
// (exl3_marlin_moe.cu:228-258), * suh_down, rotated (single-token path: computed in the down workgroups' prologue)
__device__ __forceinline__ void moe_glu4(const MoeArgs& a, const uint16_t* gu, const uint16_t* suh, int slot, int kk,
                                         _Float16 h[4]) {
  const half4_t gv = *reinterpret_cast<const half4_t*>(gu + (size_t)slot * 2 * a.I + kk);
  const half4_t uv = *reinterpret_cast<const half4_t*>(gu + (size_t)slot * 2 * a.I + a.I + kk);
  const half4_t su = *reinterpret_cast<const half4_t*>(suh + kk);
  float f[4];
  f[0] = (float)(f16_of_f32(silu32((float)gv.x) * (float)uv.x) * su.x);
  f[1] = (float)(f16_of_f32(silu32((float)gv.y) * (float)uv.y) * su.y);
  f[2] = (float)(f16_of_f32(silu32((float)gv.z) * (float)uv.z) * su.z);
  f[3] = (float)(f16_of_f32(silu32((float)gv.w) * (float)uv.w) * su.w);
  had128_x4(f[0], f[1], f[2], f[3]);
#pragma unroll
  for (int i = 0; i < 4; i++) h[i] = had_scale_f16(f[i]);
}

// 4 fp16 values into a staging-order row at positions p .. p+3 (p = 4 t): positions 4t, 4t+1 and 4t+2, 4t+3 land on
// adjacent staging slots, two 4-byte stores
__device__ __forceinline__ void store_staged4(_Float16* row, int p, const _Float16 h[4]) {
  typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
  *reinterpret_cast<half2_t*>(row + a_slot(p, 0, 0)) = half2_t{h[0], h[1]};
  *reinterpret_cast<half2_t*>(row + a_slot(p + 2, 0, 0)) = half2_t{h[2], h[3]};
}

// Routing by one 256-thread workgroup: per-expert slot counts and lists (LDS atomics; ids outside [0, E) skipped),
// the active experts in ascending order (each thread scans 4 experts, then a workgroup scan of the 256 sums).
__device__ void moe_route_block(const int* __restrict__ topk_ids, int slots, int E, int* __restrict__ counts,
                                int* __restrict__ n_active, int* __restrict__ active, int* __restrict__ lists) {
  __shared__ int cnt[1024];
  __shared__ int part[256];
  const int tid = threadIdx.x;
  for (int e = tid; e < 1024; e += 256) cnt[e] = 0;
  __syncthreads();
  // up to 8 ids per thread loaded together (2048 slots at 256 tokens: one load round trip instead of 8 in a chain);
  // a slot's place in its expert's list follows the LDS atomics, and no result depends on it (every slot is its own
  // row of the expert GEMVs)
  for (int s0 = tid; s0 < slots; s0 += 256 * 8) {
    int ev[8];
#pragma unroll
    for (int i = 0; i < 8; i++) ev[i] = s0 + 256 * i < slots ? topk_ids[s0 + 256 * i] : -1;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int e = ev[i];
      if (e >= 0 && e < E) lists[(size_t)e * slots + atomicAdd(&cnt[e], 1)] = s0 + 256 * i;
    }
  }
  __syncthreads();
  bool f[4];
  int loc = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int e = 4 * tid + i;
    f[i] = e < E && cnt[e] > 0;
    loc += f[i];
  }
  part[tid] = loc;
  __syncthreads();
  for (int d = 1; d < 256; d <<= 1) {  // inclusive Hillis-Steele scan
    const int v = tid >= d ? part[tid - d] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int base = part[tid] - loc;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int e = 4 * tid + i;
    if (e < E) {
      counts[e] = cnt[e];
      if (f[i]) active[base++] = e;
    }
  }
  if (tid == 255) *n_active = part[255];
}

constexpr int kMoePrepUnits = 4;  // 128-blocks per half-wave in moe_route_prep_kernel

// moe_route_prep_kernel: workgroup 0 routes (when `route`: the first class's launch of a mixed layer); workgroups
// 1 .. gridDim.x - 1 write the rotated gate/up inputs of every routed slot of the launch's class, one half-wave per
// (slot, shard, 4 128-blocks) (rows of unrouted slots are left alone, never read).  One launch for both: neither needs
// the other.
__global__ __launch_bounds__(256) void moe_route_prep_kernel(MoeArgs a, const void* __restrict__ x, int x_bf16,
                                                             uint16_t* __restrict__ pre, int* __restrict__ counts,
                                                             int* __restrict__ n_active, int* __restrict__ active,
                                                             int* __restrict__ lists, int route) {
  if (blockIdx.x == 0) {  // dispatched first: the routing chain is the longest at few tokens
    if (route) moe_route_block(a.topk_ids, a.slots, a.E, counts, n_active, active, lists);
    return;
  }
  // kMoePrepUnits consecutive 128-blocks of one (slot, shard) row per half-wave: their loads go out together and the
  // rotations interleave (one block per half-wave was latency-bound: 13 us for 256 tokens)
  const int kblocks = a.H >> 7, groups = (kblocks + kMoePrepUnits - 1) / kMoePrepUnits;
  const int u = (blockIdx.x - 1) * 8 + (threadIdx.x >> 5);
  const int t = threadIdx.x & 31;
  const int rest = u / groups, b0 = (u - rest * groups) * kMoePrepUnits;
  if (rest >= a.slots * 2) return;
  const int sh = rest & 1, slot = rest >> 1;
  const int el = moe_local(a, a.topk_ids[slot]);
  if (el < 0) return;
  const uint16_t* suh = a.suh[sh] + (size_t)el * a.H;
  _Float16* row = reinterpret_cast<_Float16*>(pre) + ((size_t)sh * a.slots + slot) * a.H;
  _Float16 h[kMoePrepUnits][4];
#pragma unroll
  for (int i = 0; i < kMoePrepUnits; i++)
    if (b0 + i < kblocks) moe_in4(a, x, x_bf16, suh, slot, (b0 + i) * 128 + 4 * t, h[i]);
#pragma unroll
  for (int i = 0; i < kMoePrepUnits; i++)
    if (b0 + i < kblocks) store_staged4(row, (b0 + i) * 128 + 4 * t, h[i]);
}

// PRE: activations copied from prepared rows (gate/up with several tokens; down always); else the gate/up input
// rotation is computed here (slot mode, one row).
// The prepared-row kernels with P <= 2 and K <= 4 are held to 64 VGPRs (8 waves per SIMD): P = 1 fits without
// spilling, P = 2 spills 6-8 VGPRs that live across the pass loop (stored before it, reloaded after its chunk loop,
// none inside); the others take what they need (P = 4 and K >= 5: 80-130 VGPRs; P = 4 is held to one workgroup per CU
// by its LDS anyway).
template <int K, int CB, int PHASE, int P, bool PRE, int NT>
__global__ __launch_bounds__(kMoeThreads, (PRE && P <= 2 && K <= 4) ? 8 : 1) void moe_gemv_kernel(
    MoeArgs a, const void* __restrict__ x, int x_bf16, uint16_t* __restrict__ gu, uint16_t* __restrict__ pre_dn_out,
    uint16_t* __restrict__ dn, float* partial, int* counters, int splits, int chunks, int xl) {
  typedef TileStream<K, CB, NT, PRE> Stream;  // the prepared-row chunk pipeline needs every lane loading
  // issue priority as in the dense GEMV: the short latency-bound prologue and split-K chain above the decode loop
  __builtin_amdgcn_s_setprio(2);
  constexpr int NB = Stream::NB;
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ int last_flag;
  _Float16* xs = reinterpret_cast<_Float16*>(lds);
  constexpr int mstride = a_mstride(NT);

  // expert and its slots: routed mode -- grid row = active expert, its slot list from the routing launch; slot mode
  // -- grid row = slot, one slot, its expert read from topk_ids (split counters then index slots, so repeated experts
  // in one token are still right).  Slot mode is the launch without prepared rows (PRE = false), a compile-time
  // choice, so the single-token kernel has no routed-mode argument loads ahead of its expert id, and the empty asm
  // (taking the arguments as operands) puts every argument load into the round that fetches topk_ids.
  int e, el, n_e, ctr_row;  // global expert id, its weights' row in this launch's class
  const int* list;
  if constexpr (!PRE)
    asm volatile("" ::"s"(a.tr[0]), "s"(a.tr[1]), "s"(a.tr[2]), "s"(a.suh[0]), "s"(a.suh[1]), "s"(a.suh[2]),
                 "s"(a.svh[0]), "s"(a.svh[1]), "s"(a.svh[2]), "s"(a.E), "s"(a.H), "s"(a.I), "s"(a.top_k),
                 "s"(a.topk_ids), "s"(x), "s"(x_bf16), "s"(gu), "s"(dn), "s"(partial), "s"(counters), "s"(splits),
                 "s"(chunks), "s"(a.emap));
  if constexpr (!PRE) {
    e = a.topk_ids[blockIdx.y];
    el = moe_local(a, e);
    if (el < 0) return;
    n_e = 1;
    list = nullptr;
    ctr_row = blockIdx.y;
  } else {
    if ((int)blockIdx.y >= *a.n_active) return;
    e = a.active[blockIdx.y];
    el = moe_local(a, e);
    if (el < 0) return;
    n_e = a.counts[e];
    list = a.lists + (size_t)e * a.slots;
    ctr_row = e;
  }
  auto slot_at = [&](int idx) { return !PRE ? (int)blockIdx.y : list[idx]; };
  const int cb = blockIdx.x, sp = blockIdx.z;
  const int k = PHASE ? a.I : a.H;            // input width
  const int n_out = PHASE ? a.H : 2 * a.I;    // output row width (g|u for gate/up)
  const int sh = PHASE ? 2 : (cb < a.I / 128 ? 0 : 1);
  const int n_sh = PHASE ? a.H : a.I;         // output width of the shard
  const int cbl = PHASE ? cb : cb - (sh ? a.I / 128 : 0);  // column block inside the shard
  const int tn = n_sh / 16;
  const int mat_bytes = (k >> 4) * tn * 32 * K;
  const uint32_t* trellis = (sh == 0 ? a.tr[0] : sh == 1 ? a.tr[1] : a.tr[2]) + (size_t)el * (mat_bytes / 4);
  const uint16_t* suh = (sh == 0 ? a.suh[0] : sh == 1 ? a.suh[1] : a.suh[2]) + (size_t)el * k;
  const uint16_t* svh = (sh == 0 ? a.svh[0] : sh == 1 ? a.svh[1] : a.svh[2]) + (size_t)el * n_sh;
  const uint16_t* pre = PRE ? (PHASE ? a.pre_dn : a.pre_in + (size_t)sh * a.slots * k) : nullptr;
  // this split's k range: `chunks` chunks of NB 128-row blocks, from chunk sp * chunks (the last split may hold fewer)
  const int kblocks = k >> 7;

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, c = l & 15, j = l >> 4;
  const int hw = threadIdx.x >> 5, t = threadIdx.x & 31;
  constexpr int kActBufs = moe_act_buffers<P, PRE>();
  uint8_t* stage = lds + kActBufs * kMoeRows * P * mstride * 2 + w * Stream::LDS_BYTES;

  // passes of up to 16 P slots; each decoded tile feeds the pass's `groups` 16-row MFMAs
  __builtin_amdgcn_s_setprio(0);
  for (int c0 = 0; c0 < n_e; c0 += kMoeRows * P) {
    const int M = min(kMoeRows * P, n_e - c0);
    const int groups = (M + kMoeRows - 1) / kMoeRows;
    float4_t acc[P];
#pragma unroll
    for (int p = 0; p < P; p++) acc[p] = float4_t{0.f, 0.f, 0.f, 0.f};
    if constexpr (PRE) {
      // prepared rows, chunk after chunk, with the next chunk's rows and trellis blocks in flight while this one
      // decodes: two streams alternate, and two activation buffers (or, at P = 2, one buffer refilled after a
      // barrier from the rows held in registers); the loop carries no register copies, so the compiler's in-order
      // load waits stay exact.  Every load is unconditional -- a unit past the pass's rows or
      // the split's blocks reads out of the buffer's range and gets zeros, a prefetch past the split's last chunk
      // re-reads that chunk (in range, never used) -- and the slot rows' offsets are read once per pass, so no load
      // inside the loop waits on an older one.
      constexpr int IT = kMoeRows * P * NB / (2 * kMoeWaves);
      static_assert((2 * kMoeWaves) % NB == 0, "a half-wave keeps its block across its units");
      const int nch = min(chunks, (kblocks + NB - 1) / NB - sp * chunks);  // this split's chunks (>= 1)
      const uint32_t pre_bytes = (uint32_t)a.slots * (uint32_t)k * 2u;
      const __amdgpu_buffer_rsrc_t prs =
          __builtin_amdgcn_make_buffer_rsrc((void*)pre, (short)0, (int)pre_bytes, 0x00020000);
      const int ub = hw % NB;  // the half-wave's block inside a chunk (the same for all its units)
      uint32_t rowoff[IT];     // byte offset of each unit's slot row; pre_bytes (out of range) past the pass's rows
#pragma unroll
      for (int it = 0; it < IT; it++) {
        const int m = hw / NB + it * (2 * kMoeWaves / NB);
        rowoff[it] = m < M ? (uint32_t)slot_at(c0 + m) * (uint32_t)k * 2u : pre_bytes;
      }
      auto chunk_kb0 = [&](int ch) { return (sp * chunks + (ch < nch ? ch : nch - 1)) * NB; };
      auto load_a = [&](int ch, uint2_t (&v)[IT]) {
        const int kb0 = chunk_kb0(ch);
        const bool live = ub < min(kblocks, kb0 + NB) - kb0;
        const uint32_t col = (uint32_t)((kb0 + ub) * 128 + 4 * t) * 2u;
#pragma unroll
        for (int it = 0; it < IT; it++) {
          const uint32_t off = live && rowoff[it] < pre_bytes ? rowoff[it] + col : pre_bytes;
          v[it] = __builtin_bit_cast(uint2_t, __builtin_amdgcn_raw_buffer_load_b64(prs, off, 0, 0));
        }
      };
      // every row of the buffer is written (zeros past the pass's rows), so no store is conditional either
      auto store_a = [&](_Float16* dst, const uint2_t (&v)[IT]) {
#pragma unroll
        for (int it = 0; it < IT; it++) {
          const int m = hw / NB + it * (2 * kMoeWaves / NB);
          *reinterpret_cast<uint2_t*>(dst + m * mstride + ub * 128 + 4 * t) = v[it];
        }
      };
      auto start = [&](Stream& st, int ch) {
        const int kb0 = chunk_kb0(ch);
        st.init(trellis, mat_bytes, tn, cbl * kMoeWaves + w, kb0, min(kblocks, kb0 + NB) - kb0, stage, l);
        st.start();
      };
      _Float16* xs1 = kActBufs == 2 ? xs + kMoeRows * P * mstride : xs;
      // A row of lane group c in group p: 16 p + c (group 0: min(c, M - 1)); rows >= M feed only C rows never stored
      const half8_t* ap0 = reinterpret_cast<const half8_t*>(xs + min(c, M - 1) * mstride) + j;
      const half8_t* ap1 = reinterpret_cast<const half8_t*>(xs1 + min(c, M - 1) * mstride) + j;
      Stream s0, s1;
      uint2_t v[IT];
      load_a(0, v);
      start(s0, 0);
      store_a(xs, v);
      lds_barrier();
      // chunks in pairs, then an odd last one: the loop has no early exit, so every path into its head carries the
      // same loads in flight (stream 0's) and the compiler's load waits inside stay exact
      int ch = 0;
      for (; ch + 2 <= nch; ch += 2) {
        load_a(ch + 1, v);
        start(s1, ch + 1);
        s0.template run_groups<P>(ap0, kMoeRows * mstride / 8, groups, acc);
        if constexpr (kActBufs == 1) lds_barrier();  // one buffer: every wave is done with chunk ch
        store_a(xs1, v);
        lds_barrier();  // chunk ch + 1 staged; every wave is done with buffer 0
        load_a(ch + 2, v);
        start(s0, ch + 2);
        s1.template run_groups<P>(ap1, kMoeRows * mstride / 8, groups, acc);
        if constexpr (kActBufs == 1) lds_barrier();
        store_a(xs, v);
        lds_barrier();
      }
      if (ch < nch) {  // the odd last chunk: staged in buffer 0, its blocks in stream 0
        s0.template run_groups<P>(ap0, kMoeRows * mstride / 8, groups, acc);
        lds_barrier();
      }
    } else {
      for (int ch = 0; ch < chunks; ch++) {
        const int kb0 = (sp * chunks + ch) * NB;
        if (kb0 >= kblocks) break;
        const int nb = min(kblocks, kb0 + NB) - kb0;
        Stream stream;
        stream.init(trellis, mat_bytes, tn, cbl * kMoeWaves + w, kb0, nb, stage, l);
        stream.start();
        for (int u = hw; u < M * NB; u += 2 * kMoeWaves) {
          const int m = u / NB, b = u - m * NB;
          _Float16 h[4] = {0, 0, 0, 0};
          if (b < nb) {
            if constexpr (PHASE == 0)
              moe_in4(a, x, x_bf16, suh, slot_at(c0 + m), (kb0 + b) * 128 + 4 * t, h);
            else
              moe_glu4(a, gu, suh, slot_at(c0 + m), (kb0 + b) * 128 + 4 * t, h);
          }
          // a_slot keeps each even-odd pair of positions adjacent: two 4-byte writes
          *reinterpret_cast<half2_t*>(xs + a_slot(b * 128 + 4 * t, m, mstride)) = half2_t{h[0], h[1]};
          *reinterpret_cast<half2_t*>(xs + a_slot(b * 128 + 4 * t + 2, m, mstride)) = half2_t{h[2], h[3]};
        }
        __syncthreads();
        // A row of lane group c in group p: 16 p + c (group 0: min(c, M - 1)); rows >= M feed only C rows never stored
        stream.template run_groups<P>(reinterpret_cast<const half8_t*>(xs + min(c, M - 1) * mstride) + j,
                                      kMoeRows * mstride / 8, groups, acc);
        __syncthreads();  // the next chunk or pass restages LDS
      }
    }
    // this split's partial rows: device-coherent (read by the last split, possibly on another XCD), or, with xl
    // (the host found every split of this counter on one XCD: workgroup ids that agree mod 8, and a probe that saw
    // such ids on one XCD), plain stores into that XCD's L2
    float* pdst = partial + (size_t)sp * a.slots * n_out + cb * 128 + w * 16 + c;
#pragma unroll
    for (int p = 0; p < P; p++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = kMoeRows * p + 4 * j + r;
        if (m < M) {
          if (xl)
            __hip_atomic_store(pdst + (size_t)slot_at(c0 + m) * n_out, acc[p][r], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
          else
            __hip_atomic_store(pdst + (size_t)slot_at(c0 + m) * n_out, acc[p][r], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
      }
  }
  __builtin_amdgcn_s_setprio(2);
  // arrivals: the k-splits of this column block; gate/up with several tokens (GLU) -- the k-splits of the gate block
  // and of the up block of the same 128 columns, on one counter
  constexpr bool GLU = PHASE == 0 && PRE;
  const int ctr = GLU ? ctr_row * (a.I / 128) + cbl : ctr_row * (n_out / 128) + cb;
  const int arrivals = GLU ? 2 * splits : splits;
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = xl ? __hip_atomic_fetch_add(&counters[ctr], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                        : __hip_atomic_fetch_add(&counters[ctr], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev == arrivals - 1;
  }
  __syncthreads();
  if (!last_flag) return;

  // last arrival: every slot's 128 columns (one slot per half-wave, 4 columns per lane), splits summed in order, one
  // rounding, output rotation * svh
  // the splits' loads go out 4 at a time (8-byte device-scope loads; a split past the end reads split 0 again and
  // adds nothing), then are summed in split order
  auto finish = [&](int slot, int pcol, const uint16_t* svh4, _Float16 o[4]) {
    float4_t s4 = {0.f, 0.f, 0.f, 0.f};
    for (int p0 = 0; p0 < splits; p0 += 4) {
      float4_t v[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int pp = p0 + i < splits ? p0 + i : 0;
        const uint64_t* src =
            reinterpret_cast<const uint64_t*>(partial + ((size_t)pp * a.slots + slot) * n_out + pcol);
        // (xl: this CU never read these lines before in this launch, and the L1 starts each launch empty, so the
        // L2's copy is what a plain load returns)
        const uint64_t lo = xl ? __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                               : __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t hi = xl ? __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                               : __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        v[i] = float4_t{__builtin_bit_cast(float, (uint32_t)lo), __builtin_bit_cast(float, (uint32_t)(lo >> 32)),
                        __builtin_bit_cast(float, (uint32_t)hi), __builtin_bit_cast(float, (uint32_t)(hi >> 32))};
      }
#pragma unroll
      for (int i = 0; i < 4; i++)
        if (p0 + i < splits) s4 += v[i];
    }
    const _Float16 h[4] = {(_Float16)s4.x, (_Float16)s4.y, (_Float16)s4.z, (_Float16)s4.w};
    float f0 = (float)h[0], f1 = (float)h[1], f2 = (float)h[2], f3 = (float)h[3];
    had128_x4(f0, f1, f2, f3);
    const half4_t sv = *reinterpret_cast<const half4_t*>(svh4);
    o[0] = (_Float16)(had_scale_f16(f0) * sv.x);
    o[1] = (_Float16)(had_scale_f16(f1) * sv.y);
    o[2] = (_Float16)(had_scale_f16(f2) * sv.z);
    o[3] = (_Float16)(had_scale_f16(f3) * sv.w);
  };
  if constexpr (GLU) {
    // g and u of positions kk .. kk+3 of the intermediate, then a = fp16(silu(g) * u) * suh_down rotated: the down
    // inputs of those positions (exl3_marlin_moe.cu:228-258)
    const int kk = cbl * 128 + 4 * t;
    const uint16_t* svg = a.svh[0] + (size_t)el * a.I + kk;
    const uint16_t* svu = a.svh[1] + (size_t)el * a.I + kk;
    const half4_t su = *reinterpret_cast<const half4_t*>(a.suh[2] + (size_t)el * a.I + kk);
    for (int m = hw; m < n_e; m += 2 * kMoeWaves) {
      const int slot = slot_at(m);
      _Float16 g[4], u[4];
      finish(slot, kk, svg, g);
      finish(slot, a.I + kk, svu, u);
      float f[4];
      f[0] = (float)(f16_of_f32(silu32((float)g[0]) * (float)u[0]) * su.x);
      f[1] = (float)(f16_of_f32(silu32((float)g[1]) * (float)u[1]) * su.y);
      f[2] = (float)(f16_of_f32(silu32((float)g[2]) * (float)u[2]) * su.z);
      f[3] = (float)(f16_of_f32(silu32((float)g[3]) * (float)u[3]) * su.w);
      had128_x4(f[0], f[1], f[2], f[3]);
      _Float16 h[4];
#pragma unroll
      for (int i = 0; i < 4; i++) h[i] = had_scale_f16(f[i]);
      store_staged4(reinterpret_cast<_Float16*>(pre_dn_out) + (size_t)slot * a.I, kk, h);
    }
  } else {
    // fp16 rows: d (down), or g|u (gate/up of a single token: the down prologue applies the GLU, spread over its
    // workgroups, instead of one half-wave per column block here)
    uint16_t* out = PHASE ? dn : gu;
    const int col = cb * 128 + 4 * t;
    for (int m = hw; m < n_e; m += 2 * kMoeWaves) {
      const int slot = slot_at(m);
      _Float16 o[4];
      finish(slot, col, svh + cbl * 128 + 4 * t, o);
      *reinterpret_cast<half4_t*>(out + (size_t)slot * n_out + col) = half4_t{o[0], o[1], o[2], o[3]};
    }
  }
  if (threadIdx.x == 0) {
    if (xl)
      __hip_atomic_store(&counters[ctr], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else
      __hip_atomic_store(&counters[ctr], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <bool Y_BF16>
__global__ __launch_bounds__(256) void moe_combine_kernel(const uint16_t* __restrict__ dn,
                                                          const int* __restrict__ topk_ids,
                                                          const float* __restrict__ topk_w, int tokens, int top_k,
                                                          int E, int H, void* __restrict__ y) {
  constexpr int kChunk = 8;
  const int nb = H >> 7;
  const int unit = blockIdx.x * 8 + (threadIdx.x >> 5);
  if (unit >= tokens * nb) return;
  const int t = threadIdx.x & 31;
  const int tok = unit / nb, b = unit - tok * nb;
  const int col = b * 128 + 4 * t;
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int j0 = 0; j0 < top_k; j0 += kChunk) {
    bool use[kChunk];
    float wgt[kChunk];
    half4_t v[kChunk];
#pragma unroll
    for (int i = 0; i < kChunk; i++) {
      const int slot = tok * top_k + min(j0 + i, top_k - 1);
      const int e = topk_ids[slot];
      use[i] = j0 + i < top_k && e >= 0 && e < E;
      wgt[i] = topk_w[slot];
      v[i] = *reinterpret_cast<const half4_t*>(dn + (size_t)slot * H + col);  // in bounds; unused unless use[i]
    }
#pragma unroll
    for (int i = 0; i < kChunk; i++) {
      if (use[i]) {
        acc.x = __builtin_fmaf(wgt[i], (float)v[i].x, acc.x);
        acc.y = __builtin_fmaf(wgt[i], (float)v[i].y, acc.y);
        acc.z = __builtin_fmaf(wgt[i], (float)v[i].z, acc.z);
        acc.w = __builtin_fmaf(wgt[i], (float)v[i].w, acc.w);
      }
    }
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

// k-split plan of one expert GEMV phase: a chunk is NB = NT/8 blocks of 128 input rows; the C chunks of k are
// dealt to `splits` workgroups of `chunks` consecutive chunks each.  The split count is the smallest that gives about
// 2048 working workgroups (more splits only add per-workgroup fixed costs and partials: measured at 1, 16 and 256
// tokens), and at most what keeps the fp32 partials (written and read once per slot, output column and split)
// within a quarter of the expert weight bytes streamed.  rows: grid rows that do work (active experts, or slots).
struct MoePhase {
  int splits, chunks;
};

static MoePhase moe_phase_plan(int slots, int rows, int nblk, int k, int K, int nt) {
  const int NB = nt / 8;
  const int C = (k / 128 + NB - 1) / NB;
  const double per_split = (double)slots * 8.0 / ((double)rows * k * std::max(K, 1) / 8.0);
  const int cap = std::max(1, (int)(0.25 / per_split));
  static const int target = [] {  // EXL3_MOE_TARGET_WGS: another workgroup target (A/B measurements)
    const char* e = getenv("EXL3_MOE_TARGET_WGS");
    return e ? std::max(1, atoi(e)) : 2048;
  }();
  const int want = std::max(1, (target + rows * nblk - 1) / (rows * nblk));
  const int s = std::min(C, std::min(cap, want));
  MoePhase ph{};
  ph.chunks = (C + s - 1) / s;
  ph.splits = (C + ph.chunks - 1) / ph.chunks;
  return ph;
}

struct MoePlan {
  bool slot_mode;  // a single token: grid rows = its slots, no routing or prep launches
  int groups;      // P: 16-slot groups per pass over an expert's weights (1, 2 or 4)
  int nt;          // tile rows per chunk
  MoePhase gu, dn;
  size_t off_counts, off_nactive, off_active, off_lists, off_gu, off_dn, off_cnt_gu, off_cnt_dn, off_pre_in,
      off_pre_dn, off_partial, total;
};

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static MoePlan moe_plan(int tokens, int top_k, int E, int H, int I, int K_gu, int K_dn) {
  MoePlan p{};
  const int slots = tokens * top_k;
  p.slot_mode = tokens == 1 && slots <= E;
  const int rows = p.slot_mode ? slots : std::max(1, std::min(E, slots));
  p.nt = 16;  // 32 measured slower with 256 tokens, equal with 16
  p.gu = moe_phase_plan(slots, rows, 2 * I / 128, H, K_gu, p.nt);
  p.dn = moe_phase_plan(slots, rows, H / 128, I, K_dn, p.nt);
  // enough groups that an expert with a typical-to-high slot count (mean + ~2.5 sd of a binomial count) is one pass
  const double mean = (double)slots / rows;
  const double high = mean + 2.5 * std::sqrt(mean);
  p.groups = p.slot_mode || high <= 16 ? 1 : high <= 32 ? 2 : 4;
  // the split counters first, in the fixed counter region (zero between calls whatever the shapes)
  // gate/up counters: per (expert, 128-column block of I) shared by gate and up, or per (slot, block of g|u)
  p.off_cnt_gu = 0;
  p.off_cnt_dn = (size_t)E * (2 * I / 128) * 4;
  size_t o = kCounterBytes;
  p.off_counts = o; o = align256(o + (size_t)E * 4);
  p.off_nactive = o; o = align256(o + 4);
  p.off_active = o; o = align256(o + (size_t)E * 4);
  p.off_lists = o; o = align256(o + (size_t)E * slots * 4);
  p.off_gu = o; o = align256(o + (p.slot_mode ? (size_t)slots * 2 * I * 2 : 0));
  p.off_dn = o; o = align256(o + (size_t)slots * H * 2);
  p.off_pre_in = o; o = align256(o + (p.slot_mode ? 0 : (size_t)2 * slots * H * 2));
  p.off_pre_dn = o; o = align256(o + (p.slot_mode ? 0 : (size_t)slots * I * 2));
  p.off_partial = o;
  o = align256(o + std::max((size_t)p.gu.splits * slots * 2 * I, (size_t)p.dn.splits * slots * H) * 4);
  p.total = o;
  return p;
}

template <int K, int CB, int PHASE>
static void launch_moe_gemv(const MoePlan& p, const MoePhase& ph, dim3 grid, const MoeArgs& a, const void* x,
                            int x_bf16, uint16_t* gu, uint16_t* pre_dn, uint16_t* dn, float* partial, int* counters,
                            hipStream_t st) {
  const dim3 g3(grid.x, grid.y, ph.splits);
  // a counter's splits have workgroup ids grid.x * grid.y apart; gate/up with prepared rows (the GLU launch) also
  // counts the up block I / 128 column blocks after the gate block on the same counter
  const bool glu = PHASE == 0 && !p.slot_mode;
  const int xl = xcd_groups_ok() && (grid.x * grid.y) % 8 == 0 && !(glu && (a.I / 128) % 8 != 0) ? 1 : 0;
#define EXL3_MOE_GEMV(P_, PRE_)                                                                              \
  moe_gemv_kernel<K, CB, PHASE, P_, PRE_, 16><<<g3, kMoeThreads, moe_lds_bytes<K, P_, 16, PRE_>(), st>>>(    \
      a, x, x_bf16, gu, pre_dn, dn, partial, counters, ph.splits, ph.chunks, xl)
  if (p.slot_mode)
    EXL3_MOE_GEMV(1, false);
  else if (p.groups == 4)
    EXL3_MOE_GEMV(4, true);
  else if (p.groups == 2)
    EXL3_MOE_GEMV(2, true);
  else
    EXL3_MOE_GEMV(1, true);
#undef EXL3_MOE_GEMV
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

// One K class of a layer as the launches take it: its weight stacks (local expert order), expert map and bitrates.
struct MoeClass {
  const exl3_moe_weights* w;
  const int* emap;  // null: a single class holding every expert at its global id
  int E_local, K_gu, K_dn;
};

// The classes share one plan: its k-splits come from the smallest bitrates (the partial-size cap is tightest there).
static MoePlan moe_plan_of(int tokens, int top_k, int E, int H, int I, const MoeClass* cls, int ncls) {
  int K_gu = cls[0].K_gu, K_dn = cls[0].K_dn;
  for (int c = 1; c < ncls; c++) {
    K_gu = std::min(K_gu, cls[c].K_gu);
    K_dn = std::min(K_dn, cls[c].K_dn);
  }
  return moe_plan(tokens, top_k, E, H, I, K_gu, K_dn);
}

static bool moe_shape_ok(int tokens, int top_k, int E, int H, int I) {
  return tokens > 0 && top_k > 0 && E > 0 && H > 0 && I > 0 && (int64_t)E * (2 * I + H) / 128 <= kMaxCounters;
}

static int moe_forward_impl(const char* what, const void* x, int x_bf16, int tokens, int hidden, const void* topk_ids,
                            const void* topk_weights, int top_k, int num_experts, int inter, const MoeClass* cls,
                            int ncls, int codebook, void* y, int y_bf16, void* workspace, size_t workspace_bytes,
                            hipStream_t st) {
  EXL3_CHECK_ARG(tokens == 0 || (x && y && topk_ids && topk_weights), "%s: null pointer", what);
  EXL3_CHECK_ARG(valid_cb(codebook), "%s: codebook = %d", what, codebook);
  EXL3_CHECK_ARG(tokens >= 0 && top_k >= 1 && top_k <= kMoeMaxTopK, "%s: tokens = %d, top_k = %d", what, tokens,
                 top_k);
  EXL3_CHECK_ARG(num_experts >= 1 && num_experts <= 1024, "%s: num_experts = %d (1..1024)", what, num_experts);
  EXL3_CHECK_ARG(hidden > 0 && hidden % 128 == 0 && inter > 0 && inter % 128 == 0,
                 "%s: hidden = %d, inter = %d (multiples of 128)", what, hidden, inter);
  for (int c = 0; c < ncls; c++) {
    const exl3_moe_weights* w = cls[c].w;
    EXL3_CHECK_ARG(w && w->gate_trellis && w->up_trellis && w->down_trellis && w->gate_suh && w->gate_svh &&
                       w->up_suh && w->up_svh && w->down_suh && w->down_svh,
                   "%s: class %d: null expert tensor", what, c);
    EXL3_CHECK_ARG(valid_bits(cls[c].K_gu) && valid_bits(cls[c].K_dn), "%s: class %d: K gate/up = %d, K down = %d",
                   what, c, cls[c].K_gu, cls[c].K_dn);
    EXL3_CHECK_ARG(cls[c].E_local >= 1 && cls[c].E_local <= num_experts, "%s: class %d holds %d experts of %d", what,
                   c, cls[c].E_local, num_experts);
    EXL3_CHECK_ARG(ncls == 1 || cls[c].emap, "%s: class %d of a mixed layer has no expert map", what, c);
    EXL3_CHECK_ARG((int64_t)hidden * inter * std::max(cls[c].K_gu, cls[c].K_dn) / 8 <= INT32_MAX,
                   "%s: expert matrix too large", what);
  }
  EXL3_CHECK_ARG((int64_t)num_experts * (2 * inter + hidden) / 128 <= kMaxCounters,
                 "%s: %d experts x (2 x %d + %d) / 128 split counters exceed %d", what, num_experts, inter, hidden,
                 kMaxCounters);
  if (tokens == 0) return EXL3_OK;
  const int slots = tokens * top_k;
  EXL3_CHECK_ARG((int64_t)slots * std::max(2 * inter, hidden) <= INT32_MAX / 4, "%s: too many slots", what);
  const MoePlan p = moe_plan_of(tokens, top_k, num_experts, hidden, inter, cls, ncls);
  EXL3_CHECK_ARG(workspace && workspace_bytes >= p.total, "%s: workspace %zu bytes, need %zu", what, workspace_bytes,
                 p.total);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  MoeArgs a{};
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
  a.slot_mode = p.slot_mode;
  uint16_t* gu = reinterpret_cast<uint16_t*>(ws + p.off_gu);
  uint16_t* dn = reinterpret_cast<uint16_t*>(ws + p.off_dn);
  int* cnt_gu = reinterpret_cast<int*>(ws + p.off_cnt_gu);
  int* cnt_dn = reinterpret_cast<int*>(ws + p.off_cnt_dn);
  uint16_t* pre_in = reinterpret_cast<uint16_t*>(ws + p.off_pre_in);
  uint16_t* pre_dn = reinterpret_cast<uint16_t*>(ws + p.off_pre_dn);
  float* partial = reinterpret_cast<float*>(ws + p.off_partial);
  a.pre_in = pre_in;
  a.pre_dn = pre_dn;
  // the class's view of the arguments: its weight stacks and expert map
  auto for_class = [&](int c) {
    MoeArgs ac = a;
    const exl3_moe_weights* w = cls[c].w;
    ac.tr[0] = static_cast<const uint32_t*>(w->gate_trellis);
    ac.tr[1] = static_cast<const uint32_t*>(w->up_trellis);
    ac.tr[2] = static_cast<const uint32_t*>(w->down_trellis);
    ac.suh[0] = static_cast<const uint16_t*>(w->gate_suh);
    ac.suh[1] = static_cast<const uint16_t*>(w->up_suh);
    ac.suh[2] = static_cast<const uint16_t*>(w->down_suh);
    ac.svh[0] = static_cast<const uint16_t*>(w->gate_svh);
    ac.svh[1] = static_cast<const uint16_t*>(w->up_svh);
    ac.svh[2] = static_cast<const uint16_t*>(w->down_svh);
    ac.emap = cls[c].emap;
    ac.E_local = cls[c].E_local;
    return ac;
  };

  if (!a.slot_mode) {  // routing (once) and each class's rotated gate/up inputs
    const unsigned prep_wgs =
        (unsigned)(((size_t)slots * 2 * ((hidden / 128 + kMoePrepUnits - 1) / kMoePrepUnits) + 7) / 8);
    for (int c = 0; c < ncls; c++) {
      moe_route_prep_kernel<<<prep_wgs + 1, 256, 0, st>>>(for_class(c), x, x_bf16, pre_in, counts, nactive, active,
                                                           lists, c == 0);
      EXL3_CHECK_LAUNCH();
    }
  }
  const int rows = a.slot_mode ? slots : std::min(num_experts, slots);
  // gate/up of every class (the GLU of each column block folded into its last arrival), then down of every class;
  // gate/up and down run at their own bitrates (a checkpoint may store down at another K than gate and up)
  for (int c = 0; c < ncls; c++) {
    const MoeArgs ac = for_class(c);
    const bool ok = EXL3_MOE_DISPATCH(cls[c].K_gu, codebook, {
      launch_moe_gemv<kK, kCB, 0>(p, p.gu, dim3(2 * inter / 128, rows), ac, x, x_bf16, gu, pre_dn, dn, partial,
                                  cnt_gu, st);
    });
    if (!ok) return set_error(EXL3_ERR_INVALID, "%s: unsupported K/codebook", what);
    EXL3_CHECK_LAUNCH();
  }
  for (int c = 0; c < ncls; c++) {
    const MoeArgs ac = for_class(c);
    const bool ok = EXL3_MOE_DISPATCH(cls[c].K_dn, codebook, {
      launch_moe_gemv<kK, kCB, 1>(p, p.dn, dim3(hidden / 128, rows), ac, x, x_bf16, gu, pre_dn, dn, partial, cnt_dn,
                                  st);
    });
    if (!ok) return set_error(EXL3_ERR_INVALID, "%s: unsupported K/codebook", what);
    EXL3_CHECK_LAUNCH();
  }
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

}  // namespace exl3

using namespace exl3;

extern "C" size_t exl3_moe_workspace_bytes(int tokens, int top_k, int num_experts, int hidden, int inter,
                                           int K_gate_up, int K_down) {
  if (!moe_shape_ok(tokens, top_k, num_experts, hidden, inter)) return 0;
  return moe_plan(tokens, top_k, num_experts, hidden, inter, K_gate_up, K_down).total;
}

extern "C" size_t exl3_moe_classes_workspace_bytes(int tokens, int top_k, int num_experts, int hidden, int inter,
                                                   int nclasses, const exl3_moe_class* classes_host) {
  if (!moe_shape_ok(tokens, top_k, num_experts, hidden, inter) || !classes_host || nclasses < 1 ||
      nclasses > EXL3_MOE_MAX_CLASSES)
    return 0;
  MoeClass cls[EXL3_MOE_MAX_CLASSES];
  for (int c = 0; c < nclasses; c++)
    cls[c] = MoeClass{nullptr, nullptr, 0, classes_host[c].K_gate_up, classes_host[c].K_down};
  return moe_plan_of(tokens, top_k, num_experts, hidden, inter, cls, nclasses).total;
}

extern "C" int exl3_moe_forward(const void* x, int x_bf16, int tokens, int hidden, const void* topk_ids,
                                const void* topk_weights, int top_k, int num_experts, int inter,
                                const exl3_moe_weights* w, int K_gate_up, int K_down, int codebook, void* y,
                                int y_bf16, void* workspace, size_t workspace_bytes, void* stream) {
  const MoeClass one{w, nullptr, num_experts, K_gate_up, K_down};
  return moe_forward_impl("exl3_moe_forward", x, x_bf16, tokens, hidden, topk_ids, topk_weights, top_k, num_experts,
                          inter, &one, 1, codebook, y, y_bf16, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int exl3_moe_forward_classes(const void* x, int x_bf16, int tokens, int hidden, const void* topk_ids,
                                        const void* topk_weights, int top_k, int num_experts, int inter,
                                        const exl3_moe_class* classes_host, int nclasses, int codebook, void* y,
                                        int y_bf16, void* workspace, size_t workspace_bytes, void* stream) {
  EXL3_CHECK_ARG(classes_host && nclasses >= 1 && nclasses <= EXL3_MOE_MAX_CLASSES,
                 "exl3_moe_forward_classes: nclasses = %d (1..%d)", nclasses, EXL3_MOE_MAX_CLASSES);
  MoeClass cls[EXL3_MOE_MAX_CLASSES];
  for (int c = 0; c < nclasses; c++) {
    const exl3_moe_class& h = classes_host[c];
    cls[c] = MoeClass{&h.weights, h.expert_map, h.num_local, h.K_gate_up, h.K_down};
  }
  return moe_forward_impl("exl3_moe_forward_classes", x, x_bf16, tokens, hidden, topk_ids, topk_weights, top_k,
                          num_experts, inter, cls, nclasses, codebook, y, y_bf16, workspace, workspace_bytes,
                          as_stream(stream));
}

extern "C" int exl3_moe_combine(const void* yd, const float* topk_weights, const int* topk_ids, int tokens, int top_k,
                                int hidden, int num_experts, void* y, int y_bf16, void* stream) {
  EXL3_CHECK_ARG(tokens == 0 || (yd && topk_weights && topk_ids && y), "exl3_moe_combine: null pointer");
  EXL3_CHECK_ARG(tokens >= 0 && top_k >= 1 && hidden > 0 && hidden % 128 == 0 && num_experts >= 1,
                 "exl3_moe_combine: tokens = %d, top_k = %d, hidden = %d, num_experts = %d", tokens, top_k, hidden,
                 num_experts);
  EXL3_CHECK_ARG((int64_t)tokens * top_k * hidden <= INT32_MAX, "exl3_moe_combine: too many rows");
  if (tokens == 0) return EXL3_OK;
  const dim3 grid((unsigned)(((size_t)tokens * (hidden / 128) + 7) / 8));
  hipStream_t st = as_stream(stream);
  if (y_bf16)
    moe_combine_kernel<true><<<grid, 256, 0, st>>>(static_cast<const uint16_t*>(yd), topk_ids, topk_weights, tokens,
                                                   top_k, num_experts, hidden, y);
  else
    moe_combine_kernel<false><<<grid, 256, 0, st>>>(static_cast<const uint16_t*>(yd), topk_ids, topk_weights, tokens,
                                                    top_k, num_experts, hidden, y);
  EXL3_CHECK_LAUNCH();
  return EXL3_OK;
}
