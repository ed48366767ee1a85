// Paged quantized-KV decode attention on gfx950 (one query token per sequence, GQA).
//
// Cache layout (this build's; the reference has no quantized-KV decode kernel -- its nearest relative is the paged
// fp8 gather + blockwise attention with log-sum-exp merge of xpu/exl3xpu/fp8kv_prefill.py:73-117):
//   k_cache, v_cache: 8-bit int8 [pages][Hkv][16][D], or 4-bit packed uint8 [pages][Hkv][16][D/2] (element 2i in
//                     the low nibble, 2i+1 in the high nibble, two's complement);
//   k_scale, v_scale: fp16 [pages][Hkv]; value = code * scale;
//   page_table int32 [B][max_pages]; seq_lens int32 [B]; q fp16 [B][Hq][D]; out fp16 [B][Hq][D]; D = 128.
//   Query head h reads KV head h / (Hq / Hkv).
//
// kv_decode_kernel: grid (chunks of chunk_pages pages, Hkv, B), W = 8 (or 4) waves.  Wave w takes pages w, w+W, ...
// of its workgroup's chunk, with the next page's codes in flight while it works on the current one, and keeps an
// online softmax for the G = Hq/Hkv query heads (G <= 16; MFMA columns G..15 are idle).  Per 16-token page --
// exactly one 16-wide MFMA block, so the page's two scales are wave-uniform:
//   S^T = K Q^T     4 x MFMA 16x16x32 f16.  A = the page's 16 keys (lane: key l%16, 32 dims), B = Q^T (lane: query
//                   l%16, the same 32 dims in the same order; loaded once).  C lane: query l%16, keys 4(l/16)..+3;
//   P^T             that C layout is already the B operand of the next MFMA; P' = p * v_scale rounded to fp16;
//   O^T += V^T P^T  8 x MFMA 16x16x16 f16.  A = V^T (lane: dim 8(l%16) + db for block db, keys 4(l/16)..+3): the
//                   lane loads 8 bytes of each of its 4 keys and transposes the 4 x 4 byte blocks with v_perm.
//                   C lane: dims 32(l/16) .. +31 of query l%16 over the 8 blocks.
// Codes become fp16 without conversions: code + bias (bias 128 / 8, one xor) as the low byte (nibble) under 0x64 is
// the fp16 1024 + bias + code.  V: one packed fp16 subtract of 1024 + bias leaves the code exactly (integers of
// magnitude <= 128 are exact in fp16) before it is accumulated.  K: the MFMA takes the biased codes and the page's
// logits subtract (1024 + bias) * sum(q) -- a per-page correction, never accumulated across pages.  The W waves
// merge their (m, l, O) in LDS; the workgroup writes its chunk's partial state and kv_merge_kernel combines the
// chunks by log-sum-exp, in chunk order (deterministic).  Logits are kept in the base-2 domain (scale * log2 e).
#include <math.h>
#include <stdint.h>

#include <algorithm>
#include <cstdlib>

#include "exl3_api.hpp"
#include "exl3_device.hpp"

namespace exl3 {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef uint32_t kv_u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t kv_u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kKvWaves = 8;     // waves per decode workgroup (4 when the LDS merge of 8 would not fit 64 KB)
constexpr int kMergeWaves = 4;  // waves per kv_merge_kernel workgroup
constexpr int kHeadDim = 128;
constexpr int kPage = 16;
constexpr int kMaxGroup = 16;

// 4 biased code bytes -> 4 fp16 (1024 + byte - sub); the fp16 subtract is exact for the code range
__device__ __forceinline__ half4_t codes_f16(uint32_t u, _Float16 sub) {
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x05010400u);  // bytes: u0, 0x64, u1, 0x64
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x05030402u);  // bytes: u2, 0x64, u3, 0x64
  return __builtin_bit_cast(half4_t, kv_u32x2_t{lo, hi}) - half4_t{sub, sub, sub, sub};
}

// 4 x 4 byte transpose: in[i] holds bytes 0..3 of row i; out[j] holds byte j of rows 0..3 (row order)
__device__ __forceinline__ void transpose4x4(const uint32_t in[4], uint32_t out[4]) {
  const uint32_t a = __builtin_amdgcn_perm(in[1], in[0], 0x05010400u);  // r0b0 r1b0 r0b1 r1b1
  const uint32_t b = __builtin_amdgcn_perm(in[3], in[2], 0x05010400u);  // r2b0 r3b0 r2b1 r3b1
  const uint32_t c = __builtin_amdgcn_perm(in[1], in[0], 0x07030602u);  // r0b2 r1b2 r0b3 r1b3
  const uint32_t d = __builtin_amdgcn_perm(in[3], in[2], 0x07030602u);  // r2b2 r3b2 r2b3 r3b3
  out[0] = __builtin_amdgcn_perm(b, a, 0x05040100u);
  out[1] = __builtin_amdgcn_perm(b, a, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(d, c, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(d, c, 0x07060302u);
}

// reductions over the 4 lanes l, l^16, l^32, l^48 (the 16 keys of a page for one query): v_permlane16_swap and
// v_permlane32_swap with both operands x return (x of row r, x of row r^1) and (x of half h, x of half h^1)
__device__ __forceinline__ float max_over_groups(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float sum_over_groups(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Keeps the loads above it issued here: otherwise they are free to sink to their first use, which turns the
// next-page prefetch into a load-and-wait.  Registers are not touched, so no wait is implied.  (The cache pointers
// carry no __restrict__: loads of restrict read-only memory count as invariant and would cross the fence.)
__device__ __forceinline__ void issue_fence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);  // and no instruction that waits on older loads is scheduled above them
}

// The codes one lane needs from one (page, kv head) block, and the block's scales.
template <int BITS>
struct KvRegs {
  static constexpr int ROW = BITS == 8 ? kHeadDim : kHeadDim / 2;  // bytes per token row
  static constexpr int KW = BITS == 8 ? 8 : 4;                      // K dwords per lane
  static constexpr int VW = BITS == 8 ? 8 : 4;                      // V dwords per lane
  uint32_t k[KW], v[VW];
  uint32_t ksw, vsw;  // the block's two fp16 scales, each zero-extended in a register of its own

  // lane (n, g): K row n, bytes [ROW/4 * g, +ROW/4); V rows 4g .. 4g+3, bytes [ROW/16 * n, +ROW/16)
  __device__ __forceinline__ void load(const uint8_t* kblk, const uint8_t* vblk, const uint16_t* ksc,
                                       const uint16_t* vsc, size_t bi, int n, int g) {
    // The scales first, each zero-extended into a 32-bit register that nothing copies or packs before the scales are
    // used: packed as fp16 halves of one register (a copy that must wait for both loads), and issued as the page's
    // youngest loads, their wait covered every load in flight.
    ksw = ksc[bi];
    vsw = vsc[bi];
    const kv_u32x4_t* kp = reinterpret_cast<const kv_u32x4_t*>(kblk + n * ROW + (ROW / 4) * g);
    if constexpr (BITS == 8) {
      const kv_u32x4_t a = kp[0], b = kp[1];
      k[0] = a.x, k[1] = a.y, k[2] = a.z, k[3] = a.w, k[4] = b.x, k[5] = b.y, k[6] = b.z, k[7] = b.w;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const kv_u32x2_t t = *reinterpret_cast<const kv_u32x2_t*>(vblk + (4 * g + i) * ROW + 8 * n);
        v[i] = t.x, v[4 + i] = t.y;
      }
    } else {
      const kv_u32x4_t a = kp[0];
      k[0] = a.x, k[1] = a.y, k[2] = a.z, k[3] = a.w;
#pragma unroll
      for (int i = 0; i < 4; i++) v[i] = *reinterpret_cast<const uint32_t*>(vblk + (4 * g + i) * ROW + 4 * n);
    }
  }
  __device__ __forceinline__ _Float16 kscale() const { return __builtin_bit_cast(_Float16, (uint16_t)ksw); }
  __device__ __forceinline__ _Float16 vscale() const { return __builtin_bit_cast(_Float16, (uint16_t)vsw); }

  // K fragment c, biased: 1024 + bias + code (bias 128 / 8; removed after the MFMA, per page, from the query sums).
  // Dims of lane group g, in the order the Q fragment uses: 8 bits, dwords 2c, 2c+1 = dims 32g + 8c + 0..7;
  // 4 bits, dword c = dims 32g + 8c + 0..7 as nibbles 0..7, taken in pairs (s, s+4) straight into fp16 halves.
  __device__ __forceinline__ half8_t kfrag(int c) const {
    if constexpr (BITS == 8) {
      const uint32_t x = k[2 * c] ^ 0x80808080u, y = k[2 * c + 1] ^ 0x80808080u;
      return __builtin_bit_cast(half8_t, kv_u32x4_t{__builtin_amdgcn_perm(0x64646464u, x, 0x05010400u),
                                                     __builtin_amdgcn_perm(0x64646464u, x, 0x05030402u),
                                                     __builtin_amdgcn_perm(0x64646464u, y, 0x05010400u),
                                                     __builtin_amdgcn_perm(0x64646464u, y, 0x05030402u)});
    } else {
      const uint32_t x = k[c];
      return __builtin_bit_cast(half8_t, kv_u32x4_t{(x & 0x000F000Fu) ^ 0x64086408u, ((x >> 4) & 0x000F000Fu) ^ 0x64086408u,
                                                     ((x >> 8) & 0x000F000Fu) ^ 0x64086408u,
                                                     ((x >> 12) & 0x000F000Fu) ^ 0x64086408u});
    }
  }

  // V^T fragments: vt[db] = the 4 keys' biased codes at dim 8n + db
  __device__ __forceinline__ void vtrans(uint32_t vt[8]) const {
    if constexpr (BITS == 8) {
      uint32_t lo[4] = {v[0] ^ 0x80808080u, v[1] ^ 0x80808080u, v[2] ^ 0x80808080u, v[3] ^ 0x80808080u};
      uint32_t hi[4] = {v[4] ^ 0x80808080u, v[5] ^ 0x80808080u, v[6] ^ 0x80808080u, v[7] ^ 0x80808080u};
      transpose4x4(lo, vt);
      transpose4x4(hi, vt + 4);
    } else {
      uint32_t tb[4];
      transpose4x4(v, tb);  // tb[j]: byte j (dims 8n + 2j, 8n + 2j + 1) of the 4 keys
#pragma unroll
      for (int j = 0; j < 4; j++) {
        vt[2 * j] = (tb[j] & 0x0F0F0F0Fu) ^ 0x08080808u;
        vt[2 * j + 1] = ((tb[j] >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
      }
    }
  }
};

template <int BITS>
struct KvState {
  float m = -INFINITY, l = 0.f;  // running max (base 2) and sum for query n
  float4_t o[8];

  // One page: logits in base 2 are (S - kbias * qsum) * k_scale * qk_scale.  The reference max m moves only when a
  // page max passes it by more than 4 (then every p <= 16, and P' = p * v_scale stays far inside fp16), so O and l
  // are rarely rescaled; (m, l, O) stay consistent for the merges either way.
  __device__ __forceinline__ void process(const KvRegs<BITS>& r, const half8_t qf[4], float qsum, int key0, int L,
                                          float qk_scale, int g) {
    constexpr float kBias = BITS == 8 ? 1152.0f : 1032.0f;
    float4_t st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 4; c++) st = __builtin_amdgcn_mfma_f32_16x16x32_f16(r.kfrag(c), qf[c], st, 0, 0, 0);
    const float sc = (float)r.kscale() * qk_scale;
    const float off = -kBias * qsum * sc;
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sv[i] = __builtin_fmaf(st[i], sc, off);
    if (key0 + kPage > L) {  // the sequence ends inside this page
#pragma unroll
      for (int i = 0; i < 4; i++) sv[i] = key0 + 4 * g + i < L ? sv[i] : -INFINITY;
    }
    const float pm = max_over_groups(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
    if (__builtin_amdgcn_ballot_w64(pm > m + 4.f)) {
      const float m_new = fmaxf(m, pm);
      const float alpha = __builtin_amdgcn_exp2f(m - m_new);  // 0 on the first page (m = -inf)
      m = m_new;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 8; db++) o[db] *= alpha;
    }
    const float vs = (float)r.vscale();
    float psum = 0.f;
    half4_t pf;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float p = __builtin_amdgcn_exp2f(sv[i] - m);
      psum += p;
      pf[i] = (_Float16)(p * vs);
    }
    l += sum_over_groups(psum);
    uint32_t vt[8];
    r.vtrans(vt);
#pragma unroll
    for (int db = 0; db < 8; db++)
      o[db] = __builtin_amdgcn_mfma_f32_16x16x16f16(codes_f16(vt[db], (_Float16)kBias), pf, o[db], 0, 0, 0);
  }
};

template <int BITS, int DEPTH, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void kv_decode_kernel(
    const _Float16* __restrict__ q, const uint8_t* kc, const uint8_t* vc, const uint16_t* ksc, const uint16_t* vsc,
    int num_pages,
    const int* __restrict__ page_table, int max_pages, const int* __restrict__ seq_lens, int Hq, int Hkv,
    float qk_scale, int chunk_pages, float* __restrict__ part_o, float* __restrict__ part_ml,
    _Float16* __restrict__ out) {
  constexpr int ROW = KvRegs<BITS>::ROW;
  extern __shared__ float red[];  // [WAVES][G][D + 1] then [WAVES][G][2]
  const int chunk = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int G = Hq / Hkv;
  const int L = min(seq_lens[b], max_pages * kPage);
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63;
  const int n = l & 15, g = l >> 4;

  // Q^T fragment of query n (zero for n >= G), dims in K-fragment order; qsum = sum of its 128 dims
  half8_t qf[4];
  float qpart = 0.f;
  {
    const _Float16* qrow = q + ((size_t)b * Hq + hk * G + min(n, G - 1)) * kHeadDim + 32 * g;
    const _Float16 live = n < G ? (_Float16)1.0f : (_Float16)0.0f;
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int d = BITS == 8 ? 8 * c + e : 8 * c + (e >> 1) + 4 * (e & 1);
        qf[c][e] = qrow[d] * live;
        qpart += (float)qf[c][e];
      }
  }
  const float qsum = sum_over_groups(qpart);

  KvState<BITS> s;
#pragma unroll
  for (int db = 0; db < 8; db++) s.o[db] = float4_t{0.f, 0.f, 0.f, 0.f};

  // this wave's pages: logical pages p0 + w, p0 + w + WAVES, ... below min(chunk end, pages of the sequence)
  const int p0 = chunk * chunk_pages;
  const int p_end = min(p0 + chunk_pages, (L + kPage - 1) / kPage);
  const int* ptab = page_table + (size_t)b * max_pages;
  const size_t blk_bytes = (size_t)kPage * ROW;
  int lp = p0 + w;
  if (lp < p_end) {
    // DEPTH register sets rotate: DEPTH - 1 pages are in flight while one is worked on.  The trip is unrolled over
    // the sets so each keeps its registers (no copies that would wait on their loads).  Loads past the wave's last
    // page repeat that page.  Out-of-range page ids are clamped into the cache (never dereferenced outside it).
    KvRegs<BITS> r[DEPTH];
    auto page_of = [&](int p) { return (size_t)min(max(ptab[p], 0), num_pages - 1) * Hkv + hk; };
    auto load = [&](KvRegs<BITS>& dst, int p) {
      const size_t bi = page_of(min(p, p_end - 1));
      dst.load(kc + bi * blk_bytes, vc + bi * blk_bytes, ksc, vsc, bi, n, g);
    };
#pragma unroll
    for (int j = 0; j < DEPTH - 1; j++) load(r[j], lp + j * WAVES);
    bool more = true;
    while (more) {
#pragma unroll
      for (int j = 0; j < DEPTH; j++) {
        if (more) {
          load(r[(j + DEPTH - 1) % DEPTH], lp + (DEPTH - 1) * WAVES);
          issue_fence();
          s.process(r[j], qf, qsum, lp * kPage, L, qk_scale, g);
          lp += WAVES;
          more = lp < p_end;
        }
      }
    }
  }

  // merge the waves; lane (n, g) holds dims 32g + 8i + db (i < 4, db < 8) of query n
  float* red_o = red;
  float* red_ml = red + WAVES * G * (kHeadDim + 1);
  if (n < G) {
    float* dst = red_o + (w * G + n) * (kHeadDim + 1) + 32 * g;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int db = 0; db < 8; db++) dst[8 * i + db] = s.o[db][i];
    if (g == 0) {
      red_ml[(w * G + n) * 2] = s.m;
      red_ml[(w * G + n) * 2 + 1] = s.l;
    }
  }
  __syncthreads();
  const int tq = threadIdx.x >> 4, td = (threadIdx.x & 15) * 8;  // query tq, dims td .. td+7
  if (tq >= G) return;
  float mx = -INFINITY;
#pragma unroll
  for (int ww = 0; ww < WAVES; ww++) mx = fmaxf(mx, red_ml[(ww * G + tq) * 2]);
  float lsum = 0.f, acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ww = 0; ww < WAVES; ww++) {
    const float mw = red_ml[(ww * G + tq) * 2];
    const float f = mw == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mw - mx);
    lsum += red_ml[(ww * G + tq) * 2 + 1] * f;
    const float* src = red_o + (ww * G + tq) * (kHeadDim + 1) + td;
#pragma unroll
    for (int e = 0; e < 8; e++) acc[e] += src[e] * f;
  }
  if (gridDim.x == 1) {  // one chunk per sequence: its state is the result (no merge launch)
    half8_t h;
#pragma unroll
    for (int e = 0; e < 8; e++) h[e] = (_Float16)(lsum > 0.f ? acc[e] / lsum : 0.f);
    *reinterpret_cast<half8_t*>(out + ((size_t)b * Hq + hk * G + tq) * kHeadDim + td) = h;
    return;
  }
  const size_t slot = (((size_t)b * Hkv + hk) * gridDim.x + chunk) * G + tq;
  float4_t* po = reinterpret_cast<float4_t*>(part_o + slot * kHeadDim + td);
  po[0] = float4_t{acc[0], acc[1], acc[2], acc[3]};
  po[1] = float4_t{acc[4], acc[5], acc[6], acc[7]};
  if (td == 0) {
    part_ml[slot * 2] = mx;
    part_ml[slot * 2 + 1] = lsum;
  }
}

// out[b][h] = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c.  One workgroup per query head; wave w folds chunks
// w, w+4, ... into a running (M, L, O) (lane: dims 2l, 2l+1), then the 4 waves combine in LDS.  Fixed order.
__global__ __launch_bounds__(kMergeWaves * 64) void kv_merge_kernel(const float* __restrict__ part_o,
                                                       const float* __restrict__ part_ml, int Hq, int Hkv, int chunks,
                                                       _Float16* __restrict__ out) {
  __shared__ float sm_ml[kMergeWaves][2];
  __shared__ float sm_o[kMergeWaves][kHeadDim];
  const int h = blockIdx.x, b = blockIdx.y;
  const int G = Hq / Hkv, hk = h / G, q = h - hk * G;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63;
  const size_t base = ((size_t)b * Hkv + hk) * chunks;  // slot of chunk c: (base + c) * G + q
  float M = -INFINITY, L = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll 4
  for (int c = w; c < chunks; c += kMergeWaves) {
    const size_t slot = (base + c) * G + q;
    const float mc = part_ml[slot * 2], lc = part_ml[slot * 2 + 1];
    const float2 oc = *reinterpret_cast<const float2*>(part_o + slot * kHeadDim + 2 * l);
    const float mn = fmaxf(M, mc);
    // equal maxima scale by 1 (also covers -inf == -inf: an empty chunk has l = 0, O = 0)
    const float fa = M == mn ? 1.f : __builtin_amdgcn_exp2f(M - mn);
    const float fc = mc == mn ? 1.f : __builtin_amdgcn_exp2f(mc - mn);
    L = L * fa + lc * fc;
    a0 = a0 * fa + oc.x * fc;
    a1 = a1 * fa + oc.y * fc;
    M = mn;
  }
  if (l == 0) {
    sm_ml[w][0] = M;
    sm_ml[w][1] = L;
  }
  sm_o[w][2 * l] = a0;
  sm_o[w][2 * l + 1] = a1;
  __syncthreads();
  if (threadIdx.x >= kHeadDim) return;
  const int d = threadIdx.x;
  float mx = -INFINITY;
#pragma unroll
  for (int ww = 0; ww < kMergeWaves; ww++) mx = fmaxf(mx, sm_ml[ww][0]);
  float lsum = 0.f, acc = 0.f;
#pragma unroll
  for (int ww = 0; ww < kMergeWaves; ww++) {
    const float f = sm_ml[ww][0] == mx ? 1.f : __builtin_amdgcn_exp2f(sm_ml[ww][0] - mx);
    lsum += sm_ml[ww][1] * f;
    acc += sm_o[ww][d] * f;
  }
  out[((size_t)b * Hq + h) * kHeadDim + d] = (_Float16)(lsum > 0.f ? acc / lsum : 0.f);
}

// Workgroup shape and pages per workgroup.  8 waves per workgroup and chunks that fill the GPU about one workgroup
// per CU (256) deep; groups whose 8-wave LDS merge would pass 64 KB take 4 waves and about 1024 workgroups.  Fewer
// chunks mean fewer partial states to write and merge: at 16 sequences x 8 kv heads, 2 chunks of 8 waves measured 3 %
// faster (8-bit) than 8 chunks of 4 waves, and 4 chunks of 8 waves or 2 of 16 no faster than 2 of 8.  chunk_pages is
// a multiple of the wave count.
struct KvPlan {
  int waves, chunk_pages, chunks;
};
// EXL3_KV_WAVES (4 or 8) and EXL3_KV_TARGET_WGS override the plan for measurements; read once per process, so the
// workspace size and the launch always follow the same plan.
static KvPlan kv_plan(int batch, int num_kv_heads, int group, int max_pages) {
  static const int env_waves = [] {
    const char* e = getenv("EXL3_KV_WAVES");
    return e && atoi(e) == 4 ? 4 : kKvWaves;
  }();
  static const int env_target = [] {
    const char* e = getenv("EXL3_KV_TARGET_WGS");
    return e ? std::max(1, atoi(e)) : 0;
  }();
  int waves = env_waves;
  if ((size_t)waves * group * (kHeadDim + 1 + 2) * sizeof(float) > 65536) waves = 4;
  const int target = env_target ? env_target : waves == 8 ? 256 : 1024;
  const long pairs = (long)batch * num_kv_heads;
  const long chunks = std::max(1L, std::min((long)(max_pages + waves - 1) / waves, (target + pairs - 1) / pairs));
  int cp = (int)((max_pages + chunks - 1) / chunks);
  cp = (cp + waves - 1) / waves * waves;
  return KvPlan{waves, cp, (max_pages + cp - 1) / cp};
}

}  // namespace exl3

using namespace exl3;

extern "C" size_t exl3_kv_decode_workspace_bytes(int batch, int num_q_heads, int num_kv_heads, int max_pages) {
  if (batch <= 0 || num_kv_heads <= 0 || num_q_heads < num_kv_heads || max_pages <= 0) return 0;
  const int G = num_q_heads / num_kv_heads;
  const KvPlan plan = kv_plan(batch, num_kv_heads, G, max_pages);
  const size_t slots = (size_t)batch * num_kv_heads * plan.chunks * G;
  return slots * (kHeadDim + 2) * sizeof(float);
}

extern "C" int exl3_kv_decode_attention(const void* q, const void* k_cache, const void* v_cache, const void* k_scale,
                                        const void* v_scale, int num_pages, const void* page_table, int max_pages,
                                        const void* seq_lens, int batch, int num_q_heads, int num_kv_heads,
                                        int head_dim, int page_size, int bits, float sm_scale, void* out,
                                        void* workspace, size_t workspace_bytes, void* stream) {
  EXL3_CHECK_ARG((batch == 0 || (q && page_table && seq_lens && out)) && k_cache && v_cache && k_scale && v_scale,
                 "exl3_kv_decode_attention: null pointer");
  EXL3_CHECK_ARG(head_dim == kHeadDim && page_size == kPage,
                 "exl3_kv_decode_attention: head_dim = %d, page_size = %d (supported: 128, 16)", head_dim, page_size);
  EXL3_CHECK_ARG(bits == 4 || bits == 8, "exl3_kv_decode_attention: bits = %d (4 or 8)", bits);
  EXL3_CHECK_ARG(batch >= 0 && num_pages >= 1 && max_pages >= 1 && num_kv_heads >= 1 &&
                     num_q_heads % num_kv_heads == 0 && num_q_heads / num_kv_heads >= 1 &&
                     num_q_heads / num_kv_heads <= kMaxGroup,
                 "exl3_kv_decode_attention: batch = %d, pages = %d, max_pages = %d, heads %d / %d (group <= 16)",
                 batch, num_pages, max_pages, num_q_heads, num_kv_heads);
  if (batch == 0) return EXL3_OK;
  const size_t need = exl3_kv_decode_workspace_bytes(batch, num_q_heads, num_kv_heads, max_pages);
  EXL3_CHECK_ARG(workspace && workspace_bytes >= need, "exl3_kv_decode_attention: workspace %zu bytes, need %zu",
                 workspace_bytes, need);
  const int G = num_q_heads / num_kv_heads;
  const KvPlan plan = kv_plan(batch, num_kv_heads, G, max_pages);
  const int chunks = plan.chunks;
  float* part_o = static_cast<float*>(workspace);
  float* part_ml = part_o + (size_t)batch * num_kv_heads * chunks * G * kHeadDim;
  const float qk_scale = sm_scale * 1.4426950408889634f;  // logits in base 2
  const size_t lds = (size_t)plan.waves * G * (kHeadDim + 1 + 2) * sizeof(float);
  hipStream_t st = as_stream(stream);
  const dim3 grid(chunks, num_kv_heads, batch);
  auto qp = static_cast<const _Float16*>(q);
  auto kp = static_cast<const uint8_t*>(k_cache);
  auto vp = static_cast<const uint8_t*>(v_cache);
  auto ksp = static_cast<const uint16_t*>(k_scale);  // fp16 bits
  auto vsp = static_cast<const uint16_t*>(v_scale);
  auto pt = static_cast<const int*>(page_table);
  auto sl = static_cast<const int*>(seq_lens);
  static const int depth = [] {  // register page sets per wave (prefetch distance + 1); deeper sets measured no faster
    const char* e = getenv("EXL3_KV_DEPTH");
    return e ? std::min(5, std::max(2, atoi(e))) : 2;
  }();
  using Kern = decltype(&kv_decode_kernel<8, 2, 4>);
  static const Kern table[2][2][4] = {
      {{kv_decode_kernel<4, 2, 4>, kv_decode_kernel<4, 3, 4>, kv_decode_kernel<4, 4, 4>, kv_decode_kernel<4, 5, 4>},
       {kv_decode_kernel<8, 2, 4>, kv_decode_kernel<8, 3, 4>, kv_decode_kernel<8, 4, 4>, kv_decode_kernel<8, 5, 4>}},
      {{kv_decode_kernel<4, 2, 8>, kv_decode_kernel<4, 3, 8>, kv_decode_kernel<4, 4, 8>, kv_decode_kernel<4, 5, 8>},
       {kv_decode_kernel<8, 2, 8>, kv_decode_kernel<8, 3, 8>, kv_decode_kernel<8, 4, 8>, kv_decode_kernel<8, 5, 8>}}};
  table[plan.waves == 8][bits == 8][depth - 2]<<<grid, plan.waves * 64, lds, st>>>(
      qp, kp, vp, ksp, vsp, num_pages, pt, max_pages, sl, num_q_heads, num_kv_heads, qk_scale, plan.chunk_pages,
      part_o, part_ml, static_cast<_Float16*>(out));
  EXL3_CHECK_LAUNCH();
  if (chunks > 1) {
    kv_merge_kernel<<<dim3(num_q_heads, batch), kMergeWaves * 64, 0, st>>>(part_o, part_ml, num_q_heads,
                                                                           num_kv_heads, chunks,
                                                                           static_cast<_Float16*>(out));
    EXL3_CHECK_LAUNCH();
  }
  return EXL3_OK;
}
