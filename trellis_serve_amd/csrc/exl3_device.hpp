// Device building blocks of the EXL3 hot path on gfx950 (CDNA4, wave64).
//
// Format (core/src/trellis_core/reference.py:1-16): a linear's trellis is int16 [k/16, n/16, 16K]; each 16x16 tile
// is 256*K bits, read as uint32 words w[m] = h[2m] | h[2m+1] << 16 (a little-endian dword load), bits MSB first.
// Element t (0..255) of a tile is the codebook value of the 16-bit window that ENDS at bit (t+1)K, circular in the
// tile (reference.py:80-99); it lands at row 8((t>>1)&1) + 2((t>>3)&3) + (t&1), column (t>>5) + 8((t>>2)&1)
// (reference.py:30-45, the closed form of xpu/csrc/exl3_esimd.h:6-8).
//
// Lane geometry used by every kernel here: one wave64 owns one tile; lane l takes column c = l % 16 and the group
// j = l / 16 of four stream-consecutive elements t0..t0+3, t0 = 32(c&7) + 4(c>>3) + 8j, which sit at rows
// 2j, 2j+1, 2j+8, 2j+9 of column c.  Four consecutive elements need 3K+16 bits, always inside two adjacent tile
// dwords (wrapping at the tile end for t0 = 0), so a lane loads two dwords per tile, funnels them with one
// v_alignbit into a 32-bit chunk and pulls the four 16-bit states with v_bfe.  The group is exactly one lane's
// slice of an MFMA 16x16x16 f16 B operand (lane l: column l%16, k-chunk l/16), so decoded values feed the matrix
// core straight from registers; the A operand (activations) uses the same row order.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace exl3 {

enum Codebook : int { CB_3INST = 0, CB_MCG = 1, CB_MUL1 = 2 };

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));

// 1/sqrt(128) as the reference kernels write it (cuda/csrc/exl3_marlin.cu:251)
constexpr float kHadScale = 0.088388347648f;

// fp16 of an fp32 product with two roundings, fp32 product then fp16, as the reference's __float2half_rn(a * b)
// (here: the rotation scale, the SiLU product).  The empty asm keeps the fp32 product in a register: otherwise the backend may fuse multiply and conversion into
// one v_fma_mixlo_f16 (a single rounding, one ulp apart in rare cases) in some expansions of an expression and not
// in others, so two kernels evaluating the same expression could disagree.
__device__ __forceinline__ _Float16 f16_of_f32(float p) {
  __asm__("" : "+v"(p));
  return (_Float16)p;
}
__device__ __forceinline__ _Float16 had_scale_f16(float f) { return f16_of_f32(f * kHadScale); }

// SiLU in fp32 (the MoE GLU, cuda/csrc/exl3_marlin_moe.cu:228-258)
__device__ __forceinline__ float silu32(float v) { return v / (1.0f + __expf(-v)); }

// s_waitcnt immediate for "vmcnt <= n" with expcnt and lgkmcnt unconstrained (gfx9 encoding: vmcnt bits 3:0 and
// 15:14, expcnt 6:4, lgkmcnt 11:8)
__host__ __device__ constexpr int waitcnt_vm(int n) { return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }

// Workgroup barrier that waits for this wave's LDS accesses only.  __syncthreads() adds a workgroup fence, which
// makes the compiler wait for every outstanding global load (vmcnt(0)) and would drain loads that are meant to stay
// in flight across the barrier; LDS data written from loaded values is waited for by its own data dependence.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// ---- per-lane tile geometry ----------------------------------------------------------------------------------
struct LaneGeo {
  int dw0, dw1;  // tile dwords holding the lane's bits (dw1 = dw0 + 1, circular)
  int sh;        // v_alignbit shift that puts stream bit S (first window bit) at chunk bit 31
  int pS;        // position of S inside the 64-bit pair (1..32)
};

// c: tile column 0..15, j: group 0..3
template <int K>
__device__ __forceinline__ LaneGeo lane_geo(int c, int j) {
  const int t0 = 32 * (c & 7) + 4 * (c >> 3) + 8 * j;
  const int S = (t0 + 1) * K - 16;  // first bit of element t0's window; -16 < S only wraps for t0 = 0
  const int d0 = (S - 1) >> 5;      // floor((S-1)/32): arithmetic shift, -1 for the wrapping lane
  LaneGeo g;
  g.pS = S - 32 * d0;
  g.sh = 32 - g.pS;
  g.dw0 = (d0 + 8 * K) % (8 * K);
  g.dw1 = (d0 + 1) % (8 * K);
  return g;
}

// four 16-bit states of the lane's group from its two dwords (w0 = dword dw0, w1 = dword dw1)
template <int K>
__device__ __forceinline__ void group_states(uint32_t w0, uint32_t w1, const LaneGeo& g, uint32_t s[4]) {
  const uint32_t ch = __builtin_amdgcn_alignbit(w0, w1, g.sh);
#pragma unroll
  for (int e = 0; e < 4; e++) {
    if (16 - e * K >= 0)
      s[e] = __builtin_amdgcn_ubfe(ch, 16 - e * K, 16);
    else  // window starts beyond the first chunk (K = 6, 8 at e = 3): funnel it to the bottom
      s[e] = __builtin_amdgcn_alignbit(w0, w1, 48 - g.pS - e * K) & 0xFFFFu;
  }
}

// ---- codebooks (reference.py:52-73; cuda/csrc/third_party/exllamav3/codebook.cuh:28-123) --------------------
// x = s * C (+ A) mod 2^32 with s < 2^16: one v_mul_lo_u32 (MCG, MUL1) or v_mad_u64_u32 (3INST), both full rate on
// gfx950 (about 59 lane-ops/clk/CU measured, as fast as v_add).
constexpr uint32_t kMcgMult = 0xCBAC1FEDu;
constexpr uint32_t kMul1Mult = 0x83DCD12Du;
constexpr uint32_t k3InstMult = 89226354u;
constexpr uint32_t k3InstAdd = 64248484u;

template <int CB>
__device__ __forceinline__ uint32_t cb_hash_masked(uint32_t s) {
  uint32_t x;
  if constexpr (CB == CB_MCG)
    x = s * kMcgMult;
  else
    x = (uint32_t)((uint64_t)s * k3InstMult + k3InstAdd);
  return (x & 0x8FFF8FFFu) ^ 0x3B603B60u;  // one v_bitop3_b32
}

// fp16 pair [lo + hi of y0, lo + hi of y1], each sum rounded once (v_add_f16 == __hadd).
#ifndef EXL3_PERM_HALF_SUMS
// SDWA reads the halves in place and writes the second sum into the upper half: one VALU op per weight.  The
// compiler cannot see the VGPR writes inside the asm, so where the sums feed an MFMA (MFMA_NEXT) the block ends with
// the wait states an MFMA needs before reading a VGPR a VALU op wrote (without them the next MFMA has read a stale B
// operand).  Sums that are stored (to LDS or memory) need no wait states: the store waits for its data like any
// other instruction (prefill GEMM without them: 2 % faster, same results).
template <bool MFMA_NEXT = true>
__device__ __forceinline__ uint32_t half_sums(uint32_t y0, uint32_t y1) {
  uint32_t r;
  if constexpr (MFMA_NEXT)
    asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "v_add_f16_sdwa %0, %2, %2 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "s_nop 2"
        : "=&v"(r)
        : "v"(y0), "v"(y1));
  else
    asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "v_add_f16_sdwa %0, %2, %2 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
        : "=&v"(r)
        : "v"(y0), "v"(y1));
  return r;
}
#else
// Two v_perm gather the low and the high halves, one v_pk_add_f16 adds them: 1.5 VALU ops per weight, all visible
// to the compiler's hazard tracking.
template <bool MFMA_NEXT = true>
__device__ __forceinline__ uint32_t half_sums(uint32_t y0, uint32_t y1) {
  const uint32_t lo = __builtin_amdgcn_perm(y1, y0, 0x05040100u);  // [y0.lo, y1.lo]
  const uint32_t hi = __builtin_amdgcn_perm(y1, y0, 0x07060302u);  // [y0.hi, y1.hi]
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2_t, lo) + __builtin_bit_cast(half2_t, hi));
}
#endif

// two states -> packed fp16 [v(sa), v(sb)], bit-exact with codebook_lut
template <int CB, bool MFMA_NEXT = true>
__device__ __forceinline__ uint32_t cb_pair(uint32_t sa, uint32_t sb) {
  if constexpr (CB == CB_MUL1) {
    // h = fp16 bits 0x6400 + bytesum(x) = 1024 + bytesum exactly; v = fma(h, 0x1EEE, 0xC931) rounded once
    const uint32_t ha = __builtin_amdgcn_udot4(sa * kMul1Mult, 0x01010101u, 0x6400u, false);
    const uint32_t hb = __builtin_amdgcn_udot4(sb * kMul1Mult, 0x01010101u, 0x6400u, false);
    const half2_t h = __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(hb, ha, 0x05040100u));
    const half2_t inv = __builtin_bit_cast(half2_t, 0x1EEE1EEEu);
    const half2_t bias = __builtin_bit_cast(half2_t, 0xC931C931u);
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(h, inv, bias));
  } else {
    return half_sums<MFMA_NEXT>(cb_hash_masked<CB>(sa), cb_hash_masked<CB>(sb));
  }
}

// the lane's four decoded weights (rows 2j, 2j+1, 2j+8, 2j+9 of column c) as an MFMA operand (MFMA_NEXT), or as
// values to store
template <int K, int CB, bool MFMA_NEXT = true>
__device__ __forceinline__ half4_t decode_group(uint32_t w0, uint32_t w1, const LaneGeo& g) {
  uint32_t s[4];
  group_states<K>(w0, w1, g, s);
  uint2_t p;
  p.x = cb_pair<CB, MFMA_NEXT>(s[0], s[1]);
  p.y = cb_pair<CB, MFMA_NEXT>(s[2], s[3]);
  return __builtin_bit_cast(half4_t, p);
}

// The lane's weights of two tiles (its group of tile a, then of tile b) as one 8-half MFMA 16x16x32 B fragment,
// rounded as decode_group rounds them.  For MCG / 3INST the eight half sums sit in one asm block, so one set of MFMA
// wait states follows all of them (the compiler may order separate blocks either way round).
template <int K, int CB>
__device__ __forceinline__ half8_t decode_two_groups(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1,
                                                     const LaneGeo& g) {
  uint32_t s[8];
  group_states<K>(a0, a1, g, s);
  group_states<K>(b0, b1, g, s + 4);
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  u32x4 r;
  if constexpr (CB == CB_MUL1) {
    r = u32x4{cb_pair<CB>(s[0], s[1]), cb_pair<CB>(s[2], s[3]), cb_pair<CB>(s[4], s[5]), cb_pair<CB>(s[6], s[7])};
  } else {
    uint32_t y[8];
#pragma unroll
    for (int e = 0; e < 8; e++) y[e] = cb_hash_masked<CB>(s[e]);
    uint32_t r0, r1, r2, r3;
    asm("v_add_f16_sdwa %0, %4, %4 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "v_add_f16_sdwa %1, %6, %6 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "v_add_f16_sdwa %2, %8, %8 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "v_add_f16_sdwa %3, %10, %10 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "v_add_f16_sdwa %0, %5, %5 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "v_add_f16_sdwa %1, %7, %7 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "v_add_f16_sdwa %2, %9, %9 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "v_add_f16_sdwa %3, %11, %11 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1\n\t"
        "s_nop 2"
        : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
        : "v"(y[0]), "v"(y[1]), "v"(y[2]), "v"(y[3]), "v"(y[4]), "v"(y[5]), "v"(y[6]), "v"(y[7]));
    r = u32x4{r0, r1, r2, r3};
  }
  return __builtin_bit_cast(half8_t, r);
}

// ---- fp16 / bf16 boundary conversions (torch value conversions, RNE) -----------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40);  // NaN stays (quiet) NaN
  u += 0x7FFFu + ((u >> 16) & 1u);                                          // round to nearest even
  return (uint16_t)(u >> 16);
}

// ---- 128-point Hadamard on 32 lanes x 4 values (lane t holds block positions 4t..4t+3) -----------------------
// Sylvester order: H128 = H32 (lanes) x H4 (in-lane); the in-lane part is the 4-point butterfly, the lane part five
// xor-butterflies.  fp32 throughout, as cuda/csrc/exl3_had.cuh:20-84.
//
// The partner value of a lane-xor stage comes from the VALU's cross-lane paths, not the LDS unit (ds_bpermute):
// xor 1 and 2 are DPP quad permutes, xor 8 a DPP row rotate by 8, xor 4 two DPP row rotates (by 12 and by 4: the
// lanes whose bit 2 is clear take the lane 4 above, the others the lane 4 below; neither wraps inside the 16-lane
// row; row_ror:n gives lane i the value of lane i - n of its row), xor 16 v_permlane16_swap (rows 2r and 2r+1).  Each stage computes partner + (+-own): the lower lane
// a + b and the upper lane a - b of the pair (a, b), exactly the sums of the xor-shuffle form.
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
  const int x = __builtin_bit_cast(int, v);
  if constexpr (M == 1) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
  } else if constexpr (M == 2) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
  } else if constexpr (M == 4) {
    const int up = __builtin_amdgcn_mov_dpp(x, 0x12C, 0xF, 0xF, false);  // row_ror:12 -> lane i + 4 of the row
    const int dn = __builtin_amdgcn_mov_dpp(x, 0x124, 0xF, 0xF, false);  // row_ror:4  -> lane i - 4 of the row
    return __builtin_bit_cast(float, (__lane_id() & 4) ? dn : up);
  } else if constexpr (M == 8) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, false));  // row_ror:8
  } else {
    static_assert(M == 16, "lane xor 1, 2, 4, 8 or 16");
    // with both operands x the swap returns (x of the even row, x of the odd row) in every lane of the row pair
    const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return __builtin_bit_cast(float, (int)((__lane_id() & 16) ? p[0] : p[1]));
  }
}

template <int M>
__device__ __forceinline__ void had_stage(float& h0, float& h1, float& h2, float& h3) {
  const uint32_t flip = (__lane_id() & M) ? 0x80000000u : 0u;  // the upper lane subtracts its own value
  auto step = [&](float& h) { h = lane_xor<M>(h) + __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, h) ^ flip); };
  step(h0);
  step(h1);
  step(h2);
  step(h3);
}

__device__ __forceinline__ void had128_x4(float& h0, float& h1, float& h2, float& h3) {
  const float s0 = h0 + h1, d0 = h0 - h1, s1 = h2 + h3, d1 = h2 - h3;
  h0 = s0 + s1;
  h1 = d0 + d1;
  h2 = s0 - s1;
  h3 = d0 - d1;
  had_stage<1>(h0, h1, h2, h3);
  had_stage<2>(h0, h1, h2, h3);
  had_stage<4>(h0, h1, h2, h3);
  had_stage<8>(h0, h1, h2, h3);
  had_stage<16>(h0, h1, h2, h3);
}

}  // namespace exl3
