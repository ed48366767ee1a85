// EXL3 prefill: fused decode-GEMM on gfx950 MFMA (v_mfma_f32_16x16x32_f16), y = Had(xh @ W_inner) * svh.
//
// Reference semantics: the reference's prefill is decode-to-HBM + cuBLAS between its rotation launches
// (cuda/src/sglang_exl3/runtime/ops.py:36-59); the fused Marlin path serves < 256 rows
// (exl3_marlin_template.h).  Here the weights are decoded into LDS inside the GEMM and never reach HBM.
//
// Operands
//   A: xh in "fragment order": the rotated activations with k permuted inside every 32-wide block so that the 8
//      halves one MFMA lane needs are contiguous: xh_f[m][32b + 8q + 4tr + e] = xh[m][32b + 16tr + r(q, e)],
//      r(q, e) = 2q + (e & 1) + 8(e >> 1) (written by had_in_frag_kernel).
//   B: the trellis.  A k-step covers 32 rows = 2 tile rows.  The lane-geometry decode of exl3_device.hpp gives lane
//      (c, j) of a tile the 4 weights of column c at rows r(j, 0..3); tile row tr of the k-step supplies halves
//      4tr..4tr+3 of the lane's 8-half B fragment.  A and B then agree on the k order of every MFMA.
//
// Tiling: workgroup 256 rows x 128 columns (one output rotation block), 4 waves as 2 x 2, wave tile 128 x 64
// (8 x 4 MFMA 16x16x32 tiles, 128 fp32 accumulators per lane).  Grid: x = column blocks (fastest: consecutive
// workgroups share the A rows in L2), y = row blocks.
//
// Pipeline: kStages-deep LDS ring of raw k-step inputs, filled by direct-to-LDS 16-byte buffer loads (no VGPR
// staging): per k-step each wave issues 4 A pieces (one m-block of 64 lanes x 16 B each: a lane's 16 bytes land
// exactly where its MFMA A fragment lives) and 1 piece of trellis bits (its 4 tiles of the k-step).  The compiler
// does not order LDS-DMA writes before LDS reads, so the waits are explicit: vmcnt(5 (kStages - 2)) leaves the
// younger stages in flight, and a barrier covers the other waves' pieces.  Each iteration runs the MFMAs of k-step
// kt next to the decode of k-step kt+1 (16 tiles per workgroup, 4 per wave, into a double-buffered fp16 B fragment
// area), so VALU decode work overlaps matrix work.
#include <stdlib.h>

#include <algorithm>

#include "exl3_api.hpp"
#include "exl3_device.hpp"

namespace exl3 {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBN = 128, kBK = 32;
constexpr int kGemmThreads = 256;
constexpr int kAStage = kBM * kBK * 2;   // 16 KB: [16 m-blocks][64 lanes][8 halves]
constexpr int kBStage = kBN * kBK * 2;   // 8 KB:  [8 n-blocks][64 lanes][8 halves]
constexpr int kCStride = kBN + 8;        // epilogue fp16 C tile row stride (halves)

struct GemmShards {
  const uint32_t* trellis[EXL3_MAX_SHARDS];
  const uint16_t* svh[EXL3_MAX_SHARDS];
  const uint16_t* xh[EXL3_MAX_SHARDS];  // per-shard rotated activations in fragment order [M][k]
  int tn[EXL3_MAX_SHARDS];
  int col0[EXL3_MAX_SHARDS];
  int blk0[EXL3_MAX_SHARDS + 1];
  int count;
};


// Workgroup barrier that waits for this wave's LDS accesses only.  __syncthreads() adds a workgroup fence, which
// makes the compiler wait for every outstanding load (vmcnt(0)) and would drain the direct-to-LDS pipeline; the
// direct-to-LDS writes are waited for explicitly (waitcnt_vm) before each barrier instead.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int K>
__host__ __device__ constexpr int gemm_bits_stage() { return 4 * 32 * K; }  // 4 tiles per wave
constexpr int kBitsRegion = 64 * 16;  // one 16-byte direct-to-LDS load lands at lane * 16: a full wave's span

// one ring stage: A pieces (kAStage) then the 4 waves' trellis bits regions
template <int K>
__host__ __device__ constexpr int gemm_ring_stage() { return kAStage + 4 * kBitsRegion; }

template <int K, int STAGES>
__host__ __device__ constexpr int gemm_lds_bytes() {
  return STAGES * gemm_ring_stage<K>() + 2 * kBStage > 128 * kCStride * 2
             ? STAGES * gemm_ring_stage<K>() + 2 * kBStage
             : 128 * kCStride * 2;
}

// rotated activations in fragment order: xh_f[s*rows + r][k] for shard s (see the header comment)
template <bool X_BF16>
__global__ __launch_bounds__(256) void had_in_frag_kernel(const void* __restrict__ x, int rows, int k,
                                                          const uint16_t* __restrict__ suh_cat, int shards,
                                                          uint16_t* __restrict__ xh) {
  const int kb = k >> 7;
  const int unit = blockIdx.x * 8 + (threadIdx.x >> 5);
  if (unit >= shards * rows * kb) return;
  const int t = threadIdx.x & 31;
  const int s = unit / (rows * kb), rem = unit - s * rows * kb, r = rem / kb, b = rem - r * kb;
  const int kk = b * 128 + 4 * t;
  const uint16_t* xr = static_cast<const uint16_t*>(x) + (size_t)r * k;
  const uint16_t* su = suh_cat + (size_t)s * k;
  _Float16 v[4];
  if constexpr (X_BF16) {
    const uint2_t raw = *reinterpret_cast<const uint2_t*>(xr + kk);
    v[0] = (_Float16)bf16_to_f32((uint16_t)(raw.x & 0xFFFF));
    v[1] = (_Float16)bf16_to_f32((uint16_t)(raw.x >> 16));
    v[2] = (_Float16)bf16_to_f32((uint16_t)(raw.y & 0xFFFF));
    v[3] = (_Float16)bf16_to_f32((uint16_t)(raw.y >> 16));
  } else {
    const half4_t raw = *reinterpret_cast<const half4_t*>(xr + kk);
    v[0] = raw.x; v[1] = raw.y; v[2] = raw.z; v[3] = raw.w;
  }
  const half4_t sv = *reinterpret_cast<const half4_t*>(su + kk);
  float f0 = (float)(_Float16)(v[0] * sv.x), f1 = (float)(_Float16)(v[1] * sv.y);
  float f2 = (float)(_Float16)(v[2] * sv.z), f3 = (float)(_Float16)(v[3] * sv.w);
  had128_x4(f0, f1, f2, f3);
  const _Float16 h[4] = {(_Float16)(f0 * kHadScale), (_Float16)(f1 * kHadScale), (_Float16)(f2 * kHadScale),
                         (_Float16)(f3 * kHadScale)};
  _Float16* dst = reinterpret_cast<_Float16*>(xh) + ((size_t)s * rows + r) * k + b * 128;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int p = 4 * t + i;                // position in the 128-block
    const int blk32 = p >> 5, p32 = p & 31;  // 32-block and position inside it
    const int tr = p32 >> 4, rr = p32 & 15;
    const int q = (rr & 7) >> 1, e = (rr & 1) | ((rr >> 3) << 1);
    dst[blk32 * 32 + q * 8 + tr * 4 + e] = h[i];
  }
}

template <int K, int CB, bool Y_BF16, int kStages>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(GemmShards sa, int M, int k, void* __restrict__ y,
                                                             int n_total, int rotate_out) {
  constexpr int BITS = gemm_bits_stage<K>();
  constexpr int RING = gemm_ring_stage<K>();
  static_assert(BITS <= kBitsRegion, "a wave's 4 tiles fit its bits region");
  constexpr int CHUNKS = BITS / 16;  // 16-byte pieces of one wave's 4 tiles
  static_assert(CHUNKS <= 64, "one gather per wave per k-step");
  constexpr int kLoadsPerStage = 5;  // per wave: 4 A pieces + 1 bits piece
  extern __shared__ __align__(16) uint8_t lds[];
  uint8_t* ring = lds;                        // [kStages][A pieces | bits of 4 waves]
  uint8_t* b_lds = lds + kStages * RING;      // [2][kBStage] decoded B fragments

  const int nblk = blockIdx.x, mblk = blockIdx.y;
  int s = 0;
#pragma unroll
  for (int i = 1; i < EXL3_MAX_SHARDS; i++)
    if (i < sa.count && nblk >= sa.blk0[i]) s = i;
  const int tn = sa.tn[s];
  const int tc0 = (nblk - sa.blk0[s]) * 8;  // first tile column of this block in the shard
  const int row0 = mblk * kBM;

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63;
  const int wm = w >> 1, wn = w & 1;
  const int c = l & 15, j = l >> 4;

  // B: wave w decodes tile row tr = w >> 1, tile columns 4 (w & 1) .. +3 of every k-step
  const int btr = w >> 1, btc = 4 * (w & 1);
  const int tile_bytes = 32 * K;
  const int row_bytes = tn * tile_bytes;
  const __amdgpu_buffer_rsrc_t brsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)sa.trellis[s], (short)0, (k >> 4) * row_bytes, 0x00020000);
  // lanes past the wave's 4 tiles re-read its last piece (same bytes, never decoded)
  const int bgoff = (tc0 + btc) * tile_bytes + min(l, CHUNKS - 1) * 16;  // + tile row * row_bytes
  const LaneGeo g = lane_geo<K>(c, j);

  // A: wave w loads m-blocks 4w .. 4w+3; lane l of a piece = row (l % 16) of the m-block, k-chunk l / 16.  Rows past
  // M re-read row M-1 (finite, only feeds discarded C rows).
  const uint16_t* xh = sa.xh[s];
  const __amdgpu_buffer_rsrc_t arsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)xh, (short)0, M * k * 2, 0x00020000);
  int aoff[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int row = min(row0 + (4 * w + i) * 16 + c, M - 1);
    aoff[i] = (row * k + j * 8) * 2;
  }

  // stage `slot` of the ring <- the inputs of k-step kd
  auto issue = [&](int slot, int kd) {
    const int kt = kd;
    uint8_t* st = ring + (slot % kStages) * RING;
#pragma unroll
    for (int i = 0; i < 4; i++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (__attribute__((address_space(3))) void*)(st + (4 * w + i) * 1024),
                                               16, aoff[i], kt * kBK * 2, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(brsrc, (__attribute__((address_space(3))) void*)(st + kAStage + w * kBitsRegion),
                                             16, bgoff, (2 * kt + btr) * row_bytes, 0, 0);
  };
  auto decode_b = [&](int kt) {
    const uint32_t* tw = reinterpret_cast<const uint32_t*>(ring + (kt % kStages) * RING + kAStage + w * kBitsRegion);
    uint8_t* dst = b_lds + (kt & 1) * kBStage;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const half4_t v = decode_group<K, CB>(tw[t * 8 * K + g.dw0], tw[t * 8 * K + g.dw1], g);
      // n-block btc + t, lane (c, j), halves 4 btr .. +3
      *reinterpret_cast<half4_t*>(dst + (((btc + t) * 64 + l) * 16) + btr * 8) = v;
    }
  };

  float4_t acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; i++)
#pragma unroll
    for (int jj = 0; jj < 4; jj++) acc[i][jj] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int ksteps = k / kBK;  // >= 4 (k >= 128)
#pragma unroll
  for (int p = 0; p < kStages - 1; p++) issue(p, min(p, ksteps - 1));
  // stage 0 in: everything but the kStages-2 younger stages
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(kLoadsPerStage * (kStages - 2)));
  lds_barrier();
  decode_b(0);
  lds_barrier();

  for (int kt = 0; kt < ksteps; kt++) {
    // keep kStages-1 k-steps in flight; past the end the free slot re-reads the last k-step (in range, never used)
    issue(kt + kStages - 1, min(kt + kStages - 1, ksteps - 1));
    // stage kt+1 in: everything but the kStages-2 younger stages
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(kLoadsPerStage * (kStages - 2)));
    lds_barrier();
    const half8_t* af = reinterpret_cast<const half8_t*>(ring + (kt % kStages) * RING) + (wm * 8) * 64 + l;
    const half8_t* bf = reinterpret_cast<const half8_t*>(b_lds + (kt & 1) * kBStage) + (wn * 4) * 64 + l;
    half8_t bv[4], av[8];
#pragma unroll
    for (int jj = 0; jj < 4; jj++) bv[jj] = bf[jj * 64];
#pragma unroll
    for (int i = 0; i < 8; i++) av[i] = af[i * 64];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
      for (int jj = 0; jj < 4; jj++)
        acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[i], bv[jj], acc[i][jj], 0, 0, 0);
    // the next k-step's weights (at the last step: a stale but valid stage into a buffer nobody reads, keeping the
    // loop body one scheduling region)
    decode_b(kt + 1);
    // interleave: the fragment reads first, then one MFMA per two VALU ops of the next k-step's decode
    __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);  // DS reads of the fragments
#pragma unroll
    for (int i = 0; i < 32; i++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
    }
    lds_barrier();
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // drain the trailing re-reads of every wave before LDS is reused
  __syncthreads();

  // ---- epilogue, two halves of 128 rows: the waves of that half put their fp16 C rows in LDS, then every 32-lane
  // group rotates whole rows (128 columns), scales by svh and stores
  _Float16* cl = reinterpret_cast<_Float16*>(lds);
  const int hw = tid >> 5, t = tid & 31;
  const int col = nblk * 128 + 4 * t;
  const uint16_t* svh = sa.svh[s] + (col - sa.col0[s]);
#pragma unroll
  for (int half = 0; half < 2; half++) {
    if (wm == half) {
#pragma unroll
      for (int i = 0; i < 8; i++)
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int m = i * 16 + 4 * j + r;
            const int n = wn * 64 + jj * 16 + c;
            cl[m * kCStride + n] = (_Float16)acc[i][jj][r];
          }
    }
    __syncthreads();
    for (int ml = hw; ml < 128; ml += 8) {
      const int m = row0 + half * 128 + ml;
      _Float16 h[4];
#pragma unroll
      for (int i = 0; i < 4; i++) h[i] = cl[ml * kCStride + 4 * t + i];
      if (rotate_out) {
        float f0 = (float)h[0], f1 = (float)h[1], f2 = (float)h[2], f3 = (float)h[3];
        had128_x4(f0, f1, f2, f3);
        const half4_t sv = *reinterpret_cast<const half4_t*>(svh);
        h[0] = (_Float16)(f0 * kHadScale) * sv.x;
        h[1] = (_Float16)(f1 * kHadScale) * sv.y;
        h[2] = (_Float16)(f2 * kHadScale) * sv.z;
        h[3] = (_Float16)(f3 * kHadScale) * sv.w;
      }
      if (m < M) {
        uint16_t* yr = static_cast<uint16_t*>(y) + (size_t)m * n_total + col;
        if constexpr (Y_BF16) {
          uint2_t o;
          o.x = (uint32_t)f32_to_bf16((float)h[0]) | ((uint32_t)f32_to_bf16((float)h[1]) << 16);
          o.y = (uint32_t)f32_to_bf16((float)h[2]) | ((uint32_t)f32_to_bf16((float)h[3]) << 16);
          *reinterpret_cast<uint2_t*>(yr) = o;
        } else {
          *reinterpret_cast<half4_t*>(yr) = half4_t{h[0], h[1], h[2], h[3]};
        }
      }
    }
    __syncthreads();
  }
}

#define EXL3_GEMM_DISPATCH(K_, CB_, ...)                                  \
  [&]() -> bool {                                                         \
    switch (K_ * 4 + CB_) {                                               \
      EXL3_GCASE(2, __VA_ARGS__) EXL3_GCASE(3, __VA_ARGS__)               \
      EXL3_GCASE(4, __VA_ARGS__) EXL3_GCASE(5, __VA_ARGS__)               \
      EXL3_GCASE(6, __VA_ARGS__) EXL3_GCASE(8, __VA_ARGS__)               \
      default: return false;                                              \
    }                                                                     \
  }()
#define EXL3_GCASE(KV, ...)                                                            \
  case KV * 4 + 0: { constexpr int kK = KV, kCB = 0; __VA_ARGS__; return true; }      \
  case KV * 4 + 1: { constexpr int kK = KV, kCB = 1; __VA_ARGS__; return true; }      \
  case KV * 4 + 2: { constexpr int kK = KV, kCB = 2; __VA_ARGS__; return true; }

}  // namespace exl3

using namespace exl3;

extern "C" size_t exl3_prefill_workspace_bytes(int rows, int k, int nshards) {
  if (rows <= 0 || k <= 0 || k % 128 || nshards < 1 || nshards > EXL3_MAX_SHARDS) return 0;
  return ((size_t)nshards * rows * k * 2 + 255) & ~(size_t)255;
}

extern "C" int exl3_linear_prefill(const void* x, int x_bf16, int rows, int k, const exl3_shard* shards_host,
                                   int nshards, int K, int codebook, void* y, int y_bf16, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  EXL3_CHECK_ARG(x && y && shards_host, "exl3_linear_prefill: null pointer");
  EXL3_CHECK_ARG(valid_bits(K) && valid_cb(codebook), "exl3_linear_prefill: K = %d / codebook = %d", K, codebook);
  EXL3_CHECK_ARG(rows >= 0 && k > 0 && k % 128 == 0, "exl3_linear_prefill: rows = %d, k = %d", rows, k);
  EXL3_CHECK_ARG(nshards >= 1 && nshards <= EXL3_MAX_SHARDS, "exl3_linear_prefill: nshards = %d", nshards);
  if (rows == 0) return EXL3_OK;
  EXL3_CHECK_ARG((int64_t)rows * k * 2 <= INT32_MAX, "exl3_linear_prefill: rows * k too large for one launch");
  const size_t need = exl3_prefill_workspace_bytes(rows, k, nshards);
  EXL3_CHECK_ARG(workspace && workspace_bytes >= need, "exl3_linear_prefill: workspace %zu bytes, need %zu",
                 workspace_bytes, need);
  GemmShards sa{};
  int col = 0, blk = 0;
  for (int s = 0; s < nshards; s++) {
    const exl3_shard& sh = shards_host[s];
    EXL3_CHECK_ARG(sh.trellis && sh.suh && sh.svh, "shard %d: null tensor pointer", s);
    EXL3_CHECK_ARG(sh.n > 0 && sh.n % 128 == 0, "shard %d: n = %d is not a positive multiple of 128", s, sh.n);
    EXL3_CHECK_ARG((int64_t)k * sh.n * K / 8 <= INT32_MAX, "shard %d: trellis exceeds the 2 GiB buffer range", s);
    sa.trellis[s] = static_cast<const uint32_t*>(sh.trellis);
    sa.svh[s] = static_cast<const uint16_t*>(sh.svh);
    sa.xh[s] = static_cast<const uint16_t*>(workspace) + (size_t)s * rows * k;
    sa.tn[s] = sh.n / 16;
    sa.col0[s] = col;
    sa.blk0[s] = blk;
    col += sh.n;
    blk += sh.n / 128;
  }
  sa.blk0[nshards] = blk;
  sa.count = nshards;
  hipStream_t st = as_stream(stream);
  // input rotation of every shard, in fragment order
  for (int s = 0; s < nshards; s++) {
    // one launch per shard keeps the per-shard suh contiguous without a concatenated copy
    if (x_bf16)
      had_in_frag_kernel<true><<<dim3((unsigned)((rows * (k / 128) + 7) / 8)), 256, 0, st>>>(
          x, rows, k, static_cast<const uint16_t*>(shards_host[s].suh), 1,
          static_cast<uint16_t*>(workspace) + (size_t)s * rows * k);
    else
      had_in_frag_kernel<false><<<dim3((unsigned)((rows * (k / 128) + 7) / 8)), 256, 0, st>>>(
          x, rows, k, static_cast<const uint16_t*>(shards_host[s].suh), 1,
          static_cast<uint16_t*>(workspace) + (size_t)s * rows * k);
    EXL3_CHECK_LAUNCH();
  }
  const dim3 grid(blk, (rows + kBM - 1) / kBM);
  static const int stages = [] {
    const char* e = getenv("EXL3_GEMM_STAGES");
    return e && atoi(e) == 4 ? 4 : 3;
  }();
  bool ok;
#define EXL3_GEMM_LAUNCH(YB, ST)                                                                              \
  ok = EXL3_GEMM_DISPATCH(K, codebook, gemm_kernel<kK, kCB, YB, ST><<<grid, kGemmThreads,                    \
                                                                    gemm_lds_bytes<kK, ST>(), st>>>(         \
                                          sa, rows, k, y, col, 1))
  if (y_bf16) {
    if (stages == 3) EXL3_GEMM_LAUNCH(true, 3); else EXL3_GEMM_LAUNCH(true, 4);
  } else {
    if (stages == 3) EXL3_GEMM_LAUNCH(false, 3); else EXL3_GEMM_LAUNCH(false, 4);
  }
#undef EXL3_GEMM_LAUNCH
  if (!ok) return set_error(EXL3_ERR_INVALID, "exl3_linear_prefill: unsupported K/codebook");
  EXL3_CHECK_LAUNCH();
  return EXL3_OK;
}
