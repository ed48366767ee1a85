// EXL3 prefill: fused decode-GEMM on gfx950 MFMA (v_mfma_f32_16x16x32_f16), y = Had(xh @ W_inner) * svh.
//
// Reference semantics: the reference's prefill is decode-to-HBM + cuBLAS between its rotation launches
// (cuda/src/sglang_exl3/runtime/ops.py:36-59); the fused Marlin path serves < 256 rows
// (exl3_marlin_template.h).  Here the weights are decoded into LDS inside the GEMM and never reach HBM.
//
// Operands
//   A: xh in "fragment order", k-step major: the rotated activations with k permuted inside every 32-wide block so
//      that the 8 halves one MFMA lane needs are contiguous, and the blocks of one k-step stored together:
//      xh_f[b][m][8q + 4tr + e] = xh[m][32b + 16tr + r(q, e)], r(q, e) = 2q + (e & 1) + 8(e >> 1) (written by
//      had_in_frag_kernel).  One k-step of 256 rows is one contiguous 16 KB run: the GEMM's loads use whole lines.
//   B: the trellis.  A k-step covers 32 rows = 2 tile rows.  The lane-geometry decode of exl3_device.hpp gives lane
//      (c, j) of a tile the 4 weights of column c at rows r(j, 0..3); tile row tr of the k-step supplies halves
//      4tr..4tr+3 of the lane's 8-half B fragment.  A and B then agree on the k order of every MFMA.
//
// Tiling: workgroup 256 rows x 256 columns (two output rotation blocks; a shard of an odd number of 128-column blocks
// ends in a half tile), 8 waves as 2 x 4, wave tile 128 x 64 (8 x 4 MFMA 16x16x32 tiles, 128 fp32 accumulators per
// lane).  135 KB of LDS: one workgroup per CU, CUs tiles at once.
//
// Work decomposition (1-D grid of work items, dispatched in order): tiles are numbered column block fastest, so
// consecutive workgroups share their A rows in L2.  When the tile count is not a multiple of the machine's
// workgroup slots, the last partial round and one full round before it (stream-K tiles) are shared out as equal runs
// of k-steps over one workgroup per slot: a run crosses tile boundaries, so every workgroup finishes after the same
// number of k-steps.  The stream-K workgroups are dispatched first, then one workgroup per remaining whole tile.  A
// run's first and last segments can cover part of a tile: such a segment stores its fp32 accumulators as a partial,
// and the last of the tile's workgroups to arrive (a per-tile counter in the workspace's counter region) sums the
// tile's partials in workgroup order (deterministic, independent of arrival order), then runs the same epilogue as a
// whole tile and resets the counter.  When whole rounds would finish sooner (the partials cost about a quarter of a
// tile-time), every tile is a whole-tile item.
//
// Pipeline: direct-to-LDS 16-byte buffer loads (no VGPR staging) into two 3-slot rings, one for A (per k-step each
// wave loads 2 pieces, one m-block of 64 lanes x 16 B each: a lane's 16 bytes land exactly where its MFMA A fragment
// lives) and one for the trellis bits (each wave loads its 4 tiles of the k-step).  A bundle of loads holds A of step
// b and the bits of step b+1 and is issued two steps before its A is used, so every load has two steps of flight.
// The compiler does not order LDS-DMA writes before LDS reads, so the waits are explicit (vmcnt), and one barrier per
// k-step publishes the other waves' pieces and decoded weights.  Each k-step runs its 32 MFMAs per wave next to the
// decode of the following k-step (32 tiles per workgroup, 4 per wave, into a double-buffered fp16 B fragment area),
// so VALU decode work overlaps matrix work.
#include <stdlib.h>

#include <algorithm>

#include "exl3_api.hpp"
#include "exl3_device.hpp"

namespace exl3 {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBM = 256, kBN = 256, kBK = 32;
constexpr int kGemmWaves = 8, kGemmThreads = kGemmWaves * 64;
constexpr int kAStage = kBM * kBK * 2;            // 16 KB: [16 m-blocks][64 lanes][8 halves]
constexpr int kBStage = kBN * kBK * 2;            // 16 KB: [16 n-blocks][64 lanes][8 halves]
constexpr int kBitsStage = kGemmWaves * 64 * 16;  // 8 KB: per wave 64 lanes x 16 B (its 4 tiles of a k-step)
constexpr int kRing = 3;                          // A and bits ring slots
constexpr int kCStride = kBN + 8;                 // epilogue fp16 C tile row stride (halves)
constexpr int kCoherentStore = 1 << 4;            // buffer cache policy sc1: device-scope coherent access
constexpr int kPartialBytes = kBM * kBN * 4;      // one fp32 partial tile
constexpr int kLoadRegion = kRing * (kAStage + kBitsStage) + 2 * kBStage;
constexpr int kGemmLds = kLoadRegion > kBM * kCStride * 2 ? kLoadRegion : kBM * kCStride * 2;  // 135 KB: 1 per CU

struct GemmShards {
  const uint32_t* trellis[EXL3_MAX_SHARDS];
  const uint16_t* svh[EXL3_MAX_SHARDS];
  const uint16_t* xh[EXL3_MAX_SHARDS];  // per-shard rotated activations, fragment order, k-step major
  int tn[EXL3_MAX_SHARDS];              // tile columns of the shard
  int layout[EXL3_MAX_SHARDS];          // EXL3_LAYOUT_STORED / EXL3_LAYOUT_BLOCKS
  int col0[EXL3_MAX_SHARDS];            // first output column of the shard
  int ct0[EXL3_MAX_SHARDS + 1];         // first 256-column tile of the shard (cumulative); ct0[count] = total
  int count;
};

// The work decomposition of one launch (see the header comment).
struct GemmPlan {
  int nct;         // 256-column tiles per row block
  int sk_tiles;    // tiles 0 .. sk_tiles-1 are shared out by runs of k-steps among the stream-K workgroups
  int groups;      // stream-K workgroups: grid items 0 .. groups-1; items groups.. are whole tiles sk_tiles..
  int ksteps;      // k / 32
  float* partial;  // [groups][2 segments][8 waves][8][4][64 lanes] float4: a workgroup's first / last segment
  int* counters;   // [sk_tiles], zero between calls
};

// Stream-K: workgroup g owns the global k-steps [sk_start(g), sk_start(g + 1)) of the sk_tiles * ksteps steps (tile t
// holds steps t * ksteps ..); sk_owner(q) is the workgroup whose run holds step q.
__host__ __device__ __forceinline__ int64_t sk_start(const GemmPlan& p, int g) {
  return (int64_t)p.sk_tiles * p.ksteps * g / p.groups;
}
__host__ __device__ __forceinline__ int sk_owner(const GemmPlan& p, int64_t q) {
  const int64_t W = (int64_t)p.sk_tiles * p.ksteps;
  return (int)(((q + 1) * p.groups + W - 1) / W) - 1;
}

// lds_barrier() (exl3_device.hpp) between k-steps: the direct-to-LDS writes are waited for explicitly (waitcnt_vm)
// before each barrier.

template <int K>
__host__ __device__ constexpr int gemm_chunks() { return 4 * 32 * K / 16; }  // 16-byte pieces of a wave's 4 tiles

// per-shard input scales of one prefill call (the rotation runs every shard in one launch)
struct ShardSuh {
  const uint16_t* suh[EXL3_MAX_SHARDS];
};

// Shard s of a rotation unit and its suh (a select over the few shards keeps the pointer in scalar registers)
__device__ __forceinline__ const uint16_t* unit_suh(const ShardSuh& su_all, int s) {
  return s == 0 ? su_all.suh[0] : s == 1 ? su_all.suh[1] : s == 2 ? su_all.suh[2] : su_all.suh[3];
}

// The 8 values of a 16-lane unit's lane (positions 8t .. 8t+7) as 4 fp16 pairs: fp16(Had(fp16(x) * suh)) (ROT), or
// x as given (fp16 rows)
template <bool X_BF16, bool ROT>
__device__ __forceinline__ void frag16_values(u32x4_t xv, u32x4_t sv, uint32_t d[4]) {
  if constexpr (!ROT) {
#pragma unroll
    for (int q = 0; q < 4; q++) d[q] = xv[q];
    return;
  }
  const half8_t sc = __builtin_bit_cast(half8_t, sv);
  float f[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const uint32_t w = xv[i >> 1];
    const uint16_t raw = (uint16_t)((i & 1) ? w >> 16 : w & 0xFFFF);
    const _Float16 v = X_BF16 ? (_Float16)bf16_to_f32(raw) : __builtin_bit_cast(_Float16, raw);
    f[i] = (float)(_Float16)(v * sc[i]);
  }
#pragma unroll
  for (int h = 1; h < 8; h <<= 1)
#pragma unroll
    for (int i = 0; i < 8; i++)
      if (!(i & h)) {
        const float a = f[i], bb = f[i + h];
        f[i] = a + bb;
        f[i + h] = a - bb;
      }
  had_stage<1>(f[0], f[1], f[2], f[3]);
  had_stage<1>(f[4], f[5], f[6], f[7]);
  had_stage<2>(f[0], f[1], f[2], f[3]);
  had_stage<2>(f[4], f[5], f[6], f[7]);
  had_stage<4>(f[0], f[1], f[2], f[3]);
  had_stage<4>(f[4], f[5], f[6], f[7]);
  had_stage<8>(f[0], f[1], f[2], f[3]);
  had_stage<8>(f[4], f[5], f[6], f[7]);
#pragma unroll
  for (int q = 0; q < 4; q++)
    d[q] = __builtin_bit_cast(uint32_t, half2_t{had_scale_f16(f[2 * q]), had_scale_f16(f[2 * q + 1])});
}

// The same rotation with 16 lanes per 128-value (row, block) unit: lane t holds positions 8t .. 8t+7, read with one
// 16-byte load of x and one of suh (x and every suh 16-byte aligned; the host checks).  The butterfly runs the stages
// of had128_x4 in the same order on the same pairs -- h = 1, 2, 4 inside the lane (h = 4 was the lane-xor-1 stage
// of the 4-per-lane form: lower = a + b, upper = a - b, the same sums), then lane xor 1, 2, 4, 8 for h = 8 .. 64 --
// so the rotated values are bit-identical.  Fragment order: lane t (a = t & 3) holds, per q = 0..3, the slot pair
// (q, tr = a >> 1, e = 2 (a & 1) + 0/1); lanes a and a ^ 1 swap two dwords (DPP) so that each stores two 8-byte
// slot groups (q, tr) whole.  A 16-lane group takes U consecutive units with all loads issued first.
// ROT = false: the fp16 rows are taken as given (no sign vector, no butterfly, no rounding) and only put in fragment
// order (the rotation-free GEMM of exl3_gemm_rotated).
template <bool X_BF16, int U, bool ROT = true>
__global__ __launch_bounds__(256) void had_in_frag16_kernel(const void* __restrict__ x, int rows, int k,
                                                            ShardSuh su_all, int shards, uint16_t* __restrict__ xh) {
  const int kb = k >> 7;
  const int units = shards * rows * kb;
  const int u0 = (blockIdx.x * 16 + (threadIdx.x >> 4)) * U;
  if (u0 >= units) return;  // the whole 16-lane row: the DPP stages below stay inside rows of 16 lanes
  const int t = threadIdx.x & 15;
  u32x4_t xv[U], sv[U];
#pragma unroll
  for (int j = 0; j < U; j++) {
    const int u = min(u0 + j, units - 1);  // past the end: a repeat of the last unit, not stored
    const int s = u / (rows * kb), rem = u - s * rows * kb, r = rem / kb, b = rem - r * kb;
    const int kk = b * 128 + 8 * t;
    xv[j] = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(x) + (size_t)r * k + kk);
    sv[j] = ROT ? *reinterpret_cast<const u32x4_t*>(unit_suh(su_all, s) + kk) : u32x4_t{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int j = 0; j < U; j++) {
    const int u = u0 + j;
    if (u >= units) break;
    const int s = u / (rows * kb), rem = u - s * rows * kb, r = rem / kb, b = rem - r * kb;
    uint32_t d[4];  // d[q] = fp16 pair (positions 2q, 2q+1 of the lane)
    frag16_values<X_BF16, ROT>(xv[j], sv[j], d);
    const bool low = (t & 1) == 0;
    // lane a (even) stores q = 0, 2 as [own, partner's]; lane a + 1 stores q = 1, 3 as [partner's, own]
    const uint32_t g0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)(low ? d[1] : d[0]), 0xB1, 0xF, 0xF, false);
    const uint32_t g1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)(low ? d[3] : d[2]), 0xB1, 0xF, 0xF, false);
    const uint2_t o0 = low ? uint2_t{d[0], g0} : uint2_t{g0, d[1]};
    const uint2_t o1 = low ? uint2_t{d[2], g1} : uint2_t{g1, d[3]};
    const int a = t & 3, blk32 = t >> 2, tr = a >> 1, q0 = low ? 0 : 1;
    uint16_t* dst = xh + (size_t)s * rows * k + ((size_t)(b * 4 + blk32) * rows + r) * 32 + tr * 4;
    *reinterpret_cast<uint2_t*>(dst + q0 * 8) = o0;
    *reinterpret_cast<uint2_t*>(dst + (q0 + 2) * 8) = o1;
  }
}

// The 4 values of a 32-lane unit's lane (positions 4t .. 4t+3) as 2 fp16 pairs: fp16(Had(fp16(x) * suh)) (ROT), or
// x as given (fp16 rows)
template <bool X_BF16, bool ROT>
__device__ __forceinline__ void frag_values(uint2_t xv, uint2_t sv, uint32_t& lo_w, uint32_t& hi_w) {
  if constexpr (!ROT) {
    lo_w = xv.x;
    hi_w = xv.y;
    return;
  }
  _Float16 v[4];
  if constexpr (X_BF16) {
    v[0] = (_Float16)bf16_to_f32((uint16_t)(xv.x & 0xFFFF));
    v[1] = (_Float16)bf16_to_f32((uint16_t)(xv.x >> 16));
    v[2] = (_Float16)bf16_to_f32((uint16_t)(xv.y & 0xFFFF));
    v[3] = (_Float16)bf16_to_f32((uint16_t)(xv.y >> 16));
  } else {
    const half4_t raw = __builtin_bit_cast(half4_t, xv);
    v[0] = raw.x; v[1] = raw.y; v[2] = raw.z; v[3] = raw.w;
  }
  const half4_t sc = __builtin_bit_cast(half4_t, sv);
  float f0 = (float)(_Float16)(v[0] * sc.x), f1 = (float)(_Float16)(v[1] * sc.y);
  float f2 = (float)(_Float16)(v[2] * sc.z), f3 = (float)(_Float16)(v[3] * sc.w);
  had128_x4(f0, f1, f2, f3);
  lo_w = __builtin_bit_cast(uint32_t, half2_t{had_scale_f16(f0), had_scale_f16(f1)});
  hi_w = __builtin_bit_cast(uint32_t, half2_t{had_scale_f16(f2), had_scale_f16(f3)});
}

// rotated activations in fragment order: xh_f[s*rows + r][k] for shard s (see the header comment).  A half-wave
// takes U consecutive 128-value (row, block) units, issues all their loads first (one round of load latency per
// half-wave instead of one per unit), then rotates and stores each; lane t holds positions 4t .. 4t+3 of a block.
// U = 4 from 2^17 units (measured at 8192 rows: 60 -> 52 us; equal at 2048 rows, slower at 512 rows).
template <bool X_BF16, int U, bool ROT = true>
__global__ __launch_bounds__(256) void had_in_frag_kernel(const void* __restrict__ x, int rows, int k, ShardSuh su_all,
                                                          int shards, uint16_t* __restrict__ xh) {
  const int kb = k >> 7;
  const int units = shards * rows * kb;
  const int u0 = (blockIdx.x * 8 + (threadIdx.x >> 5)) * U;
  if (u0 >= units) return;
  const int t = threadIdx.x & 31;
  uint2_t xv[U], sv[U];
#pragma unroll
  for (int j = 0; j < U; j++) {
    const int u = min(u0 + j, units - 1);  // past the end: a repeat of the last unit, not stored
    const int s = u / (rows * kb), rem = u - s * rows * kb, r = rem / kb, b = rem - r * kb;
    const int kk = b * 128 + 4 * t;
    xv[j] = *reinterpret_cast<const uint2_t*>(static_cast<const uint16_t*>(x) + (size_t)r * k + kk);
    sv[j] = ROT ? *reinterpret_cast<const uint2_t*>(unit_suh(su_all, s) + kk) : uint2_t{0u, 0u};
  }
#pragma unroll
  for (int j = 0; j < U; j++) {
    const int u = u0 + j;
    if (u >= units) break;
    const int s = u / (rows * kb), rem = u - s * rows * kb, r = rem / kb, b = rem - r * kb;
    uint32_t lo_w, hi_w;  // fp16 pairs: positions 4t, 4t+1 and 4t+2, 4t+3
    frag_values<X_BF16, ROT>(xv[j], sv[j], lo_w, hi_w);
    // k-step major: the 32 halves of row r in k-step kt (one MFMA k-block) at [kt][r][32], so that one k-step of a
    // row block is one contiguous run and every 16-row A piece of the GEMM reads whole cache lines.  Inside a
    // 32-block, slot (q, tr, e) holds position 16 tr + 2q + (e & 1) + 8 (e >> 1).  With a = t & 3, lane t's positions
    // are 16 tr + 4a + i: lanes a < 2 hold e = 0, 1 of q = 2a (i < 2) and of q = 2a + 1 (i >= 2), lanes a + 2 the
    // e = 2, 3 of the same q.  The pair (a, a + 2) swaps one dword (a DPP quad permute) and each lane stores its q's
    // 4 slots as one 8-byte word.
    const bool low = (t & 2) == 0;
    const uint32_t got = (uint32_t)__builtin_amdgcn_mov_dpp((int)(low ? hi_w : lo_w), 0x4E, 0xF, 0xF, false);
    const uint2_t out = low ? uint2_t{lo_w, got} : uint2_t{got, hi_w};
    const int blk32 = t >> 3, tr = (t >> 2) & 1, q = 2 * (t & 1) + (low ? 0 : 1);
    uint16_t* dst = xh + (size_t)s * rows * k;
    *reinterpret_cast<uint2_t*>(dst + ((size_t)(b * 4 + blk32) * rows + r) * 32 + q * 8 + tr * 4) = out;
  }
}

// One segment of work: k-steps [kt0, kt1) of tile `tile`.  seg < 0: the whole tile, straight to the epilogue;
// seg = 0 / 1: a stream-K segment at the start / end of workgroup `item`'s run, stored as that partial slot; the
// last of the tile's workgroups to arrive sums every partial of the tile in workgroup order and runs the epilogue.
// FEW (a launch of fewer than 256 rows, one row block): the MFMAs and A-fragment reads of 16-row blocks past M are
// skipped (their accumulators stay zero and are never stored); every load, decode and barrier is unchanged.
template <int K, int CB, bool Y_BF16, bool FEW>
__device__ __forceinline__ void gemm_segment(const GemmShards& sa, const GemmPlan& plan, int M, int k,
                                             void* __restrict__ y, int n_total, int rotate_out, uint8_t* lds,
                                             int item, int tile, int kt0, int kt1, int seg) {
  constexpr int CHUNKS = gemm_chunks<K>();
  static_assert(CHUNKS <= 64, "one gather per wave per k-step");
  uint8_t* a_ring = lds;                             // [kRing][kAStage]
  uint8_t* bits_ring = lds + kRing * kAStage;        // [kRing][8 waves][64 lanes][16 B]
  uint8_t* b_lds = bits_ring + kRing * kBitsStage;   // [2][kBStage] decoded B fragments

  const int ct = tile % plan.nct, mblk = tile / plan.nct;
  int s = 0;
#pragma unroll
  for (int i = 1; i < EXL3_MAX_SHARDS; i++)
    if (i < sa.count && ct >= sa.ct0[i]) s = i;
  const int tn = sa.tn[s];
  const int tc0 = (ct - sa.ct0[s]) * 16;  // first tile column of this tile in the shard
  const int ntc = min(16, tn - tc0);      // tile columns present: 16, or 8 at the end of a shard of odd 128-blocks
  const int col0 = sa.col0[s] + tc0 * 16;  // first output column
  const int row0 = mblk * kBM;

  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l = tid & 63;
  const int wm = w >> 2, wn = w & 3;  // wave tile: rows 128 wm .., columns 64 wn ..
  const int c = l & 15, j = l >> 4;
  const bool mfma_wave = 4 * wn < ntc;  // wave-uniform: its 64 columns exist
  // 16-row blocks of the wave tile that hold rows below M (wave-uniform; all 8 unless FEW)
  const int live_mi = FEW ? max(0, min(8, (M - row0 - wm * 128 + 15) / 16)) : 8;

  // B: wave w loads and decodes tile row btr = w >> 2, tile columns btc .. btc+3 (btc = 4 (w & 3)) of every k-step;
  // past the end of a half tile it re-reads the tile's first columns (in range, decoded into n-blocks nobody reads)
  const int btr = w >> 2, btc = 4 * (w & 3);
  const int tile_bytes = 32 * K;
  const int row_bytes = tn * tile_bytes;
  const __amdgpu_buffer_rsrc_t brsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)sa.trellis[s], (short)0, (k >> 4) * row_bytes, 0x00020000);
  // STORED: the 4 tiles are adjacent in their tile row (+ tile row * row_bytes); BLOCKS: 8 tiles apart inside the
  // unit of the column block (+ the unit of the 128-row block and the row inside it, per k-step)
  const bool blocks = sa.layout[s] == EXL3_LAYOUT_BLOCKS;
  const int bj0 = tc0 + (btc < ntc ? btc : 0), bL = min(l, CHUNKS - 1);
  const int bgoff = blocks ? ((bj0 >> 3) * (k >> 7) * 64 + ((bj0 & 7) + bL / (2 * K)) * 8) * tile_bytes +
                                 (bL % (2 * K)) * 16
                           : bj0 * tile_bytes + bL * 16;
  const LaneGeo g = lane_geo<K>(c, j);

  // A: wave w loads m-blocks 2w, 2w+1; lane l of a piece = row (l % 16) of the m-block, k-chunk l / 16.  Rows past
  // M re-read row M-1 (finite, only feeds discarded C rows).
  const uint16_t* xh = sa.xh[s];
  const __amdgpu_buffer_rsrc_t arsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)xh, (short)0, M * k * 2, 0x00020000);
  int aoff[2];
#pragma unroll
  for (int q = 0; q < 2; q++) {
    const int row = min(row0 + (2 * w + q) * 16 + c, M - 1);
    aoff[q] = (row * 32 + j * 8) * 2;  // + k-step * M * 64 bytes
  }

  // Loads come in bundles: bundle b = A of step b + trellis bits of step b+1 (3 loads per wave; past the end, steps
  // clamp to the last one: in range, never used).  Step i of the item (k-step kt0 + i) reads A slot i % 3, decodes
  // the bits of step i+1 from bits slot (i+1) % 3, and issues bundle i+2, so every load has two steps of flight.
  const int nk = kt1 - kt0;  // >= 1
  // (the k-step argument kt is clamped by the caller: no device-only calls inside these lambdas, whose host-side
  // instantiation would otherwise suppress the kernel's host stub)
  auto issue_a = [&](int i, int kt) {
    uint8_t* st = a_ring + (i % kRing) * kAStage;
#pragma unroll
    for (int q = 0; q < 2; q++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (__attribute__((address_space(3))) void*)(st + (2 * w + q) * 1024),
                                               16, aoff[q], kt * M * kBK * 2, 0, 0);
  };
  auto issue_bits = [&](int i, int kt) {
    uint8_t* st = bits_ring + (i % kRing) * kBitsStage + w * 1024;
    const int tr = 2 * kt + btr;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(brsrc, (__attribute__((address_space(3))) void*)st, 16, bgoff,
                                             blocks ? ((tr >> 3) * 64 + (tr & 7)) * tile_bytes : tr * row_bytes, 0,
                                             0);
  };
  // this wave's trellis words of step i (bits slot i % 3)
  auto read_bits = [&](int i, uint32_t (&bw)[4][2]) {
    const uint32_t* tw = reinterpret_cast<const uint32_t*>(bits_ring + (i % kRing) * kBitsStage + w * 1024);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      bw[t][0] = tw[t * 8 * K + g.dw0];
      bw[t][1] = tw[t * 8 * K + g.dw1];
    }
  };
  // decoded weights of this wave's 4 tiles into decoded-B buffer i & 1: n-block btc + t, lane (c, j), halves
  // 4 btr .. +3
  auto write_b = [&](int i, const uint32_t (&bw)[4][2]) {
    uint8_t* dst = b_lds + (i & 1) * kBStage;
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const half4_t v = decode_group<K, CB, false>(bw[t][0], bw[t][1], g);  // stored to LDS: no MFMA wait states
      *reinterpret_cast<half4_t*>(dst + (((btc + t) * 64 + l) * 16) + btr * 8) = v;
    }
  };

  float4_t acc[8][4];
#pragma unroll
  for (int mi = 0; mi < 8; mi++)
#pragma unroll
    for (int jj = 0; jj < 4; jj++) acc[mi][jj] = float4_t{0.f, 0.f, 0.f, 0.f};

  issue_bits(0, kt0);
  issue_a(0, kt0);
  issue_bits(1, kt0 + min(1, nk - 1));
  issue_a(1, kt0 + min(1, nk - 1));
  issue_bits(2, kt0 + min(2, nk - 1));
  {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(6));  // the bits of step 0 in (bundles 0 and 1 may be in flight)
    lds_barrier();
    uint32_t bw[4][2];
    read_bits(0, bw);
    write_b(0, bw);
  }

  for (int i = 0; i < nk; i++) {
    // bundle i in (A of step i, bits of step i+1); bundle i+1 may still be in flight.  The barrier makes every wave's
    // pieces and decoded weights of step i visible and retires every read of step i-1, freeing A slot (i-1) % 3,
    // bits slot i % 3 and decoded-B buffer (i+1) & 1.
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(3));
    lds_barrier();
    issue_a(i + 2, kt0 + min(i + 2, nk - 1));
    issue_bits(i + 3, kt0 + min(i + 3, nk - 1));
    uint32_t bw[4][2];
    read_bits(i + 1, bw);
    if (mfma_wave) {
      const half8_t* af = reinterpret_cast<const half8_t*>(a_ring + (i % kRing) * kAStage) + (wm * 8) * 64 + l;
      const half8_t* bf = reinterpret_cast<const half8_t*>(b_lds + (i & 1) * kBStage) + (wn * 4) * 64 + l;
      half8_t bv[4], av[8];
#pragma unroll
      for (int jj = 0; jj < 4; jj++) bv[jj] = bf[jj * 64];
#pragma unroll
      for (int mi = 0; mi < 8; mi++)
        if (mi < live_mi) av[mi] = af[mi * 64];
#pragma unroll
      for (int mi = 0; mi < 8; mi++)
        if (mi < live_mi)
#pragma unroll
          for (int jj = 0; jj < 4; jj++)
            acc[mi][jj] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[mi], bv[jj], acc[mi][jj], 0, 0, 0);
    }
    // the next step's weights (at the last step: a stale but valid stage into a buffer nobody reads)
    write_b(i + 1, bw);
    // interleave: the fragment and trellis-word reads first, then one MFMA per two VALU ops of the decode, then its
    // LDS writes
    __builtin_amdgcn_sched_group_barrier(0x100, 20, 0);  // DS reads
#pragma unroll
    for (int q = 0; q < 32; q++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
    }
    __builtin_amdgcn_sched_group_barrier(0x200, 4, 0);  // DS writes
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // drain the trailing re-reads of every wave before LDS is reused
  __syncthreads();

  // ---- stream-K segment: store the partial (16-byte stores with device-scope coherence: the reader may sit on
  // another XCD, whose L2 is not this one's); the tile's last workgroup to arrive sums all of the tile's partials in
  // workgroup order (deterministic, independent of arrival order)
  if (seg >= 0) {
    __shared__ int last_flag;
    const __amdgpu_buffer_rsrc_t prsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)plan.partial, (short)0, plan.groups * 2 * kGemmWaves * 32 * 64 * 16, 0x00020000);
    auto slot_off = [&](int g, int sl) { return (((g * 2 + sl) * kGemmWaves + w) * 32 * 64 + l) * 16; };
    const int mine = slot_off(item, seg);
    // only the 16-row blocks that hold output rows (rows >= M and columns past a half tile are never stored), so a
    // few-row prefill moves a fraction of the 256 KB per partial
    const int live_rows = mfma_wave ? M - row0 - wm * 128 : 0;  // wave-uniform (mi * 16 < live_rows: mi < live_mi)
#pragma unroll
    for (int mi = 0; mi < 8; mi++)
      if (mi * 16 < live_rows)
#pragma unroll
        for (int jj = 0; jj < 4; jj++)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[mi][jj]), prsrc,
                                               mine + (mi * 4 + jj) * 64 * 16, 0, kCoherentStore);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));  // this thread's partial stores are at the coherence point
    __syncthreads();
    const int64_t q0 = (int64_t)tile * plan.ksteps;
    const int g_first = sk_owner(plan, q0), g_last = sk_owner(plan, q0 + plan.ksteps - 1);
    if (tid == 0) {
      const int prev = __hip_atomic_fetch_add(&plan.counters[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_flag = prev == g_last - g_first;
    }
    __syncthreads();
    if (!last_flag) return;
    // the sum runs in workgroup order from g_first; when this workgroup is g_first (the usual last arrival: the
    // tile is the end of its run) its registers are that first term, bit for bit what it stored
    int g = g_first;
    if (item == g_first) {
      g++;
    } else {
#pragma unroll
      for (int mi = 0; mi < 8; mi++)
#pragma unroll
        for (int jj = 0; jj < 4; jj++) acc[mi][jj] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
    for (; g <= g_last; g++) {
      const int src = slot_off(g, sk_start(plan, g) >= q0 ? 0 : 1);  // the tile is g's first segment or its last
#pragma unroll
      for (int mi = 0; mi < 8; mi++)
        if (mi * 16 < live_rows)
#pragma unroll
          for (int jj = 0; jj < 4; jj++)
            acc[mi][jj] += __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                          prsrc, src + (mi * 4 + jj) * 64 * 16, 0, kCoherentStore));
    }
    if (tid == 0) __hip_atomic_store(&plan.counters[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- epilogue: the whole fp16 C tile (256 x 256, rounded once from fp32) goes to LDS, then each thread rotates
  // one 128-column half-row in registers -- the 128-point butterfly of had128_x4 with the same pairings and order
  // (h = 1, 2, 4, ..., 64; lower = a + b, upper = a - b, fp32), so results are identical -- scales by svh (fp16
  // product) and stores it.  Per-row register butterflies have no cross-lane latency: a lane-parallel rotation chains
  // five LDS permutes per row.
  _Float16* cl = reinterpret_cast<_Float16*>(lds);
  if (mfma_wave) {
#pragma unroll
    for (int mi = 0; mi < 8; mi++)
#pragma unroll
      for (int jj = 0; jj < 4; jj++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int m = wm * 128 + mi * 16 + 4 * j + r;
          const int n = wn * 64 + jj * 16 + c;
          cl[m * kCStride + n] = (_Float16)acc[mi][jj][r];
        }
  }
  __syncthreads();
  const int er = tid & (kBM - 1), eh = tid / kBM;  // row and 128-column half of this thread
  const int m = row0 + er;
  if (m < M && 8 * eh < ntc) {
    const half8_t* src = reinterpret_cast<const half8_t*>(cl + er * kCStride + eh * 128);
    float v[128];
#pragma unroll
    for (int q = 0; q < 16; q++) {
      const half8_t h = src[q];
#pragma unroll
      for (int e = 0; e < 8; e++) v[8 * q + e] = (float)h[e];
    }
    const int col = col0 + eh * 128;
    const half8_t* sv8 = reinterpret_cast<const half8_t*>(sa.svh[s] + (col - sa.col0[s]));
    uint16_t* yr = static_cast<uint16_t*>(y) + (size_t)m * n_total + col;
    if (rotate_out) {
#pragma unroll
      for (int hs = 1; hs < 128; hs <<= 1)
#pragma unroll
        for (int p = 0; p < 128; p++)
          if (!(p & hs)) {
            const float a = v[p], bb = v[p + hs];
            v[p] = a + bb;
            v[p + hs] = a - bb;
          }
    }
#pragma unroll
    for (int q = 0; q < 16; q++) {
      half8_t o;
      if (rotate_out) {
        const half8_t sv = sv8[q];
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = had_scale_f16(v[8 * q + e]) * sv[e];
      } else {
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = (_Float16)v[8 * q + e];
      }
      if constexpr (Y_BF16) {
        u32x4 ob;
#pragma unroll
        for (int e = 0; e < 4; e++)
          ob[e] = (uint32_t)f32_to_bf16((float)o[2 * e]) | ((uint32_t)f32_to_bf16((float)o[2 * e + 1]) << 16);
        *reinterpret_cast<u32x4*>(yr + 8 * q) = ob;
      } else {
        *reinterpret_cast<half8_t*>(yr + 8 * q) = o;
      }
    }
  }
  __syncthreads();  // the C tile in LDS is read before the next segment's loads overwrite it
}

// Grid: the stream-K workgroups first (each walks the segments of its run of k-steps), then one workgroup per
// remaining whole tile.
template <int K, int CB, bool Y_BF16, bool FEW>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(GemmShards sa, GemmPlan plan, int M, int k,
                                                             void* __restrict__ y, int n_total, int rotate_out) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int item = blockIdx.x;
  if (item >= plan.groups) {
    gemm_segment<K, CB, Y_BF16, FEW>(sa, plan, M, k, y, n_total, rotate_out, lds, item,
                                plan.sk_tiles + (item - plan.groups), 0, plan.ksteps, -1);
    return;
  }
  const int64_t a = sk_start(plan, item), b = sk_start(plan, item + 1);
  for (int64_t q = a; q < b;) {
    const int t = (int)(q / plan.ksteps);
    const int64_t q0 = (int64_t)t * plan.ksteps;
    const int kt0 = (int)(q - q0), kt1 = (int)(b - q0 < plan.ksteps ? b - q0 : plan.ksteps);
    const bool whole = kt0 == 0 && kt1 == plan.ksteps;
    gemm_segment<K, CB, Y_BF16, FEW>(sa, plan, M, k, y, n_total, rotate_out, lds, item, t, kt0, kt1,
                                whole ? -1 : (q == a ? 0 : 1));
    q = q0 + kt1;
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



// Concurrent workgroups of the device (one per CU: 135 KB of LDS), per device, queried once.
static int gemm_slots() {
  static int slots[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (slots[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    slots[dev] = cus;
  }
  return slots[dev];
}

struct GemmLayout {
  int nct, sk_tiles, groups, ksteps, tiles;
  size_t xh_bytes, partial_off, total;
};

// 256-column tiles never straddle shards (each shard reads its own rotated activations): a shard of an odd number
// of 128-column blocks ends in a half tile
static int gemm_col_tiles(const int* shard_n, int nshards) {  // tiles of 256 columns over all shards
  int t = 0;
  for (int s = 0; s < nshards; s++) t += (shard_n[s] / 128 + 1) / 2;
  return t;
}

// Whole tiles in rounds of the machine, except the last (partial) round plus one full round before it (when there
// is one), which are shared out by runs of k-steps over one workgroup per slot (stream-K): every workgroup then
// finishes after the same number of k-steps, 1 to 2 tiles' worth, and writes at most two partial tiles.  A run keeps
// >= 8 k-steps so the pipeline start-up stays small against its work.  Whole rounds only, when they are sooner.
static GemmLayout gemm_layout(int rows, int k, int nct, int nshards) {
  GemmLayout L{};
  L.nct = nct;
  L.ksteps = k / kBK;
  L.tiles = ((rows + kBM - 1) / kBM) * nct;
  const int slots = gemm_slots();
  const int rounds = L.tiles / slots, rem = L.tiles - rounds * slots;
  if (rem > 0) {
    const int sk = rounds >= 1 ? rem + slots : rem;
    // in tile-times: whole tiles only take rounds + 1; stream-K takes the whole rounds left plus sk / slots plus the
    // partial tiles' store, reload and wait (measured ~0.25 of a tile-time at 5120 -> 17408: 512 rows 156 us against
    // 183 us whole, 768 rows 211 against 199)
    const double whole = rounds + 1, shared = (double)(L.tiles - sk) / slots + (double)sk / slots + 0.25;
    if (shared < whole) {
      L.sk_tiles = sk;
      L.groups = (int)std::max<int64_t>(1, std::min<int64_t>(slots, (int64_t)sk * L.ksteps / 8));
    }
  }
  // [counter region (fixed place and size)][rotated activations][partials: 2 per stream-K workgroup]
  L.xh_bytes = ((size_t)nshards * rows * k * 2 + 255) & ~(size_t)255;
  L.partial_off = kCounterBytes + L.xh_bytes;
  L.total = L.partial_off + (size_t)L.groups * 2 * kPartialBytes;
  return L;
}

}  // namespace exl3

using namespace exl3;

extern "C" size_t exl3_prefill_workspace_bytes(int rows, int k, int n_total, int nshards) {
  if (rows <= 0 || k <= 0 || k % 128 || n_total <= 0 || n_total % 128 || nshards < 1 || nshards > EXL3_MAX_SHARDS)
    return 0;
  // the column-tile count depends on how n_total splits into shards (a shard of an odd number of 128-column blocks
  // ends in a half tile): take the largest need over every possible count
  size_t need = 0;
  for (int nct = (n_total / 128 + 1) / 2; nct <= (n_total / 128 + nshards) / 2; nct++)
    need = std::max(need, gemm_layout(rows, k, nct, nshards).total);
  return need;
}

namespace exl3 {

// The input pass (rotation of every shard in fragment order, or with ROT = false the rows as given in fragment order)
// and the decode-GEMM launch of one call; sa holds the shards, its xh pointers into the workspace.
template <bool ROT>
static int launch_prefill(const void* x, bool x_bf16, int rows, int k, GemmShards& sa, const ShardSuh& su,
                          const int* shard_n, int K, int codebook, void* y, bool y_bf16, void* workspace,
                          size_t workspace_bytes, hipStream_t st, const char* what) {
  const int nshards = sa.count;
  const GemmLayout L = gemm_layout(rows, k, gemm_col_tiles(shard_n, nshards), nshards);
  EXL3_CHECK_ARG(workspace && workspace_bytes >= L.total, "%s: workspace %zu bytes, need %zu", what,
                 workspace_bytes, L.total);
  EXL3_CHECK_ARG(L.sk_tiles <= kMaxCounters, "%s: %d stream-K tiles exceed the counter region", what, L.sk_tiles);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  uint16_t* xh = reinterpret_cast<uint16_t*>(ws + kCounterBytes);
  for (int s = 0; s < nshards; s++) sa.xh[s] = xh + (size_t)s * rows * k;
  GemmPlan plan{L.nct, L.sk_tiles, L.groups, L.ksteps, reinterpret_cast<float*>(ws + L.partial_off),
                reinterpret_cast<int*>(ws)};
  int n_total = 0;
  for (int s = 0; s < nshards; s++) n_total += shard_n[s];
  // the input pass: every shard in one launch
  const size_t hunits = (size_t)nshards * rows * (k / 128);
  bool aligned16 = ((uintptr_t)x & 15) == 0;
  if constexpr (ROT)
    for (int s = 0; s < nshards; s++) aligned16 = aligned16 && ((uintptr_t)su.suh[s] & 15) == 0;
  if (aligned16) {
    const int hu = hunits >= (1u << 17) ? 4 : hunits >= (1u << 15) ? 2 : 1;
    const dim3 hgrid((unsigned)((hunits + 16 * hu - 1) / (16 * hu)));
    auto frag = x_bf16 ? (hu == 4 ? had_in_frag16_kernel<true, 4, ROT> : hu == 2 ? had_in_frag16_kernel<true, 2, ROT>
                                                                                 : had_in_frag16_kernel<true, 1, ROT>)
                       : (hu == 4 ? had_in_frag16_kernel<false, 4, ROT> : hu == 2 ? had_in_frag16_kernel<false, 2, ROT>
                                                                                  : had_in_frag16_kernel<false, 1, ROT>);
    frag<<<hgrid, 256, 0, st>>>(x, rows, k, su, nshards, xh);
  } else {
    const int hu = hunits >= (1u << 17) ? 4 : 1;
    const dim3 hgrid((unsigned)((hunits + 8 * hu - 1) / (8 * hu)));
    auto frag = x_bf16 ? (hu == 4 ? had_in_frag_kernel<true, 4, ROT> : had_in_frag_kernel<true, 1, ROT>)
                       : (hu == 4 ? had_in_frag_kernel<false, 4, ROT> : had_in_frag_kernel<false, 1, ROT>);
    frag<<<hgrid, 256, 0, st>>>(x, rows, k, su, nshards, xh);
  }
  EXL3_CHECK_LAUNCH();
  const dim3 grid((unsigned)(L.groups + L.tiles - L.sk_tiles));
  bool ok;
#define EXL3_GEMM_LAUNCH(YB, FEW)                                                                              \
  ok = EXL3_GEMM_DISPATCH(K, codebook, gemm_kernel<kK, kCB, YB, FEW><<<grid, kGemmThreads, kGemmLds, st>>>( \
                                          sa, plan, rows, k, y, n_total, ROT ? 1 : 0))
  const bool few = rows < kBM;  // one row block, mostly rows past M
  if (y_bf16 && few)
    EXL3_GEMM_LAUNCH(true, true);
  else if (y_bf16)
    EXL3_GEMM_LAUNCH(true, false);
  else if (few)
    EXL3_GEMM_LAUNCH(false, true);
  else
    EXL3_GEMM_LAUNCH(false, false);
#undef EXL3_GEMM_LAUNCH
  if (!ok) return set_error(EXL3_ERR_INVALID, "%s: unsupported K/codebook", what);
  EXL3_CHECK_LAUNCH();
  return EXL3_OK;
}

}  // namespace exl3

using namespace exl3;

extern "C" int exl3_linear_prefill(const void* x, int x_bf16, int rows, int k, const exl3_shard* shards_host,
                                   int nshards, int K, int codebook, void* y, int y_bf16, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  EXL3_CHECK_ARG((rows == 0 || (x && y)) && shards_host, "exl3_linear_prefill: null pointer");
  EXL3_CHECK_ARG(valid_bits(K) && valid_cb(codebook), "exl3_linear_prefill: K = %d / codebook = %d", K, codebook);
  EXL3_CHECK_ARG(rows >= 0 && k > 0 && k % 128 == 0, "exl3_linear_prefill: rows = %d, k = %d", rows, k);
  EXL3_CHECK_ARG(nshards >= 1 && nshards <= EXL3_MAX_SHARDS, "exl3_linear_prefill: nshards = %d", nshards);
  if (rows == 0) return EXL3_OK;
  EXL3_CHECK_ARG((int64_t)rows * k * 2 <= INT32_MAX, "exl3_linear_prefill: rows * k too large for one launch");
  GemmShards sa{};
  ShardSuh su{};
  int col = 0, ctl = 0;
  int shard_n[EXL3_MAX_SHARDS];
  for (int s = 0; s < nshards; s++) {
    const exl3_shard& sh = shards_host[s];
    EXL3_CHECK_ARG(sh.trellis && sh.suh && sh.svh, "shard %d: null tensor pointer", s);
    EXL3_CHECK_ARG(sh.n > 0 && sh.n % 128 == 0, "shard %d: n = %d is not a positive multiple of 128", s, sh.n);
    EXL3_CHECK_ARG((int64_t)k * sh.n * K / 8 <= INT32_MAX, "shard %d: trellis exceeds the 2 GiB buffer range", s);
    sa.trellis[s] = static_cast<const uint32_t*>(sh.trellis);
    sa.svh[s] = static_cast<const uint16_t*>(sh.svh);
    su.suh[s] = static_cast<const uint16_t*>(sh.suh);
    sa.tn[s] = sh.n / 16;
    EXL3_CHECK_ARG(sh.layout == EXL3_LAYOUT_STORED || sh.layout == EXL3_LAYOUT_BLOCKS, "shard %d: layout %d", s,
                   sh.layout);
    sa.layout[s] = sh.layout;
    sa.col0[s] = col;
    sa.ct0[s] = ctl;
    shard_n[s] = sh.n;
    col += sh.n;
    ctl += (sh.n / 128 + 1) / 2;
  }
  sa.ct0[nshards] = ctl;
  sa.count = nshards;
  return launch_prefill<true>(x, x_bf16 != 0, rows, k, sa, su, shard_n, K, codebook, y, y_bf16 != 0, workspace,
                              workspace_bytes, as_stream(stream), "exl3_linear_prefill");
}

namespace exl3 {

size_t prefill_plain_workspace_bytes(int rows, int k, int n) {
  const int nct = (n / 128 + 1) / 2;
  return gemm_layout(rows, k, nct, 1).total;
}

// exl3_gemm_rotated from kPrefillRows rows: the rows as given (fp16, already in the rotated basis), no output
// rotation, so one-hot rows read W_inner back through the decode-GEMM bit for bit
int prefill_plain_gemm(const void* xh, int rows, int k, const void* trellis, int n, int K, int codebook, void* out,
                       void* workspace, size_t workspace_bytes, hipStream_t st) {
  EXL3_CHECK_ARG((int64_t)rows * k * 2 <= INT32_MAX, "exl3_gemm_rotated: rows * k too large for one launch");
  GemmShards sa{};
  sa.trellis[0] = static_cast<const uint32_t*>(trellis);
  sa.tn[0] = n / 16;
  sa.ct0[1] = (n / 128 + 1) / 2;
  sa.count = 1;
  const ShardSuh su{};
  const int shard_n[1] = {n};
  return launch_prefill<false>(xh, false, rows, k, sa, su, shard_n, K, codebook, out, false, workspace,
                               workspace_bytes, st, "exl3_gemm_rotated");
}

}  // namespace exl3
