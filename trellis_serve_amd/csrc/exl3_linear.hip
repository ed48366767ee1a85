// EXL3 dense linear on gfx950: trellis decode (reconstruct), the 128-point Hadamard rotations, and the fused
// decode-GEMV for up to 16 rows per launch (MFMA 16x16x16 f16 fed from registers), with a deterministic split-K
// reduce that applies the output rotation.
//
// Reference semantics:
//   reconstruct        core/src/trellis_core/reference.py:102-115 (bit-exact)
//   input rotation     cuda/csrc/exl3_had.cuh:20-84  xh = fp16(Had(fp16(x) * suh)) (fp16 product, fp32 butterfly)
//   output rotation    cuda/csrc/exl3_had.cuh:89-117 y = fp16(Had(fp16(acc))) * svh (fp16 product)
//   split-K reduce     cuda/csrc/exl3_marlin_template.h:2234-2262 (fixed-order fp32 sum of per-split partials)
//   fused groups       cuda/csrc/exl3_marlin.cu:507-527 (shards share x, write adjacent column spans)
#include <stdlib.h>

#include <algorithm>
#include <cmath>
#include <atomic>
#include <mutex>
#include <vector>

#include "exl3_api.hpp"
#include "exl3_device.hpp"
#include "exl3_stream.hpp"

namespace exl3 {

constexpr int kGemvWaves = 8;   // one wave per tile column: a workgroup covers one 128-column block
constexpr int kGemvRows = 16;   // rows of one MFMA row group (the M of MFMA 16x16x16)
constexpr int kGemvPairRows = 32;  // rows per launch with two row groups per decoded tile (gemv_kernel<..., P = 2>)
constexpr int kGemvQuadRows = 64;  // rows per launch with four row groups (gemv_kernel<..., P = 4>)
constexpr int kGemvMaxLds = 65536;  // dynamic LDS limit of a workgroup without opt-in

struct ShardArgs {
  const uint32_t* trellis[EXL3_MAX_SHARDS];
  const uint16_t* suh[EXL3_MAX_SHARDS];
  const uint16_t* svh[EXL3_MAX_SHARDS];
  int tn[EXL3_MAX_SHARDS];            // tile columns (n / 16)
  int layout[EXL3_MAX_SHARDS];        // EXL3_LAYOUT_STORED / EXL3_LAYOUT_BLOCKS
  int col0[EXL3_MAX_SHARDS];          // first output column
  int blk0[EXL3_MAX_SHARDS + 1];      // first 128-column block (cumulative); blk0[count] = total blocks
  int count;
};

// The fields of the shard that a wave-uniform 128-column block belongs to, chosen by compares over the (at most
// EXL3_MAX_SHARDS) shards so that they stay in scalar registers.  Indexing the kernarg arrays with a computed shard
// index made the compiler load the fields through vector registers and wrap every buffer load built on the trellis
// base in a readfirstlane loop (five VALU and three SALU instructions a load, in every wave).
struct ShardView {
  const uint32_t* trellis;
  const uint16_t* suh;
  const uint16_t* svh;
  int tn, col0, blk0, layout;
};

// Every field of every shard is read into scalar registers before the compares (the empty asm statements take them
// as operands): left to itself the compiler loads only the chosen shard's fields, after the compares, which puts two
// or three dependent rounds of kernarg loads in front of the first memory request of every workgroup.
__device__ __forceinline__ ShardView shard_of_block(const ShardArgs& sa, int blk) {
  ShardView f[EXL3_MAX_SHARDS];
#pragma unroll
  for (int i = 0; i < EXL3_MAX_SHARDS; i++) {
    f[i] = ShardView{sa.trellis[i], sa.suh[i], sa.svh[i], sa.tn[i], sa.col0[i], sa.blk0[i], sa.layout[i]};
    asm volatile("" ::"s"(f[i].trellis), "s"(f[i].suh), "s"(f[i].svh), "s"(f[i].tn), "s"(f[i].col0), "s"(f[i].blk0),
                 "s"(f[i].layout));
  }
  const int count = sa.count;
  asm volatile("" ::"s"(count));
  ShardView v = f[0];
#pragma unroll
  for (int i = 1; i < EXL3_MAX_SHARDS; i++)
    if (i < count && blk >= f[i].blk0) v = f[i];
  return v;
}

__device__ __forceinline__ int find_shard(const ShardArgs& sa, int blk) {
  int s = 0;
#pragma unroll
  for (int i = 1; i < EXL3_MAX_SHARDS; i++)
    if (i < sa.count && blk >= sa.blk0[i]) s = i;
  return s;
}

// ---- input rotation of 4 values: lane t of a 32-lane group holds block positions 4t..4t+3 --------------------
// from the raw 8 bytes of x (fp16 or bf16) and of suh at those positions
template <bool X_BF16>
__device__ __forceinline__ void had_in_raw(uint2_t raw, uint2_t suraw, _Float16 h[4]) {
  _Float16 v[4];
  if constexpr (X_BF16) {
    v[0] = (_Float16)bf16_to_f32((uint16_t)(raw.x & 0xFFFF));
    v[1] = (_Float16)bf16_to_f32((uint16_t)(raw.x >> 16));
    v[2] = (_Float16)bf16_to_f32((uint16_t)(raw.y & 0xFFFF));
    v[3] = (_Float16)bf16_to_f32((uint16_t)(raw.y >> 16));
  } else {
    const half4_t hv = __builtin_bit_cast(half4_t, raw);
    v[0] = hv.x; v[1] = hv.y; v[2] = hv.z; v[3] = hv.w;
  }
  const half4_t su = __builtin_bit_cast(half4_t, suraw);
  float f0 = (float)(_Float16)(v[0] * su.x), f1 = (float)(_Float16)(v[1] * su.y);
  float f2 = (float)(_Float16)(v[2] * su.z), f3 = (float)(_Float16)(v[3] * su.w);
  had128_x4(f0, f1, f2, f3);
  h[0] = had_scale_f16(f0);
  h[1] = had_scale_f16(f1);
  h[2] = had_scale_f16(f2);
  h[3] = had_scale_f16(f3);
}

template <bool X_BF16>
__device__ __forceinline__ void had_in_4(const void* x_row, const uint16_t* __restrict__ suh, int kk, _Float16 h[4]) {
  had_in_raw<X_BF16>(*reinterpret_cast<const uint2_t*>(static_cast<const uint16_t*>(x_row) + kk),
                     *reinterpret_cast<const uint2_t*>(suh + kk), h);
}

// output rotation of 4 fp16 values (lane t of a 32-lane group: block positions 4t..4t+3), then * svh
__device__ __forceinline__ void had_out_4(_Float16 h[4], const uint16_t* __restrict__ svh4) {
  float f0 = (float)h[0], f1 = (float)h[1], f2 = (float)h[2], f3 = (float)h[3];
  had128_x4(f0, f1, f2, f3);
  const half4_t sv = *reinterpret_cast<const half4_t*>(svh4);
  h[0] = had_scale_f16(f0) * sv.x;
  h[1] = had_scale_f16(f1) * sv.y;
  h[2] = had_scale_f16(f2) * sv.z;
  h[3] = had_scale_f16(f3) * sv.w;
}

template <bool BF16>
__device__ __forceinline__ void store_4(void* row, int col, const _Float16 h[4]) {
  if constexpr (BF16) {
    uint2_t o;
    o.x = (uint32_t)f32_to_bf16((float)h[0]) | ((uint32_t)f32_to_bf16((float)h[1]) << 16);
    o.y = (uint32_t)f32_to_bf16((float)h[2]) | ((uint32_t)f32_to_bf16((float)h[3]) << 16);
    *reinterpret_cast<uint2_t*>(static_cast<uint16_t*>(row) + col) = o;
  } else {
    half4_t o = {h[0], h[1], h[2], h[3]};
    *reinterpret_cast<half4_t*>(static_cast<uint16_t*>(row) + col) = o;
  }
}

// ---- reconstruct: one wave per tile -----------------------------------------------------------------------------
template <int K, int CB>
__global__ __launch_bounds__(256) void reconstruct_kernel(const uint32_t* __restrict__ trellis, int tk, int tn,
                                                          uint16_t* __restrict__ w) {
  const int tile = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tile >= tk * tn) return;
  const int i = tile / tn, jt = tile - i * tn;
  const int l = threadIdx.x & 63, c = l & 15, j = l >> 4;
  const LaneGeo g = lane_geo<K>(c, j);
  const uint32_t* tp = trellis + (size_t)tile * 8 * K;
  const half4_t v = decode_group<K, CB>(tp[g.dw0], tp[g.dw1], g);
  const size_t n = (size_t)tn * 16;
  _Float16* base = reinterpret_cast<_Float16*>(w) + (size_t)16 * i * n + 16 * jt + c;
  base[(size_t)(2 * j) * n] = v.x;
  base[(size_t)(2 * j + 1) * n] = v.y;
  base[(size_t)(2 * j + 8) * n] = v.z;
  base[(size_t)(2 * j + 9) * n] = v.w;
}

// ---- standalone rotations -------------------------------------------------------------------------------------
template <bool X_BF16>
__global__ __launch_bounds__(256) void had_in_kernel(const void* __restrict__ x, int rows, int k,
                                                     const uint16_t* __restrict__ suh_cat, int shards,
                                                     uint16_t* __restrict__ xh) {
  const int kb = k >> 7;
  const int unit = blockIdx.x * 8 + (threadIdx.x >> 5);
  if (unit >= shards * rows * kb) return;
  const int t = threadIdx.x & 31;
  const int s = unit / (rows * kb), rem = unit - s * rows * kb, r = rem / kb, b = rem - r * kb;
  const int kk = b * 128 + 4 * t;
  _Float16 h[4];
  had_in_4<X_BF16>(static_cast<const uint16_t*>(x) + (size_t)r * k, suh_cat + (size_t)s * k, kk, h);
  store_4<false>(xh + ((size_t)s * rows + r) * k, kk, h);
}

// The rotated activations of every shard of a fused linear, xh[s][r][k] = fp16(Had(x[r] * suh_s)), each 16-position
// group stored in the GEMV's A-staging order (a_slot) so that gemv_kernel<.., PRE> stages rows by plain copies.  One
// half-wave per (shard, row, 128-block).
template <bool X_BF16>
__global__ __launch_bounds__(256) void had_in_shards_kernel(const void* __restrict__ x, int rows, int k, ShardArgs sa,
                                                            uint16_t* __restrict__ xh) {
  const int kb = k >> 7;
  const int unit = blockIdx.x * 8 + (threadIdx.x >> 5);
  if (unit >= sa.count * rows * kb) return;
  const int t = threadIdx.x & 31;
  const int s = unit / (rows * kb), rem = unit - s * rows * kb, r = rem / kb, b = rem - r * kb;
  const int kk = b * 128 + 4 * t;
  _Float16 h[4];
  had_in_4<X_BF16>(static_cast<const uint16_t*>(x) + (size_t)r * k, sa.suh[s], kk, h);
  // positions 4t, 4t+1 and 4t+2, 4t+3 land on adjacent staging slots: two 4-byte stores
  typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
  _Float16* row = reinterpret_cast<_Float16*>(xh) + ((size_t)s * rows + r) * k;
  *reinterpret_cast<half2_t*>(row + a_slot(kk, 0, 0)) = half2_t{h[0], h[1]};
  *reinterpret_cast<half2_t*>(row + a_slot(kk + 2, 0, 0)) = half2_t{h[2], h[3]};
}

template <bool OUT_BF16>
__global__ __launch_bounds__(256) void had_out_kernel(const uint16_t* __restrict__ y, int rows, int n,
                                                      const uint16_t* __restrict__ svh, void* __restrict__ out,
                                                      int ld_out, int col0) {
  const int nb = n >> 7;
  const int unit = blockIdx.x * 8 + (threadIdx.x >> 5);
  if (unit >= rows * nb) return;
  const int t = threadIdx.x & 31;
  const int r = unit / nb, b = unit - r * nb;
  const int cc = b * 128 + 4 * t;
  const half4_t v = *reinterpret_cast<const half4_t*>(y + (size_t)r * n + cc);
  _Float16 h[4] = {v.x, v.y, v.z, v.w};
  had_out_4(h, svh + cc);
  store_4<OUT_BF16>(static_cast<uint16_t*>(out) + (size_t)r * ld_out, col0 + cc, h);
}

// ---- fused decode-GEMV ------------------------------------------------------------------------------------------
// grid (128-column blocks over all shards, k-splits); 8 waves; wave w owns tile column 8*block + w of its shard
// and NT tile rows (NB = NT/8 blocks of 128 rows) starting at block kb0 = split * NB.
//
// Streaming: a block's 8 tiles of the wave's column (8 x 32K bytes, 96 B apart at K = 3) arrive with one or two
// wave-wide 16-byte-per-lane gathers (the texture addresser spends the same cycles on a 4-byte and a 16-byte lane,
// so wide lanes cut its work about 8x against per-tile dword gathers), are written to a wave-private LDS stage, and
// each lane then reads the two dwords of its group per tile from LDS.  Three blocks are in flight.  The code is
// straight-line (NT is a template parameter): no loop-carried load registers, exact in-order vmcnt waits.  A split
// shorter than NT rows (the last one) clamps its loads to its last block and sees zero activations past its end.
//
// Every two decoded tiles (tile rows 2v and 2v + 1 of the wave's column) feed one MFMA 16x16x32 f16 per 16-row
// group, on two alternating accumulators.  The prologue stages the split's rotated activations (ROTATE) or the given
// ones into LDS in MFMA A order.
//
// Split-K epilogue (the slot reduce of cuda/csrc/exl3_marlin_template.h:2234-2262, in one launch): every split
// writes its fp32 partial [split][m][col]; the last split of a column block to arrive (a per-block counter in the
// workspace) sums all partials in a fixed order, rounds once to fp16, applies the output rotation (ROTATE) and
// stores y, then resets the counter to zero for the next call.
constexpr int kGemvThreads = kGemvWaves * 64;
constexpr int kCoherentDevice = 1 << 4;  // buffer cache policy sc1: device-scope coherent access
constexpr int kBypassL1 = 1;             // buffer cache policy sc0: miss the L1, read the L2
constexpr int kWaitVmcnt0 = 0x0F70;      // s_waitcnt vmcnt(0) (expcnt, lgkmcnt unconstrained)

// LDS bytes of the GEMV: staged activations (M rows of a_mstride(NT) halves), then per wave two block stages of 256*K
// bytes; at least 16 * 128 fp32 for the epilogue reduce
__host__ __device__ constexpr int gemv_a_bytes(int M, int NT) { return ((M * a_mstride(NT) * 2) + 15) & ~15; }
__host__ __device__ constexpr int gemv_lds_bytes(int M, int NT, int K) {
  return gemv_a_bytes(M, NT) + kGemvWaves * stream_lds_bytes(K) > kGemvThreads * 16
             ? gemv_a_bytes(M, NT) + kGemvWaves * stream_lds_bytes(K)
             : kGemvThreads * 16;
}

// PRE: x is the rotated activations of every shard, [shards][pre_rows][k] in A-staging order (had_in_shards_kernel),
// staged by 8-byte copies; else x is the input rows, rotated here (ROTATE) or taken as given.
// Every decoded tile pair feeds one v_mfma_f32_16x16x32_f16 per 16-row group: P = 1 up to 16 rows
// (TileStream::run_pairs), P = 2 / 4 for 17-32 / 33-64 rows (run_groups: the weights stream once for 16 P rows
// instead of once per 16; the staged rows are padded with zeros).  Every form multiplies by the rounded fp16 weights
// of trellis_core.
template <int K, int CB, bool ROTATE, int NT, bool PRE = false, int P = 1>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(ShardArgs sa, const void* __restrict__ x, int x_bf16,
                                                             int M, int k, int splits, float* partial,
                                                             int* counters, void* __restrict__ y,
                                                             int y_bf16, int n_total, int pre_rows = 0,
                                                             int xl = 0) {
  typedef TileStream<K, CB, NT, false> Stream;
  constexpr int NB = Stream::NB;
  // Issue priority: the prologue and the split-K chain are latency-bound and short, the decode loop is VALU-bound
  // and long.  The SIMD's arbiter prefers older waves among equals, so a CU's youngest workgroup would otherwise get
  // few issue slots for its prologue and chain while older workgroups decode (gate_up 35.3 -> 34.3 us).
  __builtin_amdgcn_s_setprio(2);

  const int Mp = P == 1 ? M : kGemvRows * ((M + kGemvRows - 1) / kGemvRows);  // staged rows; rows M .. Mp-1 are 0
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ int last_flag;
  _Float16* xs = reinterpret_cast<_Float16*>(lds);
  const int blk = blockIdx.x, split = blockIdx.y;
  asm volatile("" ::"s"(x), "s"(M), "s"(k), "s"(x_bf16));  // with the shard fields: one round of kernarg loads
  const ShardView sh = shard_of_block(sa, blk);
  const int kb0 = split * NB;
  const int nb = min(k >> 7, kb0 + NB) - kb0;  // blocks of this split holding data (1..NB)
  constexpr int mstride = a_mstride(NT);
  // four consecutive activations p .. p+3 (p a multiple of 4): a_slot keeps each even-odd pair adjacent
  auto stage4 = [&](int p, int m, const _Float16 (&h)[4]) {
    *reinterpret_cast<half2_t*>(xs + a_slot(p, m, mstride)) = half2_t{h[0], h[1]};
    *reinterpret_cast<half2_t*>(xs + a_slot(p + 2, m, mstride)) = half2_t{h[2], h[3]};
  };

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63, c = l & 15, j = l >> 4;
  const int tn = sh.tn;
  // prologue: activations of the split, rotated (or as given), into LDS; blocks past the split's end are zero.  One
  // (row, block) unit per half-wave.  When every half-wave has at most one unit, its activation loads are issued
  // before the trellis loads: loads complete in issue order, so the rotation then waits only for its own data and
  // runs while the trellis blocks are in flight.
  const int hw = threadIdx.x >> 5, t = threadIdx.x & 31;
  const bool single = !PRE && Mp * NB <= 2 * kGemvWaves;
  uint2_t xv = uint2_t{0u, 0u}, sv = uint2_t{0u, 0u};
  if constexpr (!PRE) {
    const int m = hw / NB, b = hw - m * NB;
    if (single && hw < M * NB && b < nb) {
      const int kk = (kb0 + b) * 128 + 4 * t;
      xv = *reinterpret_cast<const uint2_t*>(static_cast<const uint16_t*>(x) + (size_t)m * k + kk);
      if constexpr (ROTATE) sv = *reinterpret_cast<const uint2_t*>(sh.suh + kk);
    }
  }
  __asm__ volatile("" ::: "memory");  // keep the activation loads ahead of the trellis loads

  Stream stream;
  stream.init(sh.trellis, (k >> 4) * tn * 32 * K, tn, (blk - sh.blk0) * kGemvWaves + w, kb0, nb,
              lds + gemv_a_bytes(Mp, NT) + w * Stream::LDS_BYTES, l, sh.layout == EXL3_LAYOUT_BLOCKS, k >> 7);
  // Trellis blocks issued before the prologue.  Every workgroup's activation loads queue behind the trellis loads
  // the CU's workgroups issued before them, so the prologue (and with it the first MFMA) waits less with fewer early
  // blocks; the rest of the three in flight follow the prologue's barrier (layer set at one row: 79.2 -> 78.2 us).
  // Prepared rows (PRE) need no rotation: all three go first.
  constexpr int kEarly = PRE ? 3 : NB >= 4 ? 2 : 1;
#pragma unroll
  for (int b = 0; b < kEarly && b < NB; b++) stream.issue(b);

  if constexpr (PRE) {
    // prepared rows: 8-byte copies, all loads of the half-wave issued before the stores
    constexpr int IT = kGemvRows * P * NB / (2 * kGemvWaves);
    const uint16_t* pre = static_cast<const uint16_t*>(x) + (size_t)find_shard(sa, blk) * pre_rows * k;
    uint2_t v[IT];
#pragma unroll
    for (int it = 0; it < IT; it++) {
      const int u = hw + it * 2 * kGemvWaves;
      const int m = u / NB, b = u - m * NB;
      v[it] = uint2_t{0u, 0u};
      if (u < M * NB && b < nb) v[it] = *reinterpret_cast<const uint2_t*>(pre + (size_t)m * k + (kb0 + b) * 128 + 4 * t);
    }
#pragma unroll
    for (int it = 0; it < IT; it++) {
      const int u = hw + it * 2 * kGemvWaves;
      const int m = u / NB, b = u - m * NB;
      if (u < Mp * NB) {  // rows M .. Mp-1 store the zeros v was set to
        *reinterpret_cast<uint2_t*>(xs + m * mstride + b * 128 + 4 * t) = v[it];
      }
    }
  } else if (single) {
    if (hw < Mp * NB) {
      const int m = hw / NB, b = hw - m * NB;
      _Float16 h[4] = {0, 0, 0, 0};
      if (b < nb && m < M) {
        if constexpr (ROTATE) {
          if (x_bf16)
            had_in_raw<true>(xv, sv, h);
          else
            had_in_raw<false>(xv, sv, h);
        } else {
          const half4_t v = __builtin_bit_cast(half4_t, xv);
          h[0] = v.x; h[1] = v.y; h[2] = v.z; h[3] = v.w;
        }
      }
      stage4(b * 128 + 4 * t, m, h);
    }
  } else {
    for (int u = hw; u < Mp * NB; u += 2 * kGemvWaves) {
      const int m = u / NB, b = u - m * NB;
      const int kk = (kb0 + b) * 128 + 4 * t;
      _Float16 h[4] = {0, 0, 0, 0};
      if (b < nb && m < M) {
        if constexpr (ROTATE) {
          if (x_bf16)
            had_in_4<true>(static_cast<const uint16_t*>(x) + (size_t)m * k, sh.suh, kk, h);
          else
            had_in_4<false>(static_cast<const uint16_t*>(x) + (size_t)m * k, sh.suh, kk, h);
        } else {
          const half4_t v = *reinterpret_cast<const half4_t*>(static_cast<const uint16_t*>(x) + (size_t)m * k + kk);
          h[0] = v.x; h[1] = v.y; h[2] = v.z; h[3] = v.w;
        }
      }
      stage4(b * 128 + 4 * t, m, h);
    }
  }
  __syncthreads();
#pragma unroll
  for (int b = kEarly; b < 3 && b < NB; b++) stream.issue(b);

  __builtin_amdgcn_s_setprio(0);
  // A row m = l % 16; rows m >= M read row M-1 (finite values) and only feed C rows that are never stored
  float4_t acc[P];
  if constexpr (P > 1) {
#pragma unroll
    for (int p = 0; p < P; p++) acc[p] = float4_t{0.f, 0.f, 0.f, 0.f};
    stream.template run_groups<P>(reinterpret_cast<const half8_t*>(xs + min(c, M - 1) * mstride) + j,
                                  kGemvRows * mstride / 8, Mp / kGemvRows, acc);
  } else {
    acc[0] = stream.run_pairs(reinterpret_cast<const half8_t*>(xs + min(c, M - 1) * mstride) + j);
  }


  __builtin_amdgcn_s_setprio(2);
  // this split's partial; C layout: lane l holds rows 4(l/16) + r, column l % 16.  Each XCD has its own L2.  With
  // xl (the host's check that workgroups whose linear ids agree mod 8 run on one XCD, and a column-block count that
  // is a multiple of 8: all splits of a column block then share an XCD) the partials, the arrival counter and the
  // reduce stay in that XCD's L2: plain stores, L2 atomics, loads that bypass only the L1.  Otherwise they are
  // written and read with device-scope coherence (sc1: write-through, no stale L2 hits) instead of a device-scope
  // fence, which would write back this XCD's whole L2.
  const int col_blk = blk * 128;  // first column of the block in y / partial
  const __amdgpu_buffer_rsrc_t prsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)partial, (short)0, splits * M * n_total * 4, 0x00020000);
  float* pdst = partial + (size_t)split * M * n_total + col_blk + w * 16 + c;
#pragma unroll
  for (int p = 0; p < P; p++)
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int m = kGemvRows * p + 4 * j + r;
      if (m < M) {
        if (xl)
          __hip_atomic_store(pdst + (size_t)m * n_total, acc[p][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        else
          __hip_atomic_store(pdst + (size_t)m * n_total, acc[p][r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // this thread's partial stores are at the coherence point
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = xl ? __hip_atomic_fetch_add(&counters[blk], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)
                        : __hip_atomic_fetch_add(&counters[blk], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev == splits - 1;
  }
  __syncthreads();
  if (!last_flag) return;

  // last split of this column block: units (row m, 4-column group q); p-groups G share the splits p = g, g + G, ...
  // and are combined in a fixed order.  Past 16 rows the units take passes of 512 (16 rows each).
  float4_t* red = reinterpret_cast<float4_t*>(lds);  // reuse the LDS (>= 512 * 16 B reserved)
  const int tid = threadIdx.x;
  for (int u0 = 0; u0 < M * 32; u0 += kGemvThreads) {
    const int units = min(M * 32 - u0, kGemvThreads);
    const int G = max(1, kGemvThreads / units);
    if (tid < units * G) {
      const int unit = u0 + tid % units, gq = tid / units;
      const int m = unit >> 5, q = unit & 31;
      const int base = (m * n_total + col_blk + 4 * q) * 4;
      const int pstride = M * n_total * 4;
      // up to 8 loads in flight per round (only for splits that exist), summed in split order
      float4_t a = {0.f, 0.f, 0.f, 0.f};
      for (int p0 = gq; p0 < splits; p0 += 8 * G) {
        float4_t v[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
          v[i] = p0 + i * G >= splits ? float4_t{0.f, 0.f, 0.f, 0.f}
                 : xl ? __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                            prsrc, base + (p0 + i * G) * pstride, 0, kBypassL1))
                      : __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                            prsrc, base + (p0 + i * G) * pstride, 0, kCoherentDevice));
#pragma unroll
        for (int i = 0; i < 8; i++)
          if (p0 + i * G < splits) a += v[i];
      }
      red[gq * units + unit - u0] = a;
    }
    __syncthreads();
    if (tid < units) {
      float4_t a = red[tid];
      for (int gq = 1; gq < G; gq++) a += red[gq * units + tid];
      const int m = (u0 + tid) >> 5, q = tid & 31;
      _Float16 h[4] = {(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w};
      const int col = col_blk + 4 * q;
      if constexpr (ROTATE) had_out_4(h, sh.svh + (col - sh.col0));
      uint16_t* yrow = static_cast<uint16_t*>(y) + (size_t)m * n_total;
      if (y_bf16)
        store_4<true>(yrow, col, h);
      else
        store_4<false>(yrow, col, h);
    }
    __syncthreads();  // the next pass reuses red
  }
  if (tid == 0) {
    if (xl)
      __hip_atomic_store(&counters[blk], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else
      __hip_atomic_store(&counters[blk], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---- host side --------------------------------------------------------------------------------------------------

// k-split plan of the GEMV: NT tile rows per split (a template instance: 16, 32 or 64), the largest that still gives
// enough (block, split) workgroups to fill the 256 CUs, LDS for the staged activations (and >= 16 * 128 fp32 for
// the epilogue reduce).
struct GemvPlan {
  int nt, splits;
  size_t lds;
};

// the workgroup target of the two- and four-group launches (17-64 rows), where every split's fp32 partial of M rows
// is written and read again and the last split's reduce reads all of them; one row group takes the equal-split rule
// of gemv_plan and its own minimum
constexpr int kGemvOneGroupWgs = 448;
// one-group workgroups resident at once on MI355X: 256 CUs x 4 (8 waves of <= 64 VGPRs, < 40 KB of LDS each).  A
// constant, so that the plan (and with it every workspace size) depends on the arguments alone.
constexpr int kGemvOneGroupSlots = 256 * 4;
// rows: the launch's rows (17-32: two row groups, 33-64: four).  Two-group launches aim at 512: q/k/v at 24-32 rows
// then takes 32 tile rows (640 workgroups) instead of 16 (1280), 1-1.7 us less per step, and no other layer of the
// layer set moves; four-group launches keep 768 (q/k/v at 48-64 rows 3 us slower at 512).
static int gemv_target_wgs(int rows = kGemvQuadRows) {
  static const int env = [] {
    const char* e = getenv("EXL3_GEMV_TARGET_WGS");
    return e ? std::max(1, atoi(e)) : 0;
  }();
  return env ? env : rows <= kGemvPairRows ? 512 : 768;
}

// pre: prepared rows (gemv_kernel<.., PRE>), whose 64-row-tile instance needs 132 VGPRs: at most 32 there.
// Past 16 rows (P = 2, 4) the staged activations are padded to 32 or 64 rows.  The plan does not depend on the
// codebook.
static GemvPlan gemv_plan(int k, int n_total, int M, int K, bool pre = false) {
  const int kb = k / 128, nblk = n_total / 128;
  const int Ms = M <= kGemvRows ? M : M <= kGemvPairRows ? kGemvPairRows : kGemvQuadRows;
  int nt = 16;
  if (M <= kGemvRows) {
    // one row group: the longest split of at most 40 tile rows (prepared rows: 32) that cuts k into equal splits (at
    // most 2 % of the last one empty) and still gives >= 448 workgroups.  Measured against the earlier plan (16 / 32
    // tile rows for >= 1536 workgroups below 8 rows, >= 768 from 8; same call): one row down 21.3 -> 18.6 us (32),
    // q/k/v 12.9 -> 11.9 (40), o 11.7 -> 11.0 (32), gate_up 33.7 -> 33.5 (40); 16 rows q/k/v 18.4 -> 16.7 (40),
    // o 16.2 -> 15.4 (32); 48-64 tile rows were no faster anywhere and slower on q/k/v and gate_up.
    // When the longest such split gives more workgroups than run at once, the launch runs in rounds and the last one
    // may leave most slots idle: then the candidate whose last round is fullest (workgroups / slots closest to a
    // whole number from below) wins.  One row, same call, two rounds: gate_up 40 -> 32 tile rows (2.1 -> 2.7 rounds)
    // 30.1-30.3 -> 29.8-30.1 us, down 32 -> 24 (1.3 -> 1.8 rounds) 18.0-18.1 -> 17.7-17.8 us; q/k/v and o (under one
    // round) kept their splits, which measured best for them (40 / 32).
    double best_fill = 0.0;
    for (int cand : {40, 32, 24}) {
      if (pre && cand != 32) continue;
      const int nbc = cand / 8, splits = (kb + nbc - 1) / nbc;
      if (splits * nbc * 50 <= kb * 51 && (size_t)nblk * splits >= kGemvOneGroupWgs &&
          gemv_lds_bytes(Ms, cand, K) <= kGemvMaxLds) {
        const double rounds = (double)nblk * splits / kGemvOneGroupSlots;
        if (best_fill == 0.0 && rounds <= 1.0) {  // the longest candidate fits one round: take it
          nt = cand;
          break;
        }
        const double fill = rounds <= 1.0 ? 1.0 : rounds / std::ceil(rounds);
        if (fill > best_fill + 1e-9) {
          best_fill = fill;
          nt = cand;
        }
      }
    }
    return {nt, (kb + nt / 8 - 1) / (nt / 8), (size_t)gemv_lds_bytes(Ms, nt, K)};
  }
  for (int cand : {64, 32}) {
    const int splits = (kb + cand / 8 - 1) / (cand / 8);
    if (pre && cand > 32) continue;
    if ((size_t)nblk * splits >= (size_t)gemv_target_wgs(M) && gemv_lds_bytes(Ms, cand, K) <= kGemvMaxLds) {
      nt = cand;
      break;
    }
  }
  return {nt, (kb + nt / 8 - 1) / (nt / 8), (size_t)gemv_lds_bytes(Ms, nt, K)};
}

// workspace layout: [counter region: one int per 128-column block, zero between calls][fp32 partials]; the region
// has a fixed size so that a later call of another shape never takes an earlier call's partials for counters
static size_t counters_bytes(int n_total) {
  (void)n_total;
  return kCounterBytes;
}

#define EXL3_DISPATCH_K_CB(K_, CB_, ...)                                  \
  [&]() -> bool {                                                         \
    switch (K_ * 4 + CB_) {                                               \
      EXL3_CASE_KCB(2, __VA_ARGS__) EXL3_CASE_KCB(3, __VA_ARGS__)         \
      EXL3_CASE_KCB(4, __VA_ARGS__) EXL3_CASE_KCB(5, __VA_ARGS__)         \
      EXL3_CASE_KCB(6, __VA_ARGS__) EXL3_CASE_KCB(8, __VA_ARGS__)         \
      default: return false;                                              \
    }                                                                     \
  }()
#define EXL3_CASE_KCB(KV, ...)                                                         \
  case KV * 4 + 0: { constexpr int kK = KV, kCB = 0; __VA_ARGS__; return true; }      \
  case KV * 4 + 1: { constexpr int kK = KV, kCB = 1; __VA_ARGS__; return true; }      \
  case KV * 4 + 2: { constexpr int kK = KV, kCB = 2; __VA_ARGS__; return true; }

static int build_shards(const exl3_shard* shards, int nshards, int k, int K, ShardArgs* sa, int* n_total) {
  EXL3_CHECK_ARG(shards != nullptr && nshards >= 1 && nshards <= EXL3_MAX_SHARDS,
                 "nshards = %d (1..%d)", nshards, EXL3_MAX_SHARDS);
  *sa = ShardArgs{};
  int col = 0, blk = 0;
  for (int s = 0; s < nshards; s++) {
    const exl3_shard& sh = shards[s];
    EXL3_CHECK_ARG(sh.trellis && sh.suh && sh.svh, "shard %d: null tensor pointer", s);
    EXL3_CHECK_ARG(sh.n > 0 && sh.n % 128 == 0, "shard %d: n = %d is not a positive multiple of 128", s, sh.n);
    EXL3_CHECK_ARG(blk + sh.n / 128 <= kMaxCounters, "group of more than %d output columns", kMaxCounters * 128);
    EXL3_CHECK_ARG((int64_t)k * sh.n * K / 8 <= INT32_MAX, "shard %d: trellis of %lld bytes exceeds the 2 GiB buffer range",
                   s, (long long)((int64_t)k * sh.n * K / 8));
    sa->trellis[s] = static_cast<const uint32_t*>(sh.trellis);
    sa->suh[s] = static_cast<const uint16_t*>(sh.suh);
    sa->svh[s] = static_cast<const uint16_t*>(sh.svh);
    sa->tn[s] = sh.n / 16;
    EXL3_CHECK_ARG(sh.layout == EXL3_LAYOUT_STORED || sh.layout == EXL3_LAYOUT_BLOCKS, "shard %d: layout %d", s,
                   sh.layout);
    sa->layout[s] = sh.layout;
    sa->col0[s] = col;
    sa->blk0[s] = blk;
    col += sh.n;
    blk += sh.n / 128;
  }
  sa->blk0[nshards] = blk;
  sa->count = nshards;
  *n_total = col;
  return EXL3_OK;
}

// one launch per 16 rows: decode-GEMV + in-launch split reduce (+ rotations when `rotate`)
// With many rows and much redundant rotation work (every column block's workgroup rotates the rows of its split:
// nblk x rows x k/128 half-wave units in total), the input rotation runs once per shard and row (had_in_shards_kernel)
// before the GEMV.  At M = 16 the per-workgroup rotation made the gate_up launch of the layer set LDS-bound (its
// shuffles and scattered staging writes): 51 us against 41 us with the separate rotation, 34 us at M = 1; for the
// q/k/v and o launches (under 65536 units) the extra launch costs more than it saves.
constexpr int kGemvPreRows = 8;
constexpr size_t kGemvPreUnits = 65536;

static bool gemv_pre(int rows, int k, int n_total) {
  return rows >= kGemvPreRows && (size_t)(n_total / 128) * rows * (k / 128) >= kGemvPreUnits;
}

// Rows per launch: four row groups (64) only where the layer needs 16-tile-row splits for enough workgroups anyway
// (narrow layers: q/k/v, o): there 64 staged rows fit the default LDS and one launch beats two.  Wider layers would
// need 32-tile-row splits, whose 64 staged rows exceed that LDS (and the fp32 partials of 64 rows grow with the
// splits): there 64 rows take two launches of two groups (measured at 64 rows: gate_up 102.5 us against 112.9 us with
// one four-group launch, down 73.5 against 77.8; q/k/v 47.5 -> 39.2, o 42.0 -> 37.0 with it).
static int gemv_launch_rows(int k, int n_total, int launch_rows) {
  if (launch_rows < kGemvQuadRows) return launch_rows;
  const int kb = k / 128, nblk = n_total / 128;
  return (size_t)nblk * ((kb + 3) / 4) < (size_t)gemv_target_wgs() ? kGemvQuadRows : kGemvPairRows;
}

// workspace layout: [counter region][fp32 partials of the largest launch][rotated rows, when gemv_pre].
// launch_rows: the entry point's rows per launch, 16 (exl3_gemm_rotated, exl3_linear_noalloc), or 64 where row groups
// share each decoded tile (exl3_linear; gemv_launch_rows may lower it to 32).  A call's launches are the full ones
// and the remainder, each with its own split plan: the partial region holds the larger of the two.  rotate: the
// launches rotate their inputs (exl3_linear, exl3_linear_noalloc) and may then take prepared rows, whose split plan
// differs; exl3_gemm_rotated's do not.
static size_t gemv_launch_partial_bytes(int M, int rows, int k, int n_total, int K, bool rotate) {
  const bool pre = rotate && gemv_pre(rows, k, n_total);
  return (size_t)gemv_plan(k, n_total, M, K, pre).splits * M * n_total * sizeof(float);
}
static size_t gemv_partial_bytes(int rows, int k, int n_total, int K, int launch_rows, bool rotate) {
  size_t need = 0;
  launch_rows = gemv_launch_rows(k, n_total, launch_rows);
  for (int M : {std::min(rows, launch_rows), rows % launch_rows})
    if (M > 0) need = std::max(need, gemv_launch_partial_bytes(M, rows, k, n_total, K, rotate));
  return (need + 255) & ~(size_t)255;
}
static size_t gemv_pre_bytes(int rows, int k, int n_total, bool rotate) {
  return rotate && gemv_pre(rows, k, n_total) ? (size_t)EXL3_MAX_SHARDS * rows * k * 2 : 0;
}

static size_t gemv_workspace_bytes(int rows, int k, int n_total, int K, int launch_rows, bool rotate) {
  return counters_bytes(n_total) + gemv_partial_bytes(rows, k, n_total, K, launch_rows, rotate) +
         gemv_pre_bytes(rows, k, n_total, rotate);
}

// ---- split-K chain inside one XCD ---------------------------------------------------------------------------
// The launches' grids are x = column block (fastest), y = k-split, so the splits of a column block have linear
// workgroup ids that agree mod the column-block count.  When workgroups whose ids agree mod 8 run on one XCD (the
// hardware hands workgroup i to XCD i mod 8 on an 8-XCD part; the same holds with 1, 2 or 4 XCDs per device) and the
// column-block count is a multiple of 8, every split of a column block runs on one XCD and its chain can stay in
// that XCD's L2.  exl3_init_device checks the first property with a probe launch; until it has passed on some
// device of the process, every chain uses device-coherent accesses.
static std::atomic<int> g_xcd_groups_ok{0};

__global__ __launch_bounds__(64) void xcd_probe_kernel(int* out) {
  if (threadIdx.x == 0) out[blockIdx.x] = (int)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 0xF);  // HW_REG_XCC_ID
}

int xcd_probe(int device) {
  constexpr int kProbeWgs = 4096;
  int cur = 0;
  EXL3_CHECK_HIP(hipGetDevice(&cur));
  if (cur != device) EXL3_CHECK_HIP(hipSetDevice(device));
  int cus = 0;
  EXL3_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
  const int xcds = std::max(1, std::min(8, cus / 32));  // 32 CUs per XCD on gfx950
  int* d = nullptr;
  hipError_t e = hipMalloc(&d, kProbeWgs * sizeof(int));
  int ok = 0;
  if (e == hipSuccess) {
    xcd_probe_kernel<<<kProbeWgs, 64>>>(d);
    e = hipGetLastError();
    std::vector<int> h(kProbeWgs);
    if (e == hipSuccess) e = hipMemcpy(h.data(), d, kProbeWgs * sizeof(int), hipMemcpyDeviceToHost);
    if (e == hipSuccess) {
      // the ids that agree mod 8 share an XCD, and the first 8 cover as many XCDs as the device has (a register that
      // read the same value everywhere would otherwise pass)
      ok = 1;
      for (int i = 8; i < kProbeWgs; i++) ok &= h[i] == h[i % 8];
      int distinct = 0;
      for (int i = 0; i < 8; i++) {
        bool seen = false;
        for (int q = 0; q < i; q++) seen |= h[q] == h[i];
        distinct += !seen;
      }
      ok &= distinct == xcds;
    }
    hipFree(d);
  }
  if (cur != device) (void)hipSetDevice(cur);
  if (e != hipSuccess) return set_error(EXL3_ERR_HIP, "exl3_init_device: XCD probe: %s", hipGetErrorString(e));
  if (ok) g_xcd_groups_ok.store(1);
  return EXL3_OK;
}

bool xcd_groups_ok() {
  static const bool off = [] {
    const char* e = getenv("EXL3_GEMV_XCD_LOCAL");
    return e && atoi(e) == 0;
  }();
  return !off && g_xcd_groups_ok.load(std::memory_order_relaxed) != 0;
}

static int xcd_local_chain(int nblk) { return nblk % 8 == 0 && xcd_groups_ok() ? 1 : 0; }

// launch_rows: 64 (two or four row groups per decoded tile past 16 rows; rotated launches only) or 16.  The
// workspace is checked here against the plans of exactly these launches (every entry point's size function sizes the
// same plans): a short workspace returns EXL3_ERR_INVALID before anything is launched.
static int launch_gemv(const ShardArgs& sa, const void* x, bool rotate, bool x_bf16, int rows, int k, int K, int cb,
                       int n_total, void* workspace, size_t workspace_bytes, void* y, bool y_bf16, hipStream_t st,
                       int launch_rows, const char* what) {
  const size_t need = gemv_workspace_bytes(rows, k, n_total, K, launch_rows, rotate);
  EXL3_CHECK_ARG(workspace && workspace_bytes >= need, "%s: workspace %zu bytes, need %zu", what, workspace_bytes,
                 need);
  const size_t partial_room = gemv_partial_bytes(rows, k, n_total, K, launch_rows, rotate);
  int* counters = static_cast<int*>(workspace);
  float* partial = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + counters_bytes(n_total));
  const bool pre = rotate && gemv_pre(rows, k, n_total);
  uint16_t* xh = reinterpret_cast<uint16_t*>(static_cast<uint8_t*>(workspace) + counters_bytes(n_total) +
                                             partial_room);
  if (pre) {
    const dim3 hgrid((unsigned)(((size_t)sa.count * rows * (k / 128) + 7) / 8));
    if (x_bf16)
      had_in_shards_kernel<true><<<hgrid, 256, 0, st>>>(x, rows, k, sa, xh);
    else
      had_in_shards_kernel<false><<<hgrid, 256, 0, st>>>(x, rows, k, sa, xh);
    EXL3_CHECK_LAUNCH();
  }
  launch_rows = gemv_launch_rows(k, n_total, launch_rows);
  for (int r0 = 0; r0 < rows; r0 += launch_rows) {
    const int M = std::min(launch_rows, rows - r0);
    // two or four row groups per decoded tile (rotated launches only: launch_rows is 16 otherwise)
    const bool quad = M > kGemvPairRows, pair = M > kGemvRows && !quad;
    const GemvPlan pl = gemv_plan(k, n_total, M, K, pre);
    EXL3_CHECK_ARG((size_t)pl.splits * M * n_total * sizeof(float) <= partial_room,
                   "%s: a launch of %d rows needs %zu bytes of partials, the workspace plan holds %zu", what, M,
                   (size_t)pl.splits * M * n_total * sizeof(float), partial_room);
    const dim3 grid(n_total / 128, pl.splits);
    const int xl = xcd_local_chain(n_total / 128);
    const void* xr = static_cast<const uint8_t*>(pre ? (const void*)xh : x) + (size_t)r0 * k * 2;
    void* yr = static_cast<uint8_t*>(y) + (size_t)r0 * n_total * 2;
    bool ok = false;
#define EXL3_GEMV_PAIR(NTV, PREV)                                                                                    \
  ok = EXL3_DISPATCH_K_CB(K, cb, (gemv_kernel<kK, kCB, true, NTV, PREV, 2><<<grid, kGemvThreads, pl.lds, st>>>(      \
      sa, xr, PREV ? 0 : (int)x_bf16, M, k, pl.splits, partial, counters, yr, (int)y_bf16, n_total, rows, xl)));
    if (pair) {  /* two row groups: the plan's LDS for 32 staged rows allows NT <= 32 */
      if (pl.nt == 16 && pre)
        EXL3_GEMV_PAIR(16, true)
      else if (pl.nt == 16)
        EXL3_GEMV_PAIR(16, false)
      else if (pre)
        EXL3_GEMV_PAIR(32, true)
      else
        EXL3_GEMV_PAIR(32, false)
    }
#undef EXL3_GEMV_PAIR
    // four row groups (narrow layers only, gemv_launch_rows): 64 staged rows at NT = 16 fit the default LDS
#define EXL3_GEMV_QUAD(PREV)                                                                                         \
  ok = EXL3_DISPATCH_K_CB(K, cb, (gemv_kernel<kK, kCB, true, 16, PREV, 4><<<grid, kGemvThreads, pl.lds, st>>>(       \
      sa, xr, PREV ? 0 : (int)x_bf16, M, k, pl.splits, partial, counters, yr, (int)y_bf16, n_total, rows, xl)));
    if (quad) {
      if (pl.nt != 16) return set_error(EXL3_ERR_INVALID, "four-group GEMV planned at NT = %d", pl.nt);
      if (pre)
        EXL3_GEMV_QUAD(true)
      else
        EXL3_GEMV_QUAD(false)
    }
#undef EXL3_GEMV_QUAD
#define EXL3_GEMV_LAUNCH(NTV)                                                                                        \
  if (!pair && !quad && pl.nt == NTV) {                                                                              \
    if (pre) /* the plan gives at most 32 with prepared rows */                                                      \
      ok = EXL3_DISPATCH_K_CB(K, cb, (gemv_kernel<kK, kCB, true, (NTV > 32 ? 32 : NTV), true><<<grid, kGemvThreads,  \
                                                                                             pl.lds, st>>>(          \
          sa, xr, 0, M, k, pl.splits, partial, counters, yr, (int)y_bf16, n_total, rows, xl)));                          \
    else if (rotate)                                                                                                 \
      ok = EXL3_DISPATCH_K_CB(K, cb, gemv_kernel<kK, kCB, true, NTV><<<grid, kGemvThreads, pl.lds, st>>>(           \
          sa, xr, (int)x_bf16, M, k, pl.splits, partial, counters, yr, (int)y_bf16, n_total, 0, xl));                \
    else                                                                                                             \
      ok = EXL3_DISPATCH_K_CB(K, cb, gemv_kernel<kK, kCB, false, NTV><<<grid, kGemvThreads, pl.lds, st>>>(          \
          sa, xr, (int)x_bf16, M, k, pl.splits, partial, counters, yr, (int)y_bf16, n_total, 0, xl));                \
  }
    EXL3_GEMV_LAUNCH(16)
    EXL3_GEMV_LAUNCH(32)
    EXL3_GEMV_LAUNCH(64)
#undef EXL3_GEMV_LAUNCH
    // 24 and 40 tile rows: one row group without prepared rows only
#define EXL3_GEMV_FEW(NTV)                                                                                           \
  if (!pair && !quad && !pre && pl.nt == NTV) {                                                                      \
    if (rotate)                                                                                                      \
      ok = EXL3_DISPATCH_K_CB(K, cb, gemv_kernel<kK, kCB, true, NTV><<<grid, kGemvThreads, pl.lds, st>>>(           \
          sa, xr, (int)x_bf16, M, k, pl.splits, partial, counters, yr, (int)y_bf16, n_total, 0, xl));                \
    else                                                                                                             \
      ok = EXL3_DISPATCH_K_CB(K, cb, gemv_kernel<kK, kCB, false, NTV><<<grid, kGemvThreads, pl.lds, st>>>(          \
          sa, xr, (int)x_bf16, M, k, pl.splits, partial, counters, yr, (int)y_bf16, n_total, 0, xl));                \
  }
    EXL3_GEMV_FEW(24)
    EXL3_GEMV_FEW(40)
#undef EXL3_GEMV_FEW
    if (!ok) return set_error(EXL3_ERR_INVALID, "unsupported K = %d / codebook = %d", K, cb);
    EXL3_CHECK_LAUNCH();
  }
  return EXL3_OK;
}

}  // namespace exl3

using namespace exl3;

// ---- scratch of the allocation-free entry point ----------------------------------------------------------------
// exl3_linear_noalloc runs the GEMV on this file-scope array instead of a caller's workspace: the same layout (the
// counter region, then the fp32 partials and rotated rows).  Every GPU the library runs on holds its own copy at its
// own address for the life of the process.  In host code `scratch` names a host-side stand-in, never the device
// memory: kernels and copies take the address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) uint8_t scratch[EXL3_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static void* g_scratch[kMaxDevices];
static std::mutex g_scratch_mu;

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// The scratch address on the device that `st` belongs to (the current device for the null stream), looked up (and
// its counter region cleared by a fill kernel on `st`) on the first call for that device.  The lookup runs with that
// device current, since hipGetSymbolAddress answers for the current device.  Every GEMV call leaves its counters at
// zero again, so clearing once is enough.
static int scratch_of_stream_device(hipStream_t st, void** out) {
  int cur = 0, dev = 0;
  EXL3_CHECK_HIP(hipGetDevice(&cur));
  dev = cur;
  if (st != nullptr) EXL3_CHECK_HIP(hipStreamGetDevice(st, &dev));
  EXL3_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "exl3_linear_noalloc: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch[dev] == nullptr) {
    if (dev != cur) EXL3_CHECK_HIP(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) EXL3_CHECK_HIP(hipSetDevice(cur));
    if (e != hipSuccess)
      return set_error(EXL3_ERR_HIP, "exl3_linear_noalloc: hipGetSymbolAddress: %s", hipGetErrorString(e));
    EXL3_CHECK_ARG(p != nullptr, "exl3_linear_noalloc: no device address for the scratch array");
    const int words = (int)(kCounterBytes / 4);
    zero_words_kernel<<<dim3((unsigned)((words + 255) / 256)), 256, 0, st>>>(static_cast<uint32_t*>(p), words);
    EXL3_CHECK_LAUNCH();
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return EXL3_OK;
}

extern "C" int exl3_xcd_local_chains(void) { return xcd_groups_ok() ? 1 : 0; }

extern "C" int exl3_reconstruct(const void* trellis, int k, int n, int K, int codebook, void* w_out, void* stream) {
  EXL3_CHECK_ARG(trellis && w_out, "exl3_reconstruct: null pointer");
  EXL3_CHECK_ARG(valid_bits(K) && valid_cb(codebook), "exl3_reconstruct: K = %d / codebook = %d", K, codebook);
  EXL3_CHECK_ARG(k > 0 && n > 0 && k % 16 == 0 && n % 16 == 0, "exl3_reconstruct: k = %d, n = %d", k, n);
  const int tk = k / 16, tn = n / 16;
  const dim3 grid((unsigned)(((size_t)tk * tn + 3) / 4));
  const bool ok = EXL3_DISPATCH_K_CB(K, codebook, reconstruct_kernel<kK, kCB><<<grid, 256, 0, as_stream(stream)>>>(
      static_cast<const uint32_t*>(trellis), tk, tn, static_cast<uint16_t*>(w_out)));
  if (!ok) return set_error(EXL3_ERR_INVALID, "exl3_reconstruct: unsupported K/codebook");
  EXL3_CHECK_LAUNCH();
  return EXL3_OK;
}

// ---- load-time layout (EXL3_LAYOUT_BLOCKS) -----------------------------------------------------------------------
// Tile (i, j) of the stored [k/16][n/16] tile grid goes to unit (j / 8, i / 8), position (j % 8) 8 + i % 8 of the unit:
// each (128-column block, 128-row block) unit is one contiguous run of 64 tiles, units in column block major order,
// and the 8 tiles of one tile column inside a unit are adjacent.  A workgroup of the balanced GEMV then reads one
// contiguous run (its units of a column block follow each other), each wave 256K contiguous bytes per unit.
// One thread moves one 16-byte piece; STORE_BLOCKS = false is the inverse map (unpack).
__host__ __device__ inline size_t blocks_tile_index(int i, int j, int KB) {
  return ((size_t)(j >> 3) * KB + (i >> 3)) * 64 + (j & 7) * 8 + (i & 7);
}

template <bool TO_BLOCKS>
__global__ __launch_bounds__(256) void repack_blocks_kernel(const uint4* __restrict__ in, int tk, int tn, int K,
                                                            uint4* __restrict__ out) {
  const size_t piece = (size_t)blockIdx.x * 256 + threadIdx.x;  // 16-byte piece of the stored layout
  const int per_tile = 2 * K;                                     // 16-byte pieces per tile
  if (piece >= (size_t)tk * tn * per_tile) return;
  const size_t tile = piece / per_tile;
  const int part = (int)(piece - tile * per_tile);
  const int i = (int)(tile / tn), j = (int)(tile - (size_t)i * tn);
  const size_t b = blocks_tile_index(i, j, tk / 8) * per_tile + part;
  if (TO_BLOCKS)
    out[b] = in[piece];
  else
    out[piece] = in[b];
}

static int trellis_relayout(const char* what, bool to_blocks, const void* in, int k, int n, int K, void* out,
                            void* stream) {
  EXL3_CHECK_ARG(in && out, "%s: null pointer", what);
  EXL3_CHECK_ARG(in != out, "%s: the output must not alias the input", what);
  EXL3_CHECK_ARG(valid_bits(K), "%s: K = %d", what, K);
  EXL3_CHECK_ARG(k > 0 && n > 0 && k % 128 == 0 && n % 128 == 0, "%s: k = %d, n = %d (multiples of 128)", what, k,
                 n);
  EXL3_CHECK_ARG((int64_t)k * n * K / 8 <= INT32_MAX, "%s: trellis exceeds the 2 GiB range", what);
  EXL3_CHECK_ARG(((uintptr_t)in | (uintptr_t)out) % 16 == 0, "%s: buffers must be 16-byte aligned", what);
  const int tk = k / 16, tn = n / 16;
  const size_t pieces = (size_t)tk * tn * 2 * K;
  const dim3 grid((unsigned)((pieces + 255) / 256));
  if (to_blocks)
    repack_blocks_kernel<true><<<grid, 256, 0, as_stream(stream)>>>(static_cast<const uint4*>(in), tk, tn, K,
                                                                     static_cast<uint4*>(out));
  else
    repack_blocks_kernel<false><<<grid, 256, 0, as_stream(stream)>>>(static_cast<const uint4*>(in), tk, tn, K,
                                                                      static_cast<uint4*>(out));
  EXL3_CHECK_LAUNCH();
  return EXL3_OK;
}

extern "C" int exl3_repack_trellis(const void* trellis, int k, int n, int K, void* out, void* stream) {
  return trellis_relayout("exl3_repack_trellis", true, trellis, k, n, K, out, stream);
}

extern "C" int exl3_unpack_trellis(const void* packed, int k, int n, int K, void* out, void* stream) {
  return trellis_relayout("exl3_unpack_trellis", false, packed, k, n, K, out, stream);
}

extern "C" int exl3_had_in_group(const void* x, int x_bf16, int rows, int k, const void* suh_cat, int shards,
                                 void* xh, void* stream) {
  EXL3_CHECK_ARG((rows == 0 || (x && xh)) && suh_cat, "exl3_had_in_group: null pointer");
  EXL3_CHECK_ARG(rows >= 0 && k > 0 && k % 128 == 0, "exl3_had_in_group: rows = %d, k = %d", rows, k);
  EXL3_CHECK_ARG(shards >= 1 && shards <= EXL3_MAX_SHARDS, "exl3_had_in_group: shards = %d", shards);
  if (rows == 0) return EXL3_OK;
  const size_t units = (size_t)shards * rows * (k / 128);
  const dim3 grid((unsigned)((units + 7) / 8));
  if (x_bf16)
    had_in_kernel<true><<<grid, 256, 0, as_stream(stream)>>>(x, rows, k, static_cast<const uint16_t*>(suh_cat), shards,
                                                             static_cast<uint16_t*>(xh));
  else
    had_in_kernel<false><<<grid, 256, 0, as_stream(stream)>>>(x, rows, k, static_cast<const uint16_t*>(suh_cat), shards,
                                                              static_cast<uint16_t*>(xh));
  EXL3_CHECK_LAUNCH();
  return EXL3_OK;
}

extern "C" int exl3_had_out_into(const void* y, int rows, int n, const void* svh, void* out, int out_bf16, int ld_out,
                                 int col0, void* stream) {
  EXL3_CHECK_ARG((rows == 0 || (y && out)) && svh, "exl3_had_out_into: null pointer");
  EXL3_CHECK_ARG(rows >= 0 && n > 0 && n % 128 == 0, "exl3_had_out_into: rows = %d, n = %d", rows, n);
  EXL3_CHECK_ARG(col0 >= 0 && col0 % 4 == 0 && ld_out >= col0 + n && ld_out % 4 == 0,
                 "exl3_had_out_into: col0 = %d, n = %d, ld_out = %d (4-aligned, in range)", col0, n, ld_out);
  if (rows == 0) return EXL3_OK;
  const size_t units = (size_t)rows * (n / 128);
  const dim3 grid((unsigned)((units + 7) / 8));
  if (out_bf16)
    had_out_kernel<true><<<grid, 256, 0, as_stream(stream)>>>(static_cast<const uint16_t*>(y), rows, n,
                                                              static_cast<const uint16_t*>(svh), out, ld_out, col0);
  else
    had_out_kernel<false><<<grid, 256, 0, as_stream(stream)>>>(static_cast<const uint16_t*>(y), rows, n,
                                                               static_cast<const uint16_t*>(svh), out, ld_out, col0);
  EXL3_CHECK_LAUNCH();
  return EXL3_OK;
}

extern "C" size_t exl3_linear_workspace_bytes(int rows, int k, int n_total, int K) {
  if (rows <= 0 || k <= 0 || n_total <= 0 || k % 128 || n_total % 128 || n_total / 128 > kMaxCounters ||
      !valid_bits(K))
    return 0;
  // exl3_linear's launches: up to 64 rows each (1, 2 or 4 row groups per decoded tile), then the remainder
  return gemv_workspace_bytes(rows, k, n_total, K, kGemvQuadRows, true);
}

extern "C" int exl3_linear(const void* x, int x_bf16, int rows, int k, const exl3_shard* shards_host, int nshards,
                           int K, int codebook, void* y, int y_bf16, void* workspace, size_t workspace_bytes,
                           void* stream) {
  EXL3_CHECK_ARG(rows == 0 || (x && y), "exl3_linear: null x / y");
  EXL3_CHECK_ARG(valid_bits(K) && valid_cb(codebook), "exl3_linear: K = %d / codebook = %d", K, codebook);
  EXL3_CHECK_ARG(rows >= 0 && k > 0 && k % 128 == 0, "exl3_linear: rows = %d, k = %d", rows, k);
  ShardArgs sa;
  int n_total = 0;
  if (int rc = build_shards(shards_host, nshards, k, K, &sa, &n_total)) return rc;
  if (rows == 0) return EXL3_OK;
  return launch_gemv(sa, x, true, x_bf16 != 0, rows, k, K, codebook, n_total, workspace, workspace_bytes, y,
                     y_bf16 != 0, as_stream(stream), kGemvQuadRows, "exl3_linear");
}

extern "C" size_t exl3_gemm_rotated_workspace_bytes(int rows, int k, int n, int K) {
  if (rows <= 0 || k <= 0 || n <= 0 || k % 128 || n % 128 || n / 128 > kMaxCounters || !valid_bits(K)) return 0;
  if (rows >= kPrefillRows) return prefill_plain_workspace_bytes(rows, k, n);
  return gemv_workspace_bytes(rows, k, n, K, kGemvRows, false);
}

// Rows are served by the kernel that serves the same row count in a linear: below kPrefillRows the decode-GEMV (one
// 16-row group per launch, two decoded tiles per MFMA), from there the prefill decode-GEMM, both without rotations.
extern "C" int exl3_gemm_rotated(const void* xh, int rows, int k, const void* trellis, int n, int K, int codebook,
                                 void* out, void* workspace, size_t workspace_bytes, void* stream) {
  EXL3_CHECK_ARG((rows == 0 || (xh && out)) && trellis, "exl3_gemm_rotated: null pointer");
  EXL3_CHECK_ARG(valid_bits(K) && valid_cb(codebook), "exl3_gemm_rotated: K = %d / codebook = %d", K, codebook);
  EXL3_CHECK_ARG(rows >= 0 && k > 0 && k % 128 == 0 && n > 0 && n % 128 == 0,
                 "exl3_gemm_rotated: rows = %d, k = %d, n = %d", rows, k, n);
  EXL3_CHECK_ARG((int64_t)k * n * K / 8 <= INT32_MAX, "exl3_gemm_rotated: trellis exceeds the 2 GiB buffer range");
  EXL3_CHECK_ARG(n / 128 <= kMaxCounters, "exl3_gemm_rotated: n = %d exceeds %d columns", n, kMaxCounters * 128);
  if (rows == 0) return EXL3_OK;
  if (rows >= kPrefillRows)
    return prefill_plain_gemm(xh, rows, k, trellis, n, K, codebook, out, workspace, workspace_bytes,
                              as_stream(stream));
  ShardArgs sa{};
  sa.trellis[0] = static_cast<const uint32_t*>(trellis);
  sa.tn[0] = n / 16;
  sa.blk0[1] = n / 128;
  sa.count = 1;
  return launch_gemv(sa, xh, false, false, rows, k, K, codebook, n, workspace, workspace_bytes, out, false,
                     as_stream(stream), kGemvRows, "exl3_gemm_rotated");
}

extern "C" size_t exl3_linear_noalloc_max_bytes(void) { return EXL3_NOALLOC_SCRATCH_BYTES; }

extern "C" int exl3_linear_noalloc(const void* x, int x_bf16, int rows, int k, const exl3_shard* shards_host,
                                   int nshards, int K, int codebook, void* y, int y_bf16, void* stream) {
  EXL3_CHECK_ARG(rows == 0 || (x && y), "exl3_linear_noalloc: null x / y");
  EXL3_CHECK_ARG(valid_bits(K) && valid_cb(codebook), "exl3_linear_noalloc: K = %d / codebook = %d", K, codebook);
  EXL3_CHECK_ARG(rows >= 0 && k > 0 && k % 128 == 0, "exl3_linear_noalloc: rows = %d, k = %d", rows, k);
  ShardArgs sa;
  int n_total = 0;
  if (int rc = build_shards(shards_host, nshards, k, K, &sa, &n_total)) return rc;
  if (rows == 0) return EXL3_OK;
  // 16 rows per launch here (the scratch need of the two-row-group launches would be larger)
  const size_t need = gemv_workspace_bytes(rows, k, n_total, K, kGemvRows, true);
  EXL3_CHECK_ARG(need <= (size_t)EXL3_NOALLOC_SCRATCH_BYTES,
                 "exl3_linear_noalloc: %d rows of %d -> %d need %zu bytes of scratch, the library holds %zu; use "
                 "exl3_linear with a workspace", rows, k, n_total, need, (size_t)EXL3_NOALLOC_SCRATCH_BYTES);
  hipStream_t st = as_stream(stream);
  void* ws = nullptr;
  if (int rc = scratch_of_stream_device(st, &ws)) return rc;
  return launch_gemv(sa, x, true, x_bf16 != 0, rows, k, K, codebook, n_total, ws, EXL3_NOALLOC_SCRATCH_BYTES, y,
                     y_bf16 != 0, st, kGemvRows, "exl3_linear_noalloc");
}
