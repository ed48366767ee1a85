// Per-wave weight streaming for the decode-GEMV family (dense linear, MoE experts).
//
// One wave owns one tile column (16 output columns) and NT tile rows (NB = NT/8 blocks of 128 rows) of a trellis.
// A block's 8 tiles of that column (8 x 32K bytes, one tile row apart) arrive with one or two wave-wide
// 16-byte-per-lane gathers -- the texture addresser spends the same cycles on a 4-byte and a 16-byte lane, so wide
// lanes cut its work about 8x against per-tile dword gathers -- are written to a wave-private LDS stage, and each
// lane reads the two dwords of its group per tile from LDS (lane geometry of exl3_device.hpp).  Three blocks are in
// flight in registers.  Everything is straight-line code (NT is a template parameter): no loop-carried load
// registers, exact in-order vmcnt waits.  A stream shorter than NT rows (a split's tail) clamps its loads to its
// last block; the caller gives it zero activations past its end.
//
// Decoded tiles are rounded fp16 weights, bit-identical to trellis_core's (reference.py:52-73; the reference kernel's
// __hadd, codebook.cuh:56-75).  Two consecutive tiles of the wave's column feed one MFMA 16x16x32 f16 per 16-row
// group: the lane's 4 weights of tile 2v and its 4 of tile 2v+1 are the 8-half B fragment, against the activations
// staged by the caller in the matching order (a_slot).  On gfx950 a 16x16x16 f16 MFMA takes as many cycles as a
// 16x16x32 one, so one MFMA per tile pair is half the matrix-core time of one per tile.
#pragma once
#include "exl3_device.hpp"

namespace exl3 {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// LDS bytes of one wave's stream: two block stages, each 256 K bytes (the block's data), or, with every lane loading
// (ALL_LANES), one 1 KB gather slot (64 lanes x 16 B) per 64 chunks
__host__ __device__ constexpr int stream_lds_bytes(int K, bool all_lanes = false) {
  return all_lanes ? 2 * ((16 * K + 63) / 64) * 1024 : 2 * 256 * K;
}

// Every lane issues every gather: lanes past the last chunk read from beyond the buffer's end (zeros, no memory
// request).  A lane-conditional load is a branch the compiler must assume taken or skipped, so the number of loads
// younger than a given one becomes path-dependent and its in-order load waits turn into vmcnt(0): with the lane mask
// (48 of 64 lanes at K = 3) the dense GEMV's first decode waited for all three blocks in flight and every later block
// for the one issued after it (layer set at one row 80.1 -> 75.7 us, same call).
// ALL_LANES: lanes past the last chunk also write their stage slot, so no stage write is lane-conditional either (the
// MoE chunk pipeline, whose loop keeps loads in flight across iterations).
template <int K, int CB, int NT, bool ALL_LANES = false>
struct TileStream {
  static constexpr int NB = NT / 8;               // 128-row blocks
  static constexpr int CHUNKS = 16 * K;           // 16-byte chunks in the 8 tiles of one block column
  static constexpr int LPB = (CHUNKS + 63) / 64;  // wave-wide gathers per block
  static constexpr int STAGE = ALL_LANES ? LPB * 1024 : 256 * K;  // bytes of one block stage
  static constexpr int LDS_BYTES = 2 * STAGE;                        // per wave
  static_assert(LDS_BYTES == stream_lds_bytes(K, ALL_LANES), "stage size");
  // a lane offset past every buffer this stream reads (matrices stay below 2^31 bytes; offset + block offset never
  // wraps 32 bits)
  static constexpr int kOutOfRange = 0x7FFFFFF0;

  __amdgpu_buffer_rsrc_t rsrc;
  int soff0, row_bytes, bstride, nb, lane;
  int goff[LPB];
  bool glive[LPB];
  u32x4_t buf[NB][LPB];
  uint8_t* stage;
  LaneGeo g;

  // trellis: base of the matrix (int16 [k/16, n/16, 16K], or the EXL3_LAYOUT_BLOCKS form when `blocks`, with KB
  // 128-row blocks); total_bytes: its size; tile_col: the wave's tile column; kb0: first 128-row block; nblocks:
  // blocks holding data (1..NB); stage_lds: the wave's LDS_BYTES.  Both layouts put the block's 8 tiles of the
  // column in the same stage order (tile row r at stage byte 32K r).
  __device__ __forceinline__ void init(const void* trellis, int total_bytes, int tn, int tile_col, int kb0,
                                       int nblocks, uint8_t* stage_lds, int l, bool blocks = false, int KB = 0) {
    const int tile_bytes = 32 * K;
    row_bytes = tn * tile_bytes;
    rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)trellis, (short)0, total_bytes, 0x00020000);
    soff0 = blocks ? ((tile_col >> 3) * KB + kb0) * 64 * tile_bytes + (tile_col & 7) * 8 * tile_bytes
                   : kb0 * 8 * row_bytes + tile_col * tile_bytes;
    bstride = blocks ? 64 * tile_bytes : 8 * row_bytes;
    nb = nblocks;
    lane = l;
    stage = stage_lds;
    g = lane_geo<K>(l & 15, l >> 4);
    // chunk L = i*64 + lane -> tile row L / (2K) of the block, 16-byte piece L % (2K); it lands at stage byte 16 L,
    // so each tile sits contiguously at stage byte 32K * row
#pragma unroll
    for (int i = 0; i < LPB; i++) {
      const int L = i * 64 + l;
      glive[i] = L < CHUNKS;
      goff[i] = !glive[i] ? kOutOfRange : blocks ? 16 * L : (L / (2 * K)) * row_bytes + (L % (2 * K)) * 16;
    }
  }

  __device__ __forceinline__ void issue(int b) {
    const int so = soff0 + min(b, nb - 1) * bstride;
#pragma unroll
    for (int i = 0; i < LPB; i++)
      buf[b][i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rsrc, goff[i], so, 0));
  }

  // the first three blocks; call before staging the activations so their latency overlaps
  __device__ __forceinline__ void start() {
    issue(0);
    if constexpr (NB > 1) issue(1);
    if constexpr (NB > 2) issue(2);
  }

  // One row group: ap is the lane's 8-half A fragment of tile rows 0 and 1 (a_slot order), 4 half8 per tile-row
  // pair; two accumulators alternate so that consecutive MFMAs do not wait for each other.  Returns the 16 x 16 fp32
  // C tile slice (lane l: rows 4(l/16)..+3, column l%16).
  __device__ __forceinline__ float4_t run_pairs(const half8_t* ap) {
    static_assert(NT % 2 == 0, "tile-row pairs");
    float4_t acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int b = 0; b < NB; b++) {
      uint8_t* st = stage + (b & 1) * STAGE;
#pragma unroll
      for (int i = 0; i < LPB; i++)
        if (ALL_LANES || glive[i]) *reinterpret_cast<u32x4_t*>(st + 16 * (i * 64 + lane)) = buf[b][i];
      if (b + 3 < NB) issue(b + 3);
      const uint32_t* tw = reinterpret_cast<const uint32_t*>(st);
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const uint32_t* t0 = tw + 2 * v * 8 * K;
        const half8_t bv = decode_two_groups<K, CB>(t0[g.dw0], t0[g.dw1], t0[8 * K + g.dw0], t0[8 * K + g.dw1], g);
        if (v & 1)
          acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ap[(b * 4 + v) * 4], bv, acc1, 0, 0, 0);
        else
          acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ap[(b * 4 + v) * 4], bv, acc0, 0, 0, 0);
      }
    }
    return acc0 + acc1;
  }

  // For up to P groups of 16 A rows sharing each decoded tile pair (groups <= P active, uniform): group p reads its
  // 8-half fragment gstride half8 after group p-1's and accumulates into acc[p] (one chain per group: the decode
  // between two MFMAs of a group covers their dependency).
  template <int P>
  __device__ __forceinline__ void run_groups(const half8_t* ap, int gstride, int groups, float4_t (&acc)[P]) {
    static_assert(NT % 2 == 0, "tile-row pairs");
#pragma unroll
    for (int b = 0; b < NB; b++) {
      uint8_t* st = stage + (b & 1) * STAGE;
#pragma unroll
      for (int i = 0; i < LPB; i++)
        if (ALL_LANES || glive[i]) *reinterpret_cast<u32x4_t*>(st + 16 * (i * 64 + lane)) = buf[b][i];
      if (b + 3 < NB) issue(b + 3);
      const uint32_t* tw = reinterpret_cast<const uint32_t*>(st);
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const uint32_t* t0 = tw + 2 * v * 8 * K;
        const half8_t bv = decode_two_groups<K, CB>(t0[g.dw0], t0[g.dw1], t0[8 * K + g.dw0], t0[8 * K + g.dw1], g);
#pragma unroll
        for (int p = 0; p < P; p++)
          if (p == 0 || p < groups)
            acc[p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ap[p * gstride + (b * 4 + v) * 4], bv, acc[p], 0, 0, 0);
      }
    }
  }
};

// A-operand staging in LDS, in the order of the tile-pair MFMAs: position p of the k-range (tile row u = p / 16,
// r = p % 16), row m -> m * mstride + 32 (u / 2) + 8 q + 4 (u & 1) + e with q = (r & 7) >> 1,
// e = (r & 1) | (r >> 3) << 1.  Lane (m, q) then reads its 8-half fragment [tile row 2v: rows 2q, 2q+1, 2q+8, 2q+9;
// tile row 2v+1: the same rows] -- the row order of the decoded group -- as one 16-byte word, at a 64-byte step per
// tile-row pair.  The order permutes positions inside each 32-position block only, so rows prepared in this order
// (the rotation kernels that write prepared rows) are staged by plain copies.  mstride = 16 * tile rows + 8 keeps the
// rows 16-byte aligned and the 16 rows of a read 16 bytes apart in the banks.
__host__ __device__ constexpr int a_mstride(int NT) { return NT * 16 + 8; }
__device__ __forceinline__ int a_slot(int p, int m, int mstride) {
  const int r = p & 15, u = p >> 4;
  return m * mstride + ((u >> 1) << 5) + (((r & 7) >> 1) << 3) + ((u & 1) << 2) + ((r & 1) | ((r >> 3) << 1));
}

}  // namespace exl3
