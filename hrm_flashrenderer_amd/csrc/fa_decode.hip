// Paged-KV decode attention for gfx950 (few query rows per head, long context).
//
// Semantics: the reference's flash_attn_paged with M small (decode: M == 1,
// causal=False; engine/llama_tp.py:186-200), i.e. for query row (b, hq, i)
//   o = softmax_j(q . k_j / sqrt(D)) v_j over keys j < seqlen[b]
// (and k_off + j <= q_off + i when causal), with K/V of head head_map[hq]
// (flashattention_custom/ops.py:34-60, csrc/flash_attn_sm75.cu:213-425).
//
// Design (HBM-bound; every K/V byte is read once per KV head):
//  * The work is split evenly: the (sequence, KV head, 16-token group) units
//    of the whole batch are counted on the device from seqlen, and each of W
//    workgroups takes an equal contiguous range (see decode_kernel), so
//    variable context lengths leave no tail and no idle workgroups.
//  * A workgroup serves every query row that reads its KV head: all q heads of
//    the GQA group times the M query positions, packed as the 16 columns of
//    the MFMA tiles. K/V pages are therefore read once per KV head, not once
//    per query head.
//  * The segment's groups are dealt round-robin to the 4 waves, each keeping
//    its own running (max, sum, O) state and two groups in flight ahead of
//    the one it computes.
//  * S^T = K Q^T with v_mfma_f32_16x16x32_f16: lane (n, quarter) loads K row
//    n of the group as 16-byte vectors straight from HBM (no LDS). The
//    accumulator gives each lane 4 tokens of one query row, which is exactly
//    the B-operand layout of the P^T side of O^T = V^T P^T
//    (v_mfma_f32_16x16x16f16), so the softmax stays in registers.
//  * V^T needs 4 tokens of one d per lane. Each lane loads 4 token rows, D/16
//    consecutive d each (whole 256-byte rows across a quarter-wave), and the
//    d index of the MFMA output is relabelled d = (D/16)*m + j so that the
//    transpose is a byte permute inside the lane.
//  * Each wave keeps a per-row reference max in log2 units (scores times
//    log2(e)/sqrt(D)) and rescales O only when a group's max exceeds it by more
//    than 2^8. Partial (max, sum, O) of each (segment, workgroup) go to a
//    workspace; a combine kernel merges the partials of a row in log2 space.
#include "fa_common.h"

#include <algorithm>
#include <atomic>
#include <type_traits>

namespace fa {

namespace {

constexpr int kDecodeThreads = 256;  // 4 waves
constexpr int kDecodeWaves = 4;
constexpr int kRows = 16;            // query rows per MFMA column block
constexpr int kMaxHeads = 256;       // q heads scanned per KV head
constexpr int kMaxBatch = kDecodeMaxBatch;  // sequences whose unit prefix fits in LDS
constexpr int kDecodeMaxWgs = 1024;  // workgroup capacity of a decode workspace
static_assert(kMaxHeads == kDecodeThreads, "the head map is read one head per thread");

__device__ __forceinline__ float wave_max16x(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

__device__ __forceinline__ float wave_sum16x(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// Byte permute: (low half of x, low half of y) and (high half of x, high half of y).
__device__ __forceinline__ uint32_t pack_lo(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x07060302u);
}

template <int D>
struct DecodeRegs {
  static constexpr int KSTEPS = D / 32;  // 16x16x32 MFMAs for S^T
  static constexpr int DPL = D / 16;     // d values per lane and token for V^T
  static constexpr int VW = DPL / 2;     // dwords per V row fragment
  u32x4 k[KSTEPS];
  uint32_t v[4][VW];
};

// Cache policy of the K/V page loads: non-temporal (the "nt" bit). Every page
// is read exactly once per call, so it should not displace anything in the
// caches; on MI355X this raises the sustained rate of the page stream by ~10%.
constexpr int kStreamHint = 2;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);  // raw buffer, dword format (gfx9)
}

// Per-lane byte offsets of a group's fragments from its first row (loop
// invariant), with consecutive rows `rowb` bytes apart (2*D inside a page or
// in contiguous K/V, 2*Hk*D in the token-major cache): K row n, 16-byte chunks
// 2*quarter + 4*kk; V rows 4*quarter + i, DPL halves at DPL*n.
template <int D>
struct GroupLane {
  uint32_t k;
  uint32_t v;
  uint32_t rowb;
  __device__ GroupLane(int n, int quarter, uint32_t row_bytes)
      : k((uint32_t)n * row_bytes + 16u * (uint32_t)quarter),
        v(4u * (uint32_t)quarter * row_bytes + (uint32_t)(2 * (D / 16) * n)),
        rowb(row_bytes) {}
};

// Loads the K/V fragments of one 16-token group (rows beyond `t_end` or not
// addressable read as zero, so masked keys never carry NaN garbage into P V).
// ALIGNED (pages of a multiple of 16 tokens, or unpaged K/V: contiguous or
// token-major rows at a fixed stride): the group's rows are evenly spaced from
// one wave-uniform (scalar) lookup; the loads are raw buffer loads whose range
// covers only the group's valid rows, so rows past t_end come back as zeros
// with no per-lane address math.
template <int D, bool ALIGNED>
__device__ __forceinline__ void load_group(DecodeRegs<D>& r, const AttnParams& p, const f16* kp,
                                           const f16* vp, int b, int hk, int t0, int t_end,
                                           int n, int quarter, const GroupLane<D>& gl) {
  constexpr int KSTEPS = DecodeRegs<D>::KSTEPS;
  constexpr int DPL = DecodeRegs<D>::DPL;
  constexpr int VW = DecodeRegs<D>::VW;
  if constexpr (ALIGNED) {
    // A group at or past t_end gets an empty range: its loads are issued (so
    // the count of loads in flight does not depend on the path) but touch no
    // memory and return zeros.
    const int valid = min(16, t_end - t0);
    int64_t off = valid > 0 ? p.kv.row_offset(b, hk, t0) : -1;
    // rows [0, valid): the last valid row ends (valid - 1) * rowb + 2D bytes
    // in; row `valid` starts at valid * rowb >= that, so it reads as zero
    const uint32_t nbytes = off >= 0 ? (uint32_t)(valid - 1) * gl.rowb + (uint32_t)(2 * D) : 0u;
    off = off >= 0 ? off : 0;
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kp + off, nbytes);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vp + off, nbytes);
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk)
      r.k[kk] = __builtin_amdgcn_raw_buffer_load_b128(rk, gl.k + 64 * kk, 0, kStreamHint);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (VW == 4) {
        const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(rv, gl.v + i * gl.rowb, 0, kStreamHint);
#pragma unroll
        for (int w = 0; w < 4; ++w) r.v[i][w] = x[w];
      } else {
        const u32x2 x = __builtin_amdgcn_raw_buffer_load_b64(rv, gl.v + i * gl.rowb, 0, kStreamHint);
#pragma unroll
        for (int w = 0; w < VW; ++w) r.v[i][w] = x[w];
      }
    }
    return;
  }
  {
    const int row = t0 + n;
    const int64_t off = row < t_end ? p.kv.row_offset(b, hk, row) : -1;
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk) {
      if (off >= 0) {
        r.k[kk] = *reinterpret_cast<const u32x4*>(kp + off + 32 * kk + 8 * quarter);
      } else {
        r.k[kk] = u32x4{0u, 0u, 0u, 0u};
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = t0 + 4 * quarter + i;
    const int64_t off = row < t_end ? p.kv.row_offset(b, hk, row) : -1;
    if constexpr (VW == 4) {
      u32x4 x = u32x4{0u, 0u, 0u, 0u};
      if (off >= 0) x = *reinterpret_cast<const u32x4*>(vp + off + DPL * n);
#pragma unroll
      for (int w = 0; w < 4; ++w) r.v[i][w] = x[w];
    } else {
      u32x2 x = u32x2{0u, 0u};
      if (off >= 0) x = *reinterpret_cast<const u32x2*>(vp + off + DPL * n);
#pragma unroll
      for (int w = 0; w < VW; ++w) r.v[i][w] = x[w];
    }
  }
}

// Keys of sequence b that some query row can see: keys j < the returned
// limit. Padding rows (q_lens) see no keys, so a sequence without live rows
// has none.
__device__ __forceinline__ int visible_keys(const AttnParams& p, int b) {
  const int qlen = p.q_len(b);
  int kv_lim = qlen > 0 ? p.kv_len(b) : 0;
  if (p.causal) {
    const int64_t lim = (int64_t)p.q_off(b) + (qlen - 1) - p.k_off(b) + 1;
    if (lim < kv_lim) kv_lim = lim < 0 ? 0 : (int)lim;
  }
  return kv_lim > 0 ? kv_lim : 0;
}

__device__ __forceinline__ int key_groups(int keys) { return (keys + 15) >> 4; }

// s_units[b] = Hk * (visible groups of sequences before b), s_units[B] = total,
// computed by the whole workgroup: each thread sums a chunk of sequences, a
// shuffle scan within each wave and one exchange of the four wave totals give
// the prefix (two barriers, against seventeen for a 256-wide LDS scan: the
// unit prefix is the first thing every workgroup does). The visible key limit
// of each sequence is kept in s_keys[b] for the segments, so the key counts
// are read from memory once per workgroup. With the fused append, s_app[b]
// keeps the new token's position of sequence b (read in the same round trip).
__device__ __forceinline__ void unit_prefix(const AttnParams& p, int* s_units, int* s_part,
                                            int* s_keys, int* s_app) {
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  if (p.B == 1) {
    // one sequence (the token-major step): no scan
    if (tid == 0) {
      const int keys = visible_keys(p, 0);
      s_keys[0] = keys;
      if (s_app != nullptr) s_app[0] = p.seqlen[0];
      s_units[0] = 0;
      s_units[1] = (key_groups(keys) << p.kv_pair) * p.Hk;
    }
    __syncthreads();
    return;
  }
  const int chunk = (p.B + kDecodeThreads - 1) / kDecodeThreads;
  const int b0 = tid * chunk, b1 = min(p.B, b0 + chunk);
  int sum = 0;
  for (int b = b0; b < b1; ++b) {
    const int keys = visible_keys(p, b);
    s_keys[b] = keys;
    // the fused kernels run in advance mode only (fa_abi.hip): the new
    // token goes to position seqlen[b]
    if (s_app != nullptr) s_app[b] = p.seqlen[b];
    sum += (key_groups(keys) << p.kv_pair) * p.Hk;  // a pair's segment holds both heads' groups
  }
  int incl = sum;  // inclusive prefix of the chunk sums within the wave
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off);
    if (lane >= off) incl += y;
  }
  if (lane == 63) s_part[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += s_part[w];
  int run = base + incl - sum;
  for (int b = b0; b < b1; ++b) {
    s_units[b] = run;
    run += (key_groups(s_keys[b]) << p.kv_pair) * p.Hk;
  }
  if (tid == kDecodeThreads - 1) s_units[p.B] = base + incl;
  __syncthreads();
}

// Cost split of the unit list. A workgroup that starts a (b, hk) segment
// pays a dependent chain (key count, head scan, Q, page lookup, first K/V);
// with two workgroups per CU contending for memory, that takes about as long
// as streaming kSegmentCost units (p.dec_seg_cost; 0 for the one-per-CU
// per-row variant). Unit u costs u + P * seg(u), seg(u) = b * Hk + hk being
// its segment's index (empty segments included), and workgroup w owns the
// units whose cost lies in [floor(w * C / W), floor((w + 1) * C / W)),
// C = U + P * B * Hk. With P = 0 this is the plain equal split of units; P is
// 0 unless there are at least 2W units, so that every workgroup's cost range
// holds two or more costs. Measured against the equal split: cfg3 +5 %,
// cfg4 +1.5 %.
__device__ __forceinline__ int split_cost_p(const AttnParams& p, int U, int W) {
  return U >= 2 * W ? min(p.dec_seg_cost, U / (2 * W)) : 0;
}

// floor(x * y / z) for 0 <= x * y < 2^63, z > 0: a 32-bit division when the
// operands fit (the 64-bit one is several times longer).
__device__ __forceinline__ int64_t mul_div_floor(int64_t x, int64_t y, int64_t z) {
  const uint64_t n = (uint64_t)x * (uint64_t)y;
  if ((n >> 32) == 0 && ((uint64_t)z >> 32) == 0) return (int64_t)((uint32_t)n / (uint32_t)z);
  return (int64_t)(n / (uint64_t)z);
}

// floor(n / d) for 0 <= n < 2^63, d > 0: a 32-bit division when both fit.
__device__ __forceinline__ int64_t div_floor(int64_t n, int64_t d) {
  if (((uint64_t)n >> 32) == 0 && ((uint64_t)d >> 32) == 0) return (int64_t)((uint32_t)n / (uint32_t)d);
  return n / d;
}

// Units [u0, u1) of workgroup w under the cost split: u0 is the smallest unit
// whose cost is at least floor(w * C / W) (U for w == W), and units[b0] <= u0.
// Segment j = b * Hk + hk starts at cost units[b] + hk * G_b + P * j (G_b
// groups per segment of sequence b), which grows with j. The last segment
// starting at or below a cost T lies in the last sequence b whose first
// segment does, cs(b) = units[b] + P * Hk * b <= T, at hk = min(Hk - 1,
// (T - cs(b)) / (G_b + P)); the unit of cost T is T - P * j clamped to that
// segment's units. Each wave finds b by counting the sequences with
// cs(b) <= T, 64 per ballot (one LDS read per lane, no barrier), where a
// binary search would chain ~2 log2(B Hk) dependent LDS reads and divisions
// ahead of the workgroup's first page load.
struct SplitRange {
  int u0, u1, b0;
};
__device__ __forceinline__ SplitRange split_range(const int* units, int B, int Hk, int U, int W,
                                                  int P, int w, const FastDiv& wdiv) {
  const int64_t C = (int64_t)U + (int64_t)P * B * Hk;
  // floor(w * C / W) by the multiplicative inverse of W while (w + 1) * C
  // stays below 2^31, else by a division
  const bool small = C * W < ((int64_t)1 << 31);
  const int64_t T0 = small ? fdiv((int)(w * C), wdiv) : mul_div_floor(w, C, W);
  const int64_t T1 = small ? fdiv((int)((w + 1) * C), wdiv) : mul_div_floor(w + 1, C, W);
  const int lane = threadIdx.x & 63;
  int n0 = 0, n1 = 0;  // sequences b >= 1 with cs(b) <= T0, T1
  for (int base = 1; base < B; base += 64) {
    const int b = base + lane;
    const int64_t cs = b < B ? (int64_t)units[b] + (int64_t)P * Hk * b : C + 1;
    const uint64_t m1 = __ballot(cs <= T1);
    n0 += __popcll(__ballot(cs <= T0));
    n1 += __popcll(m1);
    if (m1 != ~0ull) break;  // cs grows with b: no later sequence qualifies
  }
  auto unit_at = [&](int64_t T, int b) -> int {
    if (T >= C) return U;
    if (P == 0) return (int)T;
    const int64_t cs = (int64_t)units[b] + (int64_t)P * Hk * b;
    const int G = (units[b + 1] - units[b]) / Hk;
    const int hk = (int)min((int64_t)Hk - 1, mul_div_floor(T - cs, 1, G + P));
    const int64_t start = (int64_t)units[b] + (int64_t)hk * G;
    const int64_t u = T - (int64_t)P * ((int64_t)b * Hk + hk);
    return (int)min(max(u, start), start + G);
  };
  SplitRange r;
  r.u0 = unit_at(T0, n0);
  r.u1 = unit_at(T1, n1);
  r.b0 = n0;
  return r;
}

// Balanced decode. The work is the list of units (sequence b, KV head hk,
// 16-key group g) in (b, hk, g) order; workgroup w of W takes a contiguous
// range of it under the cost split above (an equal share of units plus
// segment starts, whatever the sequence lengths). It
// walks the (b, hk) segments of its range; for each it runs all query rows
// of hk over its groups and writes one partial (max, sum, O) per row at slot
// b*Hk + hk + w. Along the unit list both the segment and the workgroup
// index are non-decreasing and at least one grows at every change, so
// segment + workgroup is unique per (segment, workgroup) pair.
//
// QSPLIT (fp32 Q, the token-major entry): the engine computes q . k in fp32
// (scripts/deepseek_native_engine.sh:573-577). Each query row is split into
// q_hi = fp16(q') and q_lo = fp16(q' - q_hi), q' = q * 2^-e, and S^T takes
// both through the matrix cores (exact fp16 x fp16 products, fp32 sums), so
// the scores carry about 22 bits of q instead of 11. The power of two 2^e
// keeps the largest |q'| of the row below 2^15 (e = 0 unless |q| >= 2^15, so
// a q beyond the fp16 range never becomes inf) and is folded back into the
// row's score scale.
//
// NBLK (1, 2 or 4): column blocks of 16 query rows served by one pass over
// the segment's K/V. A KV head with more than 16 * NBLK query rows (heads x
// positions) is walked once per 16 * NBLK rows.
//
// APPEND (the fused append of fa_flash_attn_paged_append_fwd in advance
// mode, without rotary tables): the new token of (b, hk) at position
// s = seqlen[b] is not read from the pages, which the combine kernel writes
// only after this kernel. The wave that owns the group of s loads that group
// and the lane's fragments of the token's K and V rows after its group loop,
// and puts them into the group's registers in place of the page row before
// the group is processed. Nothing here waits on the append.
template <int D, bool ALIGNED, bool QSPLIT, int NBLK, bool APPEND>
__global__ __launch_bounds__(kDecodeThreads) void decode_kernel(AttnParams p) {
  constexpr int KSTEPS = DecodeRegs<D>::KSTEPS;
  constexpr int DPL = DecodeRegs<D>::DPL;
  constexpr int VW = DecodeRegs<D>::VW;
  constexpr int OPAD = D + 4;

  __shared__ int s_hmap[kMaxHeads];   // KV head of every query head (-1: none)
  __shared__ int s_heads[kMaxHeads];
  __shared__ int s_count;
  __shared__ int s_units[kMaxBatch + 1];
  __shared__ int s_keys[kMaxBatch];      // visible key limit per sequence
  __shared__ int s_app[APPEND ? kMaxBatch : 1];  // fused append: new token's position
  __shared__ int s_part[kDecodeWaves];
  // Wave merge buffers: waves 2 and 3 hand their state to waves 0 and 1, which
  // then publish the pairwise merge (half the LDS of one slot per wave, so four
  // workgroups fit on a CU).
  __shared__ float s_m[2][kRows];
  __shared__ float s_l[2][kRows];
  __shared__ float s_o[2][kRows][OPAD];

  // The piece of the split this workgroup takes. Dispatch places workgroup
  // blockIdx on XCD blockIdx % 8, so XCD x takes pieces [x * W/8, (x+1) * W/8):
  // neighbouring pieces (the same KV heads and sequences) share an XCD
  // (token-major step +1.0 %, cfg4 +0.3 %, cfg3 +-0, same process). The
  // mapping is a bijection when 8 divides W, else the identity; the combine
  // kernel needs only the piece index.
  const int w = (gridDim.x & 7) == 0
                    ? (int)((blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3))
                    : (int)blockIdx.x;
  const int W = gridDim.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 15;       // MFMA column: query row within the block
  const int quarter = lane >> 4; // 0..3

  // The head map is read once, in the same round trip as the key counts of
  // the unit prefix (Hq <= kMaxHeads = one head per thread), so a segment's
  // head scan below reads LDS instead of waiting on memory.
  // (the KV head itself: with kv_pair, a segment's rows are its pair's heads)
  const int my_hk = tid < p.Hq ? p.kv_head_real(tid) : -1;
  unit_prefix(p, s_units, s_part, s_keys, APPEND ? s_app : nullptr);
  s_hmap[tid] = my_hk;
  __syncthreads();
  const int U = s_units[p.B];
  if (w == 0) {
    for (int b = tid; b <= p.B; b += kDecodeThreads) {
      p.ws_units[b] = s_units[b];
      if (APPEND && b < p.B) p.ws_app[b] = s_app[b];
      // an advance step whose token the append kernel wrote first: the
      // combine kernel bumps the lengths from this copy
      if (!APPEND && p.app_advance && b < p.B) p.ws_app[b] = p.seqlen[b];
    }
  }
  const int P = split_cost_p(p, U, W);
  const SplitRange range = split_range(s_units, p.B, p.Hk, U, W, P, w, p.dec_wdiv);
  // The range is wave-uniform; the LDS reads it comes from leave it in VGPRs,
  // and the buffer resources built from it would then be rebuilt per lane
  // (a readfirstlane loop around every K/V load).
  const int u0 = __builtin_amdgcn_readfirstlane(range.u0);
  const int u1 = __builtin_amdgcn_readfirstlane(range.u1);
  if (u0 >= u1) return;

  const f16* qp = reinterpret_cast<const f16*>(p.q);
  const f16* kp = reinterpret_cast<const f16*>(p.k);
  const f16* vp = reinterpret_cast<const f16*>(p.v);
  const float c = p.scale_log2;

  // One (b, hk) segment, groups [g_begin, g_end).
  auto segment = [&](int b, int hk, int g_begin, int g_stop, int slot) {
    // The key limit comes from LDS; the offsets are read only where a row
    // needs them (causal limits, rotary positions).
    const int qo = p.causal || p.rope_cos != nullptr ? p.q_off(b) : 0;
    const int ko = p.causal ? p.k_off(b) : 0;
    const int g_end = g_stop;
    // KV-head pairs (fp32-query split only): group g of the segment holds
    // keys 16 (g >> 1) .. of KV head 2 hk + (g & 1). One KV head's keys of the
    // token-major cache fall on a subset of the memory channels, and some
    // subsets serve more slowly (at the INT8 engine's shape two heads of
    // eight ended 5 us after the others); two heads per segment even out
    // the rates.
    const bool pair = QSPLIT && p.kv_pair != 0;
    const int t_end = pair ? s_keys[b] : min(s_keys[b], g_stop << 4);
    auto g_head = [&](int g) { return pair ? 2 * hk + (g & 1) : hk; };
    auto g_key0 = [&](int g) { return pair ? (g >> 1) << 4 : g << 4; };
    // key limit of group g's loads: past the segment nothing is read
    auto g_lim = [&](int g) { return pair && g >= g_end ? 0 : t_end; };

    // Groups g_begin + wave + 4k of the segment go through a ring of RING
    // register sets: RING - 1 groups are in flight while one is processed.
    // The first pass's loads leave before the head scan and the Q loads, so
    // the segment's first K/V bytes are in flight during both.
    // Two or four blocks at D = 128 compute two or four times as long per
    // group, so one group in flight covers the load latency and keeps the
    // accumulators in registers (two blocks, M = 4 over cfg4's pool: 5768
    // against 5699 GB/s with two groups in flight).
    constexpr int RING = NBLK >= 2 && D == 128 ? 2 : 3;
    DecodeRegs<D> ring[RING];
    // Row stride: 2D bytes in pages and contiguous K/V; the fp32-query
    // (token-major) variant reads rows Hk*D apart. A compile-time 2D keeps
    // the other variants' offsets constant (+0.3 % on cfg4).
    const uint32_t row_bytes =
        QSPLIT ? (uint32_t)(2 * (p.kv.paged ? (int64_t)D : p.kv.stride_tok)) : 2u * D;
    const GroupLane<D> glane(n, quarter, row_bytes);
    const int g0 = g_begin + wave;

    // Fused append (the step's new token at position seqlen[b], the
    // sequence's last key): its group g_app is the last group of the segment
    // and the last of the wave that owns it. After the group loop that wave
    // loads the group and the token's K and V rows, puts the token's row in
    // place of the page's and processes the group. So the group loop is the
    // plain kernel's, nothing of the token is held in registers across it,
    // and the group still comes last for its wave. The token replaces the
    // page row only where some row sees it and where the append writes it (a
    // mapped page).
    int r_app = 0;
    // With ALIGNED loads every prefetch is issued unconditionally (groups past
    // the end read as empty ranges), which keeps the number of loads in flight
    // the same on every path, so each group waits only for its own loads.
    auto prefetch = [&]() {
#pragma unroll
      for (int i = 0; i < RING - 1; ++i) {
        const int gi = g0 + i * kDecodeWaves;
        if (ALIGNED || gi < g_end)
          load_group<D, ALIGNED>(ring[i], p, kp, vp, b, g_head(gi), g_key0(gi), g_lim(gi), n,
                                 quarter, glane);
      }
    };
    prefetch();

    // Query heads that read KV head hk (any head_map, not only h / group).
    if (wave == 0) {
      int count = 0;
      for (int base = 0; base < p.Hq; base += 64) {
        const int hq = base + lane;
        const bool match = hq < p.Hq && (s_hmap[hq] >> (pair ? 1 : 0)) == hk;
        const uint64_t mask = __ballot(match);
        if (match) {
          const int pos = count + __popcll(mask & ((1ull << lane) - 1ull));
          if (pos < kMaxHeads) s_heads[pos] = hq;
        }
        count += __popcll(mask);
      }
      if (lane == 0) s_count = min(count, kMaxHeads);
    }
    __syncthreads();
    const int nrows = s_count * p.M;

    // NBLK column blocks of 16 query rows share each K/V group load: the K
    // rows are the A operand of every block's S^T, and the in-lane V^T
    // operand of every block's O^T.
    for (int rc0 = 0; rc0 < nrows; rc0 += kRows * NBLK) {
      if (rc0 > 0) prefetch();  // a later pass over the same groups
      int row_lim[NBLK];            // keys j < row_lim are visible to this lane's row
      bool blk_live[NBLK];          // the block holds at least one query row (uniform)
      half8 qreg[NBLK][KSTEPS];
      half8 qlo[NBLK][QSPLIT ? KSTEPS : 1];
      float crow[NBLK];             // score scale of this lane's row (log2 units)
      int row_par[NBLK];            // with KV-head pairs: which head of the pair the row reads
      float m_ref[NBLK];            // scaled (log2) reference max of the row
      float l_run[NBLK];
      floatx4 acc_o[NBLK][DPL];
#pragma unroll
      for (int bk = 0; bk < NBLK; ++bk) {
        // This lane's query row (column n of block bk's tiles).
        const int rc = rc0 + bk * kRows;
        blk_live[bk] = rc < nrows;
        const int ridx = rc + n;
        const bool row_ok = ridx < nrows;
        const int hq = row_ok ? s_heads[ridx / p.M] : 0;
        const int qi = row_ok ? ridx % p.M : 0;
        row_lim[bk] = t_end;
        row_par[bk] = pair ? (s_hmap[hq] & 1) : 0;
        if (p.causal) {
          int64_t lim = (int64_t)qo + qi - ko + 1;
          if (lim < row_lim[bk]) row_lim[bk] = lim < 0 ? 0 : (int)lim;
        }
        crow[bk] = c;
        const int64_t qrow_off = (((int64_t)b * p.Hq + hq) * p.M + qi) * D + 8 * quarter;
        if constexpr (QSPLIT) {
          const float* qf = reinterpret_cast<const float*>(p.q);
          floatx4 x[KSTEPS][2];
          float amax = 0.f;
#pragma unroll
          for (int kk = 0; kk < KSTEPS; ++kk) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              x[kk][h] = row_ok ? *reinterpret_cast<const floatx4*>(qf + qrow_off + 32 * kk + 4 * h)
                                : floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int j = 0; j < 4; ++j) amax = fmaxf(amax, fabsf(x[kk][h][j]));
            }
          }
          // the row's four quarters hold its D values
          amax = fmaxf(amax, __shfl_xor(amax, 16));
          amax = fmaxf(amax, __shfl_xor(amax, 32));
          int ex = 0;
          if (amax >= 32768.f && amax <= 3.0e38f) {
            (void)frexpf(amax, &ex);  // amax = f * 2^ex, f in [0.5, 1)
            ex -= 15;                 // amax * 2^-ex in [2^14, 2^15)
          }
          const float down = ldexpf(1.f, -ex);
          crow[bk] = c * ldexpf(1.f, ex);
#pragma unroll
          for (int kk = 0; kk < KSTEPS; ++kk) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              const float v = x[kk][j >> 2][j & 3] * down;
              const f16 hv = (f16)v;
              qreg[bk][kk][j] = hv;
              qlo[bk][kk][j] = (f16)(v - (float)hv);  // v - hv is exact in fp32
            }
          }
        } else {
#pragma unroll
          for (int kk = 0; kk < KSTEPS; ++kk) {
            qreg[bk][kk] = row_ok ? *reinterpret_cast<const half8*>(qp + qrow_off + 32 * kk)
                                  : half8{0, 0, 0, 0, 0, 0, 0, 0};
          }
          if (p.rope_cos != nullptr && row_ok)
            rope_fragment<KSTEPS, 32>(qreg[bk], p, qo + qi, 8 * quarter);
        }
        m_ref[bk] = -INFINITY;
        l_run[bk] = 0.f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc_o[bk][j] = floatx4{0.f, 0.f, 0.f, 0.f};
      }
      const half2v ones = half2v{(f16)1.f, (f16)1.f};

      // One 16-token group: S^T on the matrix cores, online softmax with a lazy
      // reference max (O is rescaled only when the max grows by more than 2^8),
      // then O^T += V^T P^T with the in-lane V transpose.
      auto process = [&](const DecodeRegs<D>& r, int t0, int gpar) {
        half4 pb[NBLK];
#pragma unroll
        for (int bk = 0; bk < NBLK; ++bk) {
          if (!blk_live[bk]) continue;
          floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kk = 0; kk < KSTEPS; ++kk) {
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, r.k[kk]),
                                                       qreg[bk][kk], s, 0, 0, 0);
          }
          if constexpr (QSPLIT) {
#pragma unroll
            for (int kk = 0; kk < KSTEPS; ++kk) {
              s = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, r.k[kk]),
                                                         qlo[bk][kk], s, 0, 0, 0);
            }
          }
          // lane holds tokens t0 + 4*quarter + i of row n; with KV-head pairs
          // a group of the pair's other head is invisible to the row
          const int lim = !pair || gpar == row_par[bk] ? row_lim[bk] : 0;
          float sv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) sv[i] = t0 + 4 * quarter + i < lim ? s[i] : -INFINITY;
          const float gmax =
              wave_max16x(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]))) * crow[bk];
          if (__builtin_amdgcn_ballot_w64(gmax > m_ref[bk] + 8.f) != 0) {
            const float m_new = fmaxf(m_ref[bk], gmax);
            const float alpha =
                m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_ref[bk] - m_new);
            l_run[bk] *= alpha;
#pragma unroll
            for (int j = 0; j < DPL; ++j) acc_o[bk][j] = acc_o[bk][j] * alpha;
            m_ref[bk] = m_new;
          }
          const float m_use = m_ref[bk] == -INFINITY ? 0.f : m_ref[bk];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            pb[bk][i] = (f16)__builtin_amdgcn_exp2f(__builtin_fmaf(sv[i], crow[bk], -m_use));
          l_run[bk] = __builtin_amdgcn_fdot2(half2v{pb[bk][0], pb[bk][1]}, ones, l_run[bk], false);
          l_run[bk] = __builtin_amdgcn_fdot2(half2v{pb[bk][2], pb[bk][3]}, ones, l_run[bk], false);
        }
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const int w = j >> 1;
          uint32_t lo, hi;
          if ((j & 1) == 0) {
            lo = pack_lo(r.v[0][w], r.v[1][w]);
            hi = pack_lo(r.v[2][w], r.v[3][w]);
          } else {
            lo = pack_hi(r.v[0][w], r.v[1][w]);
            hi = pack_hi(r.v[2][w], r.v[3][w]);
          }
          const half4 a = __builtin_bit_cast(half4, u32x2{lo, hi});
#pragma unroll
          for (int bk = 0; bk < NBLK; ++bk) {
            if (blk_live[bk])
              acc_o[bk][j] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pb[bk], acc_o[bk][j], 0, 0, 0);
          }
        }
      };

      // the group loop's end: the new token's group (fused append) is left
      // to its owner wave, after the loop
      int g_loop = g_end;
      bool app_owner = false;
      if constexpr (APPEND) {
        const int s = __builtin_amdgcn_readfirstlane(s_app[b]);
        const bool seen = s >= 0 && s < t_end && (s >> 4) >= g_begin && (s >> 4) == g_end - 1 &&
                          p.kv.row_offset(b, hk, s) >= 0;
        if (seen) {
          g_loop = s >> 4;
          r_app = s & 15;
          app_owner = ((g_loop - g_begin) & (kDecodeWaves - 1)) == wave;
        }
      }
      for (int g = g0; g < g_loop; g += RING * kDecodeWaves) {
#pragma unroll
        for (int i = 0; i < RING; ++i) {
          const int gi = g + i * kDecodeWaves;
          if (gi >= g_loop) break;
          const int gl = gi + (RING - 1) * kDecodeWaves;
          if (ALIGNED || gl < g_loop)
            load_group<D, ALIGNED>(ring[(i + RING - 1) % RING], p, kp, vp, b, g_head(gl),
                                   g_key0(gl), g_lim(gl), n, quarter, glane);
          process(ring[i], g_key0(gi), gi & 1);
        }
      }
      if constexpr (APPEND) {
        if (app_owner) {
          DecodeRegs<D> app_regs;
          load_group<D, ALIGNED>(app_regs, p, kp, vp, b, hk, g_loop << 4, t_end, n, quarter,
                                 glane);
          const int64_t row = ((int64_t)b * p.Hk + hk) * D;
          // K: the lane's chunks 8*quarter + 32*kk of the row (row n of a group)
          u32x4 app_k[KSTEPS];
#pragma unroll
          for (int kk = 0; kk < KSTEPS; ++kk)
            app_k[kk] = *reinterpret_cast<const u32x4*>(p.app_k + row + 8 * quarter + 32 * kk);
          // V: the lane's DPL dims at DPL * n (of rows 4*quarter + i)
          uint32_t app_v[VW];
          const uint32_t* vr = reinterpret_cast<const uint32_t*>(p.app_v + row + DPL * n);
#pragma unroll
          for (int w2 = 0; w2 < VW; ++w2) app_v[w2] = vr[w2];
          // the token's row in place of the page's
          if (n == r_app) {
#pragma unroll
            for (int kk = 0; kk < KSTEPS; ++kk) app_regs.k[kk] = app_k[kk];
          }
          if (quarter == (r_app >> 2)) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              if (i == (r_app & 3)) {
#pragma unroll
                for (int w2 = 0; w2 < VW; ++w2) app_regs.v[i][w2] = app_v[w2];
              }
            }
          }
          process(app_regs, g_loop << 4, 0);
        }
      }
      (void)VW;

      // Merge the 4 waves' states block by block: m is uniform per row, l
      // needs the 4 lanes of a row summed, O^T[j][r] sits at
      // d = DPL*(4*quarter + r) + j. Waves 2, 3 pass their state to waves 0,
      // 1 (in registers there), which publish the pair merge; the workgroup
      // then merges the two pairs per element.
#pragma unroll
      for (int bk = 0; bk < NBLK; ++bk) {
        if (!blk_live[bk]) continue;
        const int rc = rc0 + bk * kRows;
        const float l_blk = wave_sum16x(l_run[bk]);
        const int half = wave & 1;
        if (wave >= 2) {
          if (quarter == 0) {
            s_m[half][n] = m_ref[bk];
            s_l[half][n] = l_blk;
          }
#pragma unroll
          for (int j = 0; j < DPL; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) s_o[half][n][DPL * (4 * quarter + r) + j] = acc_o[bk][j][r];
          }
        }
        __syncthreads();
        if (wave < 2) {
          const float m_o = s_m[half][n];
          const float mx = fmaxf(m_ref[bk], m_o);
          const float a = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_ref[bk] - mx);
          const float bsc = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_o - mx);
          const float l_pair = l_blk * a + s_l[half][n] * bsc;
#pragma unroll
          for (int j = 0; j < DPL; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float& x = s_o[half][n][DPL * (4 * quarter + r) + j];
              x = acc_o[bk][j][r] * a + x * bsc;
            }
          }
          // all lanes of the row have read s_m / s_l before they are replaced
          __builtin_amdgcn_wave_barrier();
          if (quarter == 0) {
            s_m[half][n] = mx;
            s_l[half][n] = l_pair;
          }
        }
        __syncthreads();

        for (int e = tid; e < kRows * D; e += kDecodeThreads) {
          const int row = e / D;
          const int d = e - row * D;
          const int ri = rc + row;
          if (ri >= nrows || ri >= p.dec_rows) continue;  // rows past the slot: NaN in the combine
          const float m0 = s_m[0][row], m1 = s_m[1][row];
          const float mx = fmaxf(m0, m1);
          float lsum = 0.f, osum = 0.f;
          if (mx != -INFINITY) {
            const float a0 = __builtin_amdgcn_exp2f(m0 - mx);
            const float a1 = __builtin_amdgcn_exp2f(m1 - mx);
            lsum = a0 * s_l[0][row] + a1 * s_l[1][row];
            osum = a0 * s_o[0][row][d] + a1 * s_o[1][row][d];
          }
          // partial rows are indexed by (rank of the q head among the KV head's
          // query heads, query position): ri < heads_per_kv * M
          const int64_t srow = (int64_t)slot * p.dec_rows + ri;
          p.ws_o[srow * D + d] = osum;
          if (d == 0) {
            p.ws_ml[srow * 2 + 0] = mx;
            p.ws_ml[srow * 2 + 1] = lsum;
          }
        }
        __syncthreads();
      }
    }

  };

  // The segments of [u0, u1), from the sequence the split found.
  int b = __builtin_amdgcn_readfirstlane(range.b0);
  for (int u = u0; u < u1;) {
    while (s_units[b + 1] <= u) ++b;
    const int G = fdiv(s_units[b + 1] - s_units[b], p.hk_div);
    const int rel = u - s_units[b];
    const int hk = rel / G;
    const int g_lo = rel - hk * G;
    const int uend = min(u1, s_units[b] + (hk + 1) * G);
    segment(b, hk, g_lo, g_lo + (uend - u), b * p.Hk + hk + w);
    u = uend;
  }
}


// The fused append's page writes, done by workgroups of the combine grid of
// their own (after the merge workgroups), so that their load -> page lookup
// -> store chain runs beside the merge instead of before it; the combine
// kernel runs after every read of the pages. Row (b, hk) of app_k / app_v
// goes to position ws_app[b] of the pages, one 16-byte chunk per lane,
// skipped where the page is not mapped or beyond the capacity, as
// paged_append_kernel skips it (no rows when app_k is null: the append
// kernel wrote them before the decode kernel). With app_advance, seqlen[b]
// becomes ws_app[b] + 1, the length the decode kernel read plus the token.
// `first` and `nthreads` give this thread's lanes of the grid-stride loop.
template <int D>
__device__ __forceinline__ void fused_append_writes(const AttnParams& p, int64_t first,
                                                    int64_t nthreads) {
  f16* kd = reinterpret_cast<f16*>(const_cast<void*>(p.k));
  f16* vd = reinterpret_cast<f16*>(const_cast<void*>(p.v));
  constexpr int kPerRow = D / 8;
  const int64_t total = p.app_k != nullptr ? (int64_t)p.B * p.Hk * kPerRow : 0;
  for (int64_t e = first; e < total; e += nthreads) {
    const int64_t row = e / kPerRow;
    const int c = (int)(e - row * kPerRow);
    const int b = (int)((uint32_t)row / (uint32_t)p.Hk);  // row < B * Hk < 2^31
    const int hk = (int)(row - (int64_t)b * p.Hk);
    const int pos = p.ws_app[b];
    if (pos < 0) continue;
    const int64_t dst = p.kv.row_offset(b, hk, pos);
    if (dst < 0) continue;
    const f16* ks = p.app_k + row * D;
    const f16* vs = p.app_v + row * D;
    *reinterpret_cast<u32x4*>(kd + dst + 8 * c) = *reinterpret_cast<const u32x4*>(ks + 8 * c);
    *reinterpret_cast<u32x4*>(vd + dst + 8 * c) = *reinterpret_cast<const u32x4*>(vs + 8 * c);
  }
  if (p.app_advance) {
    int32_t* sl = const_cast<int32_t*>(p.seqlen);
    for (int64_t b = first; b < p.B; b += nthreads) sl[b] = p.ws_app[b] + 1;
  }
}

// Merges the partials of one query row (one wave per row (b, hq, i)): the
// workgroups whose unit range meets the row's segment are recomputed from the
// unit prefix the decode kernel stored.
// WIDE = false: one wave per row, four rows per workgroup. WIDE = true (few
// rows, each with many slots, as with one long sequence): one workgroup of
// kWideWaves waves per row, wave w merges slots wa + w, wa + w + kWideWaves,
// ..., and wave 0 merges the waves' states.
constexpr int kWideWaves = 8;
template <int D, bool WIDE>
__global__ __launch_bounds__(WIDE ? 64 * kWideWaves : 256) void decode_combine_kernel(AttnParams p) {
  constexpr int DPW = D / 64;  // d values per lane
  const int total = p.B * p.Hq * p.M;
  const int merge_wgs = WIDE ? total : (total + 3) / 4;
  if ((int)blockIdx.x >= merge_wgs) {
    // the fused append's workgroups (launch_combine adds them)
    const int64_t nthreads = (int64_t)(gridDim.x - merge_wgs) * blockDim.x;
    fused_append_writes<D>(p, (int64_t)(blockIdx.x - merge_wgs) * blockDim.x + threadIdx.x,
                           nthreads);
    return;
  }
  const int wave = threadIdx.x >> 6;
  const int row = WIDE ? (int)blockIdx.x : (int)blockIdx.x * 4 + wave;
  const int lane = threadIdx.x & 63;
  if (row >= total) return;
  const int qi = row % p.M;
  const int hq = (row / p.M) % p.Hq;
  const int b = row / (p.M * p.Hq);

  const int hk = p.kv_head(hq);
  // The decode kernel stores the partial rows of KV head hk's query heads in
  // head order: row rank(hq) * M + qi of the slot, rank(hq) = number of heads
  // before hq that read hk. A head map that sends more heads to hk than the
  // slots hold (heads_per_kv) leaves the heads past it without partials: NaN.
  int rank = 0;
  if (hk >= 0) {
    for (int base = 0; base < hq; base += 64) {
      const int h2 = base + lane;
      rank += __popcll(__ballot(h2 < hq && p.kv_head(h2) == hk));
    }
  }
  const int ri = rank * p.M + qi;
  float result[DPW];
  // With an advance step, this kernel advances seqlen: the key count comes
  // from the length the decode kernel published.
  const int kv_len = p.app_advance ? min(max(p.ws_app[b] + 1, 0), p.N) : p.kv_len(b);
  if (qi >= p.q_len(b)) {
    // padding row (q_lens): zeros
#pragma unroll
    for (int k = 0; k < DPW; ++k) result[k] = 0.f;
  } else if (hk < 0 || ri >= p.dec_rows) {
#pragma unroll
    for (int k = 0; k < DPW; ++k) result[k] = __builtin_nanf("");
  } else if (kv_len == 0) {
    // Zero keys: softmax over an empty row times an empty V is zero
    // (flashattention_custom/ops.py:39, 52-59 with slen == 0).
#pragma unroll
    for (int k = 0; k < DPW; ++k) result[k] = 0.f;
  } else {
    const int U = p.ws_units[p.B];
    const int G = (p.ws_units[b + 1] - p.ws_units[b]) / p.Hk;
    const int US = p.ws_units[b] + hk * G;
    const int UE = US + G;
    const int W = p.dec_wgs;
    const int64_t rbase = (int64_t)(b * p.Hk + hk) * p.dec_rows + ri;
    float mx = -INFINITY, lsum = 0.f;
    float acc[DPW];
#pragma unroll
    for (int k = 0; k < DPW; ++k) acc[k] = 0.f;
    // workgroups owning the segment's units under the decode kernel's cost split
    const int P = split_cost_p(p, U, W);
    const int64_t C = (int64_t)U + (int64_t)P * p.B * p.Hk;
    const int64_t seg_cost = (int64_t)P * (b * p.Hk + hk);
    if (G > 0) {
      const int wa = (int)min((int64_t)W - 1, div_floor((US + seg_cost + 1) * W - 1, C));
      const int wb = (int)min((int64_t)W - 1, div_floor((UE + seg_cost) * W - 1, C));
      const int first = WIDE ? wa + wave : wa;
      constexpr int STEP = WIDE ? kWideWaves : 1;
      // Slots in batches with every load issued before the merge (8 per wave
      // with a workgroup of 8 waves per row, so the 64 slots of a row of the
      // token-major step, with its KV-head pairs, take one round trip);
      // slots of workgroups with an empty unit range were never written.
      constexpr int kBatch = WIDE ? 8 : 4;
      for (int w0 = first; w0 <= wb; w0 += kBatch * STEP) {
        float pm[kBatch], pl[kBatch], po[kBatch][DPW];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
          const int w = w0 + i * STEP;
          // a piece's cost range is empty only when the cost is below the
          // piece count (C < W): the divisions are skipped otherwise
          const bool live =
              w <= wb && (C >= W || mul_div_floor(w, C, W) != mul_div_floor(w + 1, C, W));
          const int64_t srow = rbase + (int64_t)w * p.dec_rows;
          pm[i] = live ? p.ws_ml[srow * 2] : -INFINITY;
          pl[i] = live ? p.ws_ml[srow * 2 + 1] : 0.f;
#pragma unroll
          for (int k = 0; k < DPW; ++k) po[i][k] = live ? p.ws_o[srow * D + lane + 64 * k] : 0.f;
        }
        float bm = mx;
#pragma unroll
        for (int i = 0; i < kBatch; ++i) bm = fmaxf(bm, pm[i]);
        if (bm == -INFINITY) continue;
        const float r = __builtin_amdgcn_exp2f(mx - bm);  // mx == -inf gives 0
        lsum *= r;
#pragma unroll
        for (int k = 0; k < DPW; ++k) acc[k] *= r;
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
          const float sc = __builtin_amdgcn_exp2f(pm[i] - bm);
          lsum += sc * pl[i];
#pragma unroll
          for (int k = 0; k < DPW; ++k) acc[k] += sc * po[i][k];
        }
        mx = bm;
      }
    }
    if constexpr (WIDE) {
      __shared__ float s_mx[kWideWaves], s_l[kWideWaves];
      __shared__ float s_acc[kWideWaves][D];
      if (lane == 0) {
        s_mx[wave] = mx;
        s_l[wave] = lsum;
      }
#pragma unroll
      for (int k = 0; k < DPW; ++k) s_acc[wave][lane + 64 * k] = acc[k];
      __syncthreads();
      if (wave != 0) return;
      float m_all = s_mx[0];
#pragma unroll
      for (int w = 1; w < kWideWaves; ++w) m_all = fmaxf(m_all, s_mx[w]);
      lsum = 0.f;
#pragma unroll
      for (int k = 0; k < DPW; ++k) acc[k] = 0.f;
      if (m_all != -INFINITY) {
#pragma unroll
        for (int w = 0; w < kWideWaves; ++w) {
          const float sc = __builtin_amdgcn_exp2f(s_mx[w] - m_all);  // -inf slot: 0
          lsum += sc * s_l[w];
#pragma unroll
          for (int k = 0; k < DPW; ++k) acc[k] += sc * s_acc[w][lane + 64 * k];
        }
      }
    }
    // No visible key (lsum == 0): 0 * inf = NaN, the reference's result for a
    // fully masked row.
    const float inv = 1.f / lsum;
#pragma unroll
    for (int k = 0; k < DPW; ++k) result[k] = acc[k] * inv;
  }
  if (WIDE && wave != 0) return;
  if (p.o_f32) {
    float* of = reinterpret_cast<float*>(p.o) + (int64_t)row * D;
#pragma unroll
    for (int k = 0; k < DPW; ++k) of[lane + 64 * k] = result[k];
  } else {
    f16* op = reinterpret_cast<f16*>(p.o) + (int64_t)row * D;
#pragma unroll
    for (int k = 0; k < DPW; ++k) op[lane + 64 * k] = (f16)result[k];
  }
}

// The decode kernel variant a call runs: row loads from whole 16-token
// groups (ALIGNED: pages of a multiple of 16 tokens, or unpaged rows at a
// fixed stride whose 16-row span fits a buffer range), the fp32-query split
// (the token-major entry, one row block per pass), and the row blocks served
// per K/V pass: enough 16-row blocks for a KV head's query rows
// (heads_per_kv * M = dec_rows), up to 4.
struct DecodeVariant {
  bool aligned;
  bool qsplit;
  int nblk;
  bool append;  // fused append (at most two row blocks: fused_append_ok)
};

// Row blocks per pass: four (64 rows), except the per-row load variant at
// D = 128, whose four blocks spill; it walks larger groups in passes of 32
// rows. At D = 128 the four-block variant keeps one 16-key group in flight
// per wave (their O accumulators alone take 128 registers).
constexpr int max_row_blocks(int D, bool aligned) { return D == 128 && !aligned ? 2 : 4; }

DecodeVariant decode_variant(const AttnParams& p) {
  DecodeVariant v;
  v.qsplit = p.q_f32 != 0;
  // Unpaged rows D apart (contiguous K/V), or, with the fp32 query split
  // (whose variant takes the row stride at run time), any stride whose 16-row
  // span fits a 32-bit buffer range.
  v.aligned = p.kv.paged ? (p.kv.PS % 16) == 0
            : v.qsplit   ? p.kv.stride_tok >= p.kv.D && p.kv.stride_tok <= ((int64_t)1 << 24)
                         : p.kv.stride_tok == p.kv.D;
  const int want = p.dec_rows <= kRows ? 1 : p.dec_rows <= 2 * kRows ? 2 : 4;
  v.nblk = v.qsplit ? 1 : std::min(want, max_row_blocks(p.kv.D, v.aligned));
  v.append = p.app_k != nullptr;
  return v;
}

template <int D, bool ALIGNED>
const void* decode_fn_rows(int nblk, bool append) {
  constexpr int NB4 = max_row_blocks(D, ALIGNED) >= 4 ? 4 : 2;
  if (append)
    return nblk == 1 ? reinterpret_cast<const void*>(&decode_kernel<D, ALIGNED, false, 1, true>)
                     : reinterpret_cast<const void*>(&decode_kernel<D, ALIGNED, false, 2, true>);
  return nblk == 1 ? reinterpret_cast<const void*>(&decode_kernel<D, ALIGNED, false, 1, false>)
       : nblk == 2 ? reinterpret_cast<const void*>(&decode_kernel<D, ALIGNED, false, 2, false>)
                   : reinterpret_cast<const void*>(&decode_kernel<D, ALIGNED, false, NB4, false>);
}

template <int D>
const void* decode_fn(DecodeVariant v) {
  if (v.qsplit)
    return v.aligned ? reinterpret_cast<const void*>(&decode_kernel<D, true, true, 1, false>)
                     : reinterpret_cast<const void*>(&decode_kernel<D, false, true, 1, false>);
  return v.aligned ? decode_fn_rows<D, true>(v.nblk, v.append)
                   : decode_fn_rows<D, false>(v.nblk, v.append);
}

int decode_grid_wgs(int D, DecodeVariant var) {
  // One workgroup per CU of the current device (when the variant fits a CU at
  // all), cached per device and kernel variant: every workgroup takes its
  // equal share in a single round. Against as many workgroups as are resident
  // (two per CU for most variants), same process: token-major +7.8 %, cfg3
  // +2.2 %, cfg4 +1.1 %. Two workgroups on a CU share its memory pipeline
  // unevenly (the older one is served first), so the younger half ends late,
  // and each workgroup's prologue and merge are paid over half the units.
  // A partial second round (e.g. 320 or 384 workgroups) is slower still.
  static std::atomic<int> cache[64][64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  const int blk = var.nblk == 1 ? 0 : var.nblk == 2 ? 1 : 2;
  const int idx = (var.append ? 32 : 0) + (D == 128 ? 16 : 0) + blk * 4 + (var.qsplit ? 2 : 0) +
                  (var.aligned ? 1 : 0);
  int v = cache[dev][idx].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int cus = 0, per_cu = 0;
  const void* fn = D == 128 ? decode_fn<128>(var) : decode_fn<64>(var);
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kDecodeThreads, 0) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  v = per_cu > 0 ? cus : 0;
  if (v > 0) cache[dev][idx].store(v, std::memory_order_relaxed);
  return v;
}

}  // namespace

bool use_decode_path(int B, int M, int Hq, int Hk, int heads_per_kv) {
  // (a batch of more than kDecodeMaxBatch sequences runs in launches of at
  // most that many: the unit prefix of one launch lives in LDS)
  if (Hk <= 0 || Hq > kMaxHeads || B < 0 || M < 1) return false;
  const int64_t rows = (int64_t)M * ((Hq + Hk - 1) / Hk);  // query rows per KV head
  if (rows <= 2 * kRows) return true;
  // With M < 128 and a heads_per_kv bound, the prefill kernel packs a KV
  // head's (head, position) rows into 128-row tiles: one pass over its pages
  // for all of them at prefill MFMA rates. That wins once the tiles fill the
  // device; with fewer, the decode kernels (split over the whole device)
  // serve the rows in passes of up to 64. Over cfg4's pool at 64/8 heads,
  // M = 16 (two decode passes): B = 1 82 us decode against 293 packed, B = 16
  // 358 against 361, B = 32 (256 tiles) packed 396, B = 64 559 against 1281;
  // M = 8 (one decode pass, half-empty tiles): B = 32 350 decode against 389
  // packed, B = 64 (512 tiles) 512 packed against 651.
  const bool packable = heads_per_kv >= 2 && M < 128;
  if (packable) {
    const int64_t hpk = std::min(heads_per_kv, Hq);
    const int64_t tiles = (int64_t)B * Hk * ((hpk * M + 127) / 128);
    if (tiles >= (rows <= 4 * kRows ? 2 : 1) * kPackedMinTiles) return false;
  }
  return rows <= 4 * kRows || (packable && rows <= 16 * kRows);
}

bool fused_append_ok(int B, int M, int Hq, int Hk, int heads_per_kv) {
  if (!use_decode_path(B, M, Hq, Hk, heads_per_kv)) return false;
  const int64_t hpk = heads_per_kv <= 0 || heads_per_kv > Hq ? Hq : heads_per_kv;
  return hpk * M <= 2 * kRows;
}

int decode_launch_wgs(const DecodePlan& plan, const AttnParams& p, int D) {
  const int r = decode_grid_wgs(D, decode_variant(p));
  return r > 0 ? std::min(plan.wgs, r) : plan.wgs;
}

DecodePlan plan_decode(int B, int Hq, int M, int D, int Hk, int capacity_tokens,
                       int heads_per_kv) {
  DecodePlan plan;
  B = std::min(B, kDecodeMaxBatch);  // the sequences of one launch
  // Workspace capacity: up to kDecodeMaxWgs workgroups, but not more than the
  // largest possible number of 16-key groups divided by 8. The launch uses
  // min(this, one workgroup per CU).
  const int64_t max_units = (int64_t)B * Hk * ((capacity_tokens + 15) / 16);
  const int64_t wgs = std::min<int64_t>(kDecodeMaxWgs, std::max<int64_t>(1, max_units / 8));
  plan.wgs = (int)wgs;
  // a slot holds the rows of one KV head's query heads
  const int hpk = heads_per_kv <= 0 || heads_per_kv > Hq ? Hq : heads_per_kv;
  plan.rows = hpk * M;
  const size_t slots = (size_t)B * Hk + (size_t)plan.wgs;
  plan.o_bytes = (slots * plan.rows * D * sizeof(float) + 255) / 256 * 256;
  plan.ml_bytes = (slots * plan.rows * 2 * sizeof(float) + 255) / 256 * 256;
  // unit prefix [B + 1], then the fused append's positions [B]
  plan.ws_bytes = plan.o_bytes + plan.ml_bytes + (size_t)(2 * B + 1) * sizeof(int);
  return plan;
}

// Rows with many partial slots (few rows: one long sequence, or a few) merge
// with a workgroup per row; otherwise a wave per row.
// With the fused append, workgroups for its page writes follow the merge
// workgroups in the same grid (one lane per chunk, at most 1024 workgroups).
template <int D>
void launch_combine(const AttnParams& p, int rows, hipStream_t stream) {
  int64_t app_wgs = 0;
  if (p.app_k != nullptr || p.app_advance) {
    // page rows (fused append) or only the lengths (advance after the append kernel)
    const int64_t lanes = p.app_k != nullptr ? (int64_t)p.B * p.Hk * (D / 8) : (int64_t)p.B;
    app_wgs = std::min<int64_t>(1024, std::max<int64_t>(1, (lanes + 255) / 256));
  }
  if (rows <= 512)
    hipLaunchKernelGGL((decode_combine_kernel<D, true>), dim3((unsigned)(rows + app_wgs)),
                       dim3(64 * kWideWaves), 0, stream, p);
  else
    hipLaunchKernelGGL((decode_combine_kernel<D, false>),
                       dim3((unsigned)((rows + 3) / 4 + app_wgs)), dim3(256), 0, stream, p);
}

hipError_t launch_decode(const AttnParams& p_in, int D, hipStream_t stream) {
  AttnParams p = p_in;
  p.dec_wdiv = make_fastdiv(p.dec_wgs);
  p.hk_div = make_fastdiv(p.Hk);
  const dim3 grid((unsigned)p.dec_wgs);
  const int rows = p.B * p.Hq * p.M;
  const DecodeVariant var = decode_variant(p);
  const dim3 block(kDecodeThreads);
  const void* fn = D == 128 ? decode_fn<128>(var) : decode_fn<64>(var);
  void* args[] = {const_cast<AttnParams*>(&p)};
  hipError_t e = hipLaunchKernel(fn, grid, block, args, 0, stream);
  if (e != hipSuccess) return e;
  if (D == 128)
    launch_combine<128>(p, rows, stream);
  else
    launch_combine<64>(p, rows, stream);
  return hipGetLastError();
}

}  // namespace fa
