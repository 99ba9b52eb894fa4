// Shared definitions of the gfx950 attention kernels: vector types, the page
// map (logical page -> physical page -> element offset), and the launcher
// prototypes the C-ABI layer (fa_abi.hip) dispatches to.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fa {

typedef _Float16 f16;
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

// Where the K/V rows of one (sequence, KV head) live.
//
// Contiguous K/V [B, Hk, N, D]: row j of (b, hk) is at ((b*Hk + hk)*N + j)*D;
// in general b*stride_nb + hk*stride_hk + j*stride_tok, which also covers the
// token-major cache [N, Hk, D] (stride_hk = D, stride_tok = Hk*D).
// Paged K/V [NB, Hk, P, PS, D]: logical page p = j / PS of sequence b maps to
// a physical id phi (identity b*P + p, or block_table[b*max_blocks + p]), and
// the row sits at (((phi/P)*Hk + hk)*P + phi%P)*PS*D + (j%PS)*D. The map follows
// the reference's PagedAccessor (csrc/flash_attn_sm75.cu:54-86) with the block
// table as an additive indirection.
struct KVMap {
  const int32_t* block_table;  // nullable
  int64_t stride_nb;           // Hk*P*PS*D (paged) ; Hk*N*D (contiguous)
  int64_t stride_hk;           // P*PS*D           ; N*D
  int64_t stride_page;         // PS*D             ; unused
  int64_t stride_tok;          // unused           ; D (Hk*D token-major)
  int max_blocks;              // logical pages per sequence (P without table)
  int P;                       // pages per row of the pool
  int num_phys;                // NB*P: valid physical ids are [0, num_phys)
  int PS;                      // tokens per page
  int ps_shift;                // log2(PS) when PS is a power of two, else -1
  int D;
  int paged;                   // 0: contiguous K/V

  // Element offset of row j of (b, hk); -1 when the row is not addressable
  // (page beyond the capacity or an out-of-range physical id). With uniform
  // arguments every step is scalar: the block table is read through the
  // constant address space (s_load), and the physical id is split into
  // (pool row, page) only when the pool has more than one row.
  __device__ __forceinline__ int64_t row_offset(int b, int hk, int j) const {
    if (!paged) return (int64_t)b * stride_nb + (int64_t)hk * stride_hk + (int64_t)j * stride_tok;
    unsigned page, slot;
    if (ps_shift >= 0) {
      page = (unsigned)j >> ps_shift;
      slot = (unsigned)j & (unsigned)(PS - 1);
    } else {
      page = (unsigned)j / (unsigned)PS;
      slot = (unsigned)j - page * (unsigned)PS;
    }
    if (page >= (unsigned)max_blocks) return -1;
    unsigned nb, pp;
    if (block_table != nullptr) {
      typedef const __attribute__((address_space(4))) int32_t ctable;
      const int phi = ((ctable*)block_table)[(int64_t)b * max_blocks + page];
      if ((unsigned)phi >= (unsigned)num_phys) return -1;
      if (num_phys <= P) {
        nb = 0;
        pp = (unsigned)phi;
      } else {
        nb = (unsigned)phi / (unsigned)P;
        pp = (unsigned)phi - nb * (unsigned)P;
      }
    } else {
      nb = (unsigned)b;
      pp = page;
    }
    return (int64_t)nb * stride_nb + (int64_t)hk * stride_hk + (int64_t)pp * stride_page +
           (int64_t)slot * D;
  }
};

// n / d for 0 <= n < 2^31 and 1 <= d < 2^31 by one high multiply: the
// round-up method of Granlund and Montgomery ("Division by invariant integers
// using multiplication", PLDI 1994). With s = ceil(log2 d) and
// m = floor(2^32 (2^s - d) / d) + 1, n / d = (umulhi(n, m) + n) >> s; the sum
// fits 32 bits because umulhi(n, m) <= n < 2^31. Built on the host, so the
// kernels' index arithmetic is a few instructions instead of a reciprocal
// and a correction sequence per division.
struct FastDiv {
  uint32_t m;
  uint32_t s;
  int d;
};

inline FastDiv make_fastdiv(int d) {
  FastDiv f;
  d = d < 1 ? 1 : d;  // never divided by: the entry points return before launch on empty shapes
  f.d = d;
  uint32_t s = 0;
  while ((1ull << s) < (uint64_t)d) ++s;
  f.s = s;
  f.m = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << s) - (uint64_t)d)) / (uint64_t)d + 1);
  return f;
}

__device__ __forceinline__ int fdiv(int n, const FastDiv& f) {
  return (int)((__umulhi((uint32_t)n, f.m) + (uint32_t)n) >> f.s);
}

// Per-call arguments of the attention kernels (both contiguous and paged).
struct AttnParams {
  const void* q;      // [B, Hq, M, D]
  const void* k;      // contiguous [B, Hk, N, D] or pool [NB, Hk, P, PS, D]
  const void* v;
  void* o;            // [B, Hq, M, D]
  const int32_t* seqlen;    // paged: [B]; contiguous: nullptr (all N)
  const int32_t* head_map;  // paged: [Hq]; contiguous: nullptr (h / group)
  const int32_t* q_offsets; // nullable [B]
  const int32_t* k_offsets; // nullable [B]
  const int32_t* q_lens;    // nullable [B]: rows >= q_lens[b] of sequence b are padding
                            // (not computed; written as zeros)
  KVMap kv;
  int B, Hq, Hk, M, N;  // N: contiguous key count, or per-sequence capacity in tokens
  int group;            // Hq / Hk (contiguous head mapping)
  int causal;
  int q_offset, k_offset;
  float scale_log2;     // log2(e) / sqrt(D)
  // balanced decode scratch: partial results of (segment, workgroup) pairs at
  // slot = segment + workgroup, segment = b*Hk + hk (see fa_decode.hip)
  float* ws_o;          // [B*Hk + dec_wgs, dec_rows, D]
  float* ws_ml;         // [B*Hk + dec_wgs, dec_rows, 2]  (log2 max, sum)
                        // row rank * M + i of a slot: query position i of the
                        // rank-th q head (in head order) that reads the slot's KV head
  int* ws_units;        // [B + 1] units (16-key groups x Hk) before sequence b
  int dec_wgs;          // workgroups of the decode kernel
  int dec_seg_cost;     // units charged per segment start in the decode split (fa_decode.hip)
  int dec_rows;         // row capacity of a slot: heads_per_kv * M
  FastDiv dec_wdiv;     // dec_wgs and Hk as divisors (set by launch_decode)
  FastDiv hk_div;
  // optional rotary embedding of Q at load time (nullptr: none): fp16 tables
  // [rope_len, D/2]; query row i of sequence b sits at position q_off(b) + i
  const f16* rope_cos;
  const f16* rope_sin;
  int rope_len;
  // decode only: fp32 Q and O (converted on load / store) and, without a head
  // map, the q-head -> KV-head map hq % Hk (instead of hq / group)
  int q_f32;
  int o_f32;
  int head_mod;
  // decode with the fp32-query split only: 1 when each segment serves a pair
  // of KV heads (2j, 2j + 1), alternating their 16-key groups; Hk then counts
  // the pairs, and kv_head() gives a q head's pair (kv_head_real() its head)
  int kv_pair;
  // prefill with M < 128 rows per q head: > 0 packs the (head, position) rows
  // of each KV head's q heads into 128-row tiles, at most pack_heads heads
  // per KV head (fa_prefill.hip); 0 keeps one q head per tile
  int pack_heads;
  // Append of one new token per (sequence, KV head) fused into the decode
  // step (fa_flash_attn_paged_append_fwd, advance mode). app_k / app_v
  // [B, Hk, 1, D] go to position seqlen[b] of the pages (k / v), the length
  // before the append. The decode kernel takes the token's row from app_k /
  // app_v, and the combine kernel, which runs after every page read, writes
  // it into the pages and stores seqlen[b] + 1. With app_advance the
  // attention sees seqlen[b] + 1 keys, also on the kernels that take the
  // step without the fused path (the append kernel ran first).
  const f16* app_k;              // nullptr: no fused append
  const f16* app_v;
  int app_advance;               // 0 or 1
  int* ws_app;                   // [B] positions the decode kernel publishes to the combine kernel

  __device__ __forceinline__ int q_off(int b) const { return q_offsets ? q_offsets[b] : q_offset; }
  __device__ __forceinline__ int k_off(int b) const { return k_offsets ? k_offsets[b] : k_offset; }
  // Query rows of sequence b that are not padding, in [0, M].
  __device__ __forceinline__ int q_len(int b) const {
    if (q_lens == nullptr) return M;
    const int n = q_lens[b];
    return n < 0 ? 0 : n > M ? M : n;
  }
  // Number of keys of sequence b (clamped to the capacity).
  __device__ __forceinline__ int kv_len(int b) const {
    if (seqlen == nullptr) return N;
    int n = seqlen[b] + app_advance;
    n = n < 0 ? 0 : n;
    return n > N ? N : n;
  }
  // K/V head of query head hq, or -1 if the head map points outside the
  // heads; with kv_pair, the head's pair.
  __device__ __forceinline__ int kv_head(int hq) const {
    if (kv_pair == 0) {
      if (head_map == nullptr) return head_mod ? hq % Hk : hq / group;
      int hk = head_map[hq];
      return (hk >= 0 && hk < Hk) ? hk : -1;
    }
    const int r = kv_head_real(hq);
    return r < 0 ? -1 : r >> 1;
  }
  // The K/V head itself (the same as kv_head without kv_pair).
  __device__ __forceinline__ int kv_head_real(int hq) const {
    const int nh = Hk << kv_pair;
    if (head_map == nullptr) return head_mod ? hq % nh : hq / group;
    int hk = head_map[hq];
    return (hk >= 0 && hk < nh) ? hk : -1;
  }
};

// One rotary pair in the fp16 operation order of the reference's apply_rope
// (engine/rope.py:15-24, half-split layout): y1 = x1*c - x2*s, y2 = x1*s + x2*c
// with every product and the sum rounded to fp16. Each step is one fp32
// operation rounded to fp16; fp32 carries more than 2*11+2 bits, so this is
// the correctly rounded fp16 operation, the same result torch's fp16 ops give.
__device__ __forceinline__ void rope_pair(f16 x1, f16 x2, f16 c, f16 s, f16& y1, f16& y2) {
  // each product is rounded before the sum: no fused multiply-add
#pragma clang fp contract(off)
  const f16 a = (f16)((float)x1 * (float)c);
  const f16 b = (f16)((float)x2 * (float)s);
  const f16 e = (f16)((float)x1 * (float)s);
  const f16 f = (f16)((float)x2 * (float)c);
  y1 = (f16)((float)a - (float)b);
  y2 = (f16)((float)e + (float)f);
}

// Rotary embedding of the query fragment a lane holds: q[i] holds dims
// base + STRIDE*i + (0..7) of one query row, N*STRIDE == D, so the partner
// d + D/2 of a dim d < D/2 is in q[i + N/2] at the same element. Rows at a
// position outside the table become NaN.
template <int N, int STRIDE>
__device__ __forceinline__ void rope_fragment(half8* q, const AttnParams& p, int pos, int base) {
  constexpr int HALF = N * STRIDE / 2;
  const bool ok = pos >= 0 && pos < p.rope_len;
  const int64_t row = (int64_t)(ok ? pos : 0) * HALF + base;
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const half8 c = *reinterpret_cast<const half8*>(p.rope_cos + row + STRIDE * i);
    const half8 s = *reinterpret_cast<const half8*>(p.rope_sin + row + STRIDE * i);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      f16 y1, y2;
      rope_pair(q[i][j], q[i + N / 2][j], c[j], s[j], y1, y2);
      q[i][j] = ok ? y1 : (f16)__builtin_nanf("");
      q[i + N / 2][j] = ok ? y2 : (f16)__builtin_nanf("");
    }
  }
}

// rope_fragment in two steps, so that the table loads can leave early: the
// tables' rows for the fragment (c[i], s[i] for i < N/2), then the rotation
// (ok: the position is inside the table; otherwise NaN).
template <int N, int STRIDE>
__device__ __forceinline__ void rope_tables(half8* c, half8* s, const AttnParams& p, int pos,
                                            int base) {
  constexpr int HALF = N * STRIDE / 2;
  const bool ok = pos >= 0 && pos < p.rope_len;
  const int64_t row = (int64_t)(ok ? pos : 0) * HALF + base;
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    c[i] = *reinterpret_cast<const half8*>(p.rope_cos + row + STRIDE * i);
    s[i] = *reinterpret_cast<const half8*>(p.rope_sin + row + STRIDE * i);
  }
}
template <int N>
__device__ __forceinline__ void rope_rotate(half8* q, const half8* c, const half8* s, bool ok) {
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      f16 y1, y2;
      rope_pair(q[i][j], q[i + N / 2][j], c[i][j], s[i][j], y1, y2);
      q[i][j] = ok ? y1 : (f16)__builtin_nanf("");
      q[i + N / 2][j] = ok ? y2 : (f16)__builtin_nanf("");
    }
  }
}

// Launchers (return hipSuccess or the launch error).
hipError_t launch_paged_append(void* k_pages, void* v_pages, const void* k_new, const void* v_new,
                               const KVMap& map, int B, int Hk, int T, int start_pos,
                               const int32_t* start_positions, const int32_t* token_positions,
                               const f16* rope_cos, const f16* rope_sin, int rope_len,
                               hipStream_t stream);
hipError_t launch_prefill(const AttnParams& p, int D, int dtype, hipStream_t stream);
hipError_t launch_decode(const AttnParams& p, int D, hipStream_t stream);

// Sequences of one decode launch: a larger batch runs in launches of at most
// this many consecutive sequences, one after another on the stream, which
// share the workspace (plan_decode sizes it for one launch).
constexpr int kDecodeMaxBatch = 2048;

// Decode sizing (host side; depends on sizes only).
struct DecodePlan {
  int wgs;          // workgroup capacity of the workspace
  int rows;         // row capacity of a partial slot
  size_t o_bytes;   // partial O, 256-byte aligned
  size_t ml_bytes;  // partial (max, sum), 256-byte aligned
  size_t ws_bytes;  // total, including the unit prefix
};
// heads_per_kv: most q heads one KV head serves (<= 0: Hq, no assumption).
DecodePlan plan_decode(int B, int Hq, int M, int D, int Hk, int capacity_tokens,
                       int heads_per_kv);
// Workgroups to launch for a plan on the current device (<= plan.wgs), for the
// decode kernel variant the arguments select.
int decode_launch_wgs(const DecodePlan& plan, const AttnParams& p, int D);
// Units a segment start is charged in the paged decode split: the dependent
// chain that opens a (sequence, KV head) segment, measured in streamed units
// with two decode workgroups per CU (a sweep of 0-32 peaks at 12-16 for both
// benchmark decode shapes).
constexpr int kSegmentCost = 12;
// Whether paged attention with M query rows per sequence runs on the decode
// kernels (split over the device, partial results merged by a second
// kernel; needs the workspace of plan_decode) or on the prefill kernel.
constexpr int kPackedMinTiles = 256;
bool use_decode_path(int B, int M, int Hq, int Hk, int heads_per_kv);
// Whether a paged call with a fused append (one new token per sequence, at
// position seqlen[b]) runs the append inside the decode kernels: the decode path
// with at most two 16-row blocks of query rows per KV head (the fused
// variants keep the new token's fragments in registers beside them).
bool fused_append_ok(int B, int M, int Hq, int Hk, int heads_per_kv);
// seqlen[b] += 1 for b < B (the fused append's advance when the step does
// not run on the fused decode kernels).
hipError_t launch_advance_lengths(int32_t* seqlen, int B, hipStream_t stream);

}  // namespace fa
