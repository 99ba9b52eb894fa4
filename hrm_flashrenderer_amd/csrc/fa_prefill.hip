// Causal / non-causal flash-attention prefill for gfx950 (contiguous or paged
// K/V, MHA or GQA), and an fp32 variant of the contiguous op.
//
// Semantics: the reference's flash_attn / flash_attn_paged
// (flashattention_custom/ops.py:19-60, csrc/flash_attn_sm75.cu:89-425):
//   O[b,h,i] = sum_j softmax_j(Q[b,h,i] . K[b,hk,j] / sqrt(D)) V[b,hk,j]
// over keys j < N_b with k_off + j <= q_off + i when causal.
//
// fp16 kernels (MFMA-bound), common to both:
//  * A workgroup owns 128 query rows of one (b, hq): 4 waves x 32 rows. Q stays
//    in registers as the B operand of S^T = K Q^T (v_mfma_f32_32x32x16_f16).
//  * Both products keep the query row as the MFMA column: every lane owns one
//    query row, the softmax max/sum is an in-lane reduction plus one exchange
//    with lane ^ 32, and the rescale of O^T by exp(m_old - m_new) is a single
//    per-lane factor. P never leaves registers: the S^T accumulator registers
//    are already in the B-operand layout of the P^T side (with the key order
//    inside a 16-key step permuted identically on the V^T side).
//  * Causal tiles beyond the diagonal are never loaded; waves whose rows see
//    none of a tile skip its math; the q-tile order is reversed so the longest
//    rows start first.
// Kernels: prefill_b32_kernel streams K/V tiles into LDS by DMA (pages of a
// multiple of 16 tokens, or contiguous K/V; see the section below);
// prefill_f16_kernel stages tiles through registers and looks up every key
// row on its own (any page size); prefill_f32_kernel is the exact-fp32
// contiguous op.
//
// prefill_f16_kernel: the next 64-key tile's rows are fetched from HBM into
// registers while the current tile is computed. K is stored row-major
// (padded rows); V is stored transposed (Vt[d][key], padded) by a byte
// permute in registers, so that the A operand of O^T = V^T P^T is two 8-byte
// LDS reads per MFMA.
#include "fa_common.h"


#include <type_traits>

namespace fa {

namespace {

constexpr int kBM = 128;     // query rows per workgroup
constexpr int kMaxPackHeads = 256;  // q heads listed per KV head in the packed layout
constexpr int kBN = 64;      // keys per tile
constexpr int kThreads = 256;

__device__ __forceinline__ uint32_t pack_lo(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t x, uint32_t y) {
  return __builtin_amdgcn_perm(y, x, 0x07060302u);
}

// Key limit of one query row: keys j < limit are visible.
__device__ __forceinline__ int row_key_limit(int kv_len, int causal, int qo, int ko, int row) {
  int lim = kv_len;
  if (causal) {
    const int64_t c = (int64_t)qo + row - ko + 1;
    if (c < lim) lim = c < 0 ? 0 : (int)c;
  }
  return lim;
}

template <int D>
struct TileRegs {
  static constexpr int KCH = kBN * D / 8 / kThreads;   // 16-byte K chunks per thread
  static constexpr int KPT = kBN * D / 8 / kThreads;   // keys per thread for V (x 8 d)
  u32x4 k[KCH];
  u32x4 v[KPT];
};

__device__ __forceinline__ int64_t pick4(const int64_t (&v)[4], int g) {
  return g == 0 ? v[0] : g == 1 ? v[1] : g == 2 ? v[2] : v[3];
}

// Fetches the K/V rows of the 64-key tile starting at k0 into registers.
// Rows at or beyond kv_len (or not addressable) read as zero.
//
// ALIGNED (contiguous K/V, or pages of a multiple of 16 tokens): the 16 keys
// of each quarter of the tile share one page, so the page lookup is one
// uniform (scalar) block-table read per quarter and rows are plain offsets
// from it. Scalar reads complete on their own counter, so the vector loads of
// the tile are issued back to back and stay in flight while the current tile
// is computed. Otherwise every row is looked up on its own.
template <int D, bool ALIGNED>
__device__ __forceinline__ void load_tile(TileRegs<D>& r, const AttnParams& p, const f16* kp,
                                          const f16* vp, int b, int hk, int k0, int kv_len,
                                          int tid) {
  constexpr int CPR = D / 8;  // 16-byte chunks per row
  constexpr int KCH = TileRegs<D>::KCH;
  constexpr int KPT = TileRegs<D>::KPT;
  constexpr int RPP = kThreads / CPR;  // rows per pass of the K loader
  int64_t goff[4];
  if constexpr (ALIGNED) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int key = k0 + 16 * g;
      goff[g] = key < kv_len ? p.kv.row_offset(b, hk, key) : -1;
    }
  }
  auto row_off = [&](int row) -> int64_t {
    const int j = k0 + row;
    if (j >= kv_len) return -1;
    if constexpr (ALIGNED) {
      const int64_t base = pick4(goff, row >> 4);
      return base < 0 ? -1 : base + (int64_t)(row & 15) * D;
    } else {
      return p.kv.row_offset(b, hk, j);
    }
  };
  const int col = tid % CPR;
#pragma unroll
  for (int i = 0; i < KCH; ++i) {
    const int64_t off = row_off(tid / CPR + RPP * i);
    r.k[i] = off >= 0 ? *reinterpret_cast<const u32x4*>(kp + off + 8 * col)
                      : u32x4{0u, 0u, 0u, 0u};
  }
  const int kg = tid / CPR;  // key group: keys KPT*kg .. +KPT
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int64_t off = row_off(KPT * kg + i);
    r.v[i] = off >= 0 ? *reinterpret_cast<const u32x4*>(vp + off + 8 * col)
                      : u32x4{0u, 0u, 0u, 0u};
  }
}

template <int D>
__device__ __forceinline__ void store_tile(const TileRegs<D>& r, f16* sK, f16* sVt, int tid) {
  constexpr int CPR = D / 8;
  constexpr int KPAD = D + 8;
  constexpr int VPAD = kBN + 8;
  constexpr int KCH = TileRegs<D>::KCH;
  constexpr int KPT = TileRegs<D>::KPT;
#pragma unroll
  for (int i = 0; i < KCH; ++i) {
    const int c = tid + kThreads * i;
    const int row = c / CPR;
    const int col = c % CPR;
    *reinterpret_cast<u32x4*>(sK + row * KPAD + 8 * col) = r.k[i];
  }
  const int kg = tid / CPR;
  const int dc = tid % CPR;
  // Transpose KPT keys x 8 d into 8 rows of Vt holding KPT consecutive keys.
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    if constexpr (KPT == 4) {
      const u32x2 lo = u32x2{pack_lo(r.v[0][w], r.v[1][w]), pack_lo(r.v[2][w], r.v[3][w])};
      const u32x2 hi = u32x2{pack_hi(r.v[0][w], r.v[1][w]), pack_hi(r.v[2][w], r.v[3][w])};
      *reinterpret_cast<u32x2*>(sVt + (8 * dc + 2 * w) * VPAD + KPT * kg) = lo;
      *reinterpret_cast<u32x2*>(sVt + (8 * dc + 2 * w + 1) * VPAD + KPT * kg) = hi;
    } else {
      *reinterpret_cast<uint32_t*>(sVt + (8 * dc + 2 * w) * VPAD + KPT * kg) =
          pack_lo(r.v[0][w], r.v[1][w]);
      *reinterpret_cast<uint32_t*>(sVt + (8 * dc + 2 * w + 1) * VPAD + KPT * kg) =
          pack_hi(r.v[0][w], r.v[1][w]);
    }
  }
}

template <int D, bool ALIGNED>
__global__ __launch_bounds__(kThreads) void prefill_f16_kernel(AttnParams p) {
  constexpr int KSTEPS = D / 16;  // k-steps of S^T
  constexpr int DBLK = D / 32;    // 32-row blocks of O^T
  constexpr int KPAD = D + 8;
  constexpr int VPAD = kBN + 8;
  __shared__ __attribute__((aligned(16))) f16 sK[kBN * KPAD];
  __shared__ __attribute__((aligned(16))) f16 sVt[D * VPAD];

  const int qt = gridDim.x - 1 - blockIdx.x;
  const int hq = blockIdx.y;
  const int b = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31;   // query row within the wave
  const int half_id = lane >> 5;

  const int q0 = qt * kBM;
  const int qrow = q0 + wave * 32 + col;
  f16* op = reinterpret_cast<f16*>(p.o) + ((int64_t)b * p.Hq + hq) * p.M * D;

  const int hk = p.kv_head(hq);
  if (hk < 0) {
    if (qrow < p.M) {
      const f16 fill = qrow < p.q_len(b) ? (f16)__builtin_nanf("") : (f16)0.f;
      for (int d = half_id * (D / 2); d < (half_id + 1) * (D / 2); ++d)
        op[(int64_t)qrow * D + d] = fill;
    }
    return;
  }

  const int kv_len = p.kv_len(b);
  const int qo = p.q_off(b);
  const int ko = p.k_off(b);
  const int qlen = p.q_len(b);  // rows at or past qlen are padding: zeros, no tiles
  const int last_row = min(q0 + kBM, qlen) - 1;
  const int wg_lim = q0 < qlen ? row_key_limit(kv_len, p.causal, qo, ko, last_row) : 0;
  const int ntiles = (wg_lim + kBN - 1) / kBN;

  const int wrow0 = q0 + wave * 32;
  const int wrow1 = min(wrow0 + 31, qlen - 1);
  const bool wave_rows = wrow0 < qlen;
  const int wave_lim_max = wave_rows ? row_key_limit(kv_len, p.causal, qo, ko, wrow1) : 0;
  const int wave_lim_min = wave_rows ? row_key_limit(kv_len, p.causal, qo, ko, wrow0) : 0;
  const int lim = row_key_limit(kv_len, p.causal, qo, ko, qrow);

  const f16* qp = reinterpret_cast<const f16*>(p.q) + ((int64_t)b * p.Hq + hq) * p.M * D;
  const f16* kp = reinterpret_cast<const f16*>(p.k);
  const f16* vp = reinterpret_cast<const f16*>(p.v);

  half8 qreg[KSTEPS];
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) {
    qreg[ks] = qrow < p.M
                   ? *reinterpret_cast<const half8*>(qp + (int64_t)qrow * D + 16 * ks + 8 * half_id)
                   : half8{0, 0, 0, 0, 0, 0, 0, 0};
  }
  if (p.rope_cos != nullptr && qrow < p.M) rope_fragment<KSTEPS, 16>(qreg, p, qo + qrow, 8 * half_id);

  floatx16 acc_o[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) acc_o[i] = floatx16{};
  float m_run = -INFINITY;
  float l_run = 0.f;
  const float c = p.scale_log2;

  TileRegs<D> regs;
  if (ntiles > 0) load_tile<D, ALIGNED>(regs, p, kp, vp, b, hk, 0, kv_len, tid);

  for (int t = 0; t < ntiles; ++t) {
    const int k0 = t * kBN;
    __syncthreads();
    store_tile<D>(regs, sK, sVt, tid);
    __syncthreads();
    if (t + 1 < ntiles) load_tile<D, ALIGNED>(regs, p, kp, vp, b, hk, k0 + kBN, kv_len, tid);
    if (k0 >= wave_lim_max) continue;

    // S^T[key][row]: two 32-key blocks.
    floatx16 s0 = floatx16{}, s1 = floatx16{};
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const half8 a0 = *reinterpret_cast<const half8*>(sK + col * KPAD + 16 * ks + 8 * half_id);
      const half8 a1 =
          *reinterpret_cast<const half8*>(sK + (32 + col) * KPAD + 16 * ks + 8 * half_id);
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, qreg[ks], s0, 0, 0, 0);
      s1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, qreg[ks], s1, 0, 0, 0);
    }
    // Register r of block mb holds key k0 + 32*mb + 8*(r/4) + 4*half_id + r%4.
    if (k0 + kBN > wave_lim_min) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 8 * (r >> 2) + 4 * half_id + (r & 3);
        if (key >= lim) s0[r] = -INFINITY;
        if (key + 32 >= lim) s1[r] = -INFINITY;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(s0[r], s1[r]));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_use) * c);
    const float mc = m_use * c;
    float psum = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s0[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[r], c, -mc));
      s1[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[r], c, -mc));
      psum += s0[r] + s1[r];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int i = 0; i < DBLK; ++i) acc_o[i] = acc_o[i] * alpha;

    // P^T operands of the four 16-key steps.
    half8 pb[4];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pb[0][j] = (f16)s0[j];
      pb[1][j] = (f16)s0[8 + j];
      pb[2][j] = (f16)s1[j];
      pb[3][j] = (f16)s1[8 + j];
    }
    // O^T[d][row] += V^T[d][key] P^T[key][row]; within step s the lane's k
    // slot j maps to key 16*s + 8*(j/4) + 4*half_id + j%4.
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int i = 0; i < DBLK; ++i) {
        const f16* vrow = sVt + (32 * i + col) * VPAD + 16 * s + 4 * half_id;
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 8);
        const half8 a = __builtin_bit_cast(half8, u32x4{lo[0], lo[1], hi[0], hi[1]});
        acc_o[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[s], acc_o[i], 0, 0, 0);
      }
    }
  }

  if (qrow >= p.M) return;
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  // kv_len == 0: zeros (empty softmax times empty V); otherwise a row without
  // visible keys gives 0 * inf = NaN, as the reference does. Padding rows
  // (qrow >= qlen) are zeros whatever their Q held.
  const bool live = qrow < qlen;
  const float inv = kv_len == 0 ? 0.f : 1.f / l_tot;
  f16* orow = op + (int64_t)qrow * D;
#pragma unroll
  for (int i = 0; i < DBLK; ++i) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      half4 h = half4{(f16)(acc_o[i][4 * g + 0] * inv), (f16)(acc_o[i][4 * g + 1] * inv),
                      (f16)(acc_o[i][4 * g + 2] * inv), (f16)(acc_o[i][4 * g + 3] * inv)};
      if (!live) h = half4{0, 0, 0, 0};
      *reinterpret_cast<half4*>(orow + 32 * i + 8 * g + 4 * half_id) = h;
    }
  }
}

// ---------------------------------------------------------------------------
// Tile-DMA prefill kernel (pages of a multiple of 16 tokens, or contiguous
// K/V): prefill_b32_kernel (32-key tiles). Design:
//
//  * K and V tiles go from HBM straight into LDS with buffer_load ... lds
//    (16 bytes per lane), no staging registers. Each wave moves one slab of
//    the tile (16 or 8 keys), which lies in one page, through one buffer
//    resource whose size covers only the slab's valid rows: rows past seqlen
//    land in LDS as zeros.
//  * LDS holds two K and two V tiles (double buffer, one barrier per tile;
//    three of each for the packed rows, see the kernel).
//    Rows are 2*D bytes; 16-byte chunks are XOR-swizzled per row so that the
//    reads below are free of bank conflicts: K chunk c of row r is stored at
//    c ^ (r % CH) (32 rows read at one column by ds_read_b128), V chunk c at
//    c ^ (4r % CH) (4 rows x 32 bytes per 16 lanes for the transposing read).
//  * S^T = K Q^T (A = K from LDS, B = Q in registers) and O^T = V^T P^T with
//    v_mfma_f32_32x32x16_f16. The V^T operand comes from ds_read_b64_tr_b16:
//    in each 16-lane group, lane s points at V[k0 + s/4][d0 + 4(s%4)] and
//    lane i receives V[k0 + j][d0 + i], j = 0..3 (4 keys of one d).
//  * Online softmax keeps a per-row reference max and rescales O only when a
//    tile's max exceeds it by more than 2^8 (then P <= 256 fits fp16 exactly as
//    well as P <= 1 does; the final division uses the same reference).
//  * Work order is XCD-aware: consecutive dispatch slots go round-robin over
//    the 8 XCDs, so slot L runs item (L % 8) * per_xcd + L / 8 of a list
//    ordered by (sequence, KV-head group, q tile descending, head in group):
//    all q tiles and heads that share one KV head run on one XCD's L2, longest
//    rows first. When the (sequence, KV group) pairs divide evenly over the
//    XCDs, XCD x owns pairs x, x + 8, ... (each XCD gets a share of every
//    sequence length) and runs them longest sequence first: four at a time
//    with their items interleaved when four pairs' K/V fit the L2, otherwise
//    one after another with only the last two interleaved (see the kernel).
// ---------------------------------------------------------------------------

constexpr uint32_t kRsrcWord3 = 0x00020000u;  // raw buffer, dword data format (gfx9)
constexpr float kRescaleLog2 = 8.f;

// v_max3_f32 without the canonicalising moves fmaxf adds for inputs the
// compiler cannot prove canonical (MFMA results): the hardware max already
// treats a quiet NaN input as missing, and no input here is a signalling NaN.
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// Max of 16 values as a depth-3 tree of max3 (six independent max3, then two,
// then one), instead of a dependent chain of eight.
__device__ __forceinline__ float max16(const floatx16& s) {
  const float a0 = vmax3(s[0], s[1], s[2]), a1 = vmax3(s[3], s[4], s[5]);
  const float a2 = vmax3(s[6], s[7], s[8]), a3 = vmax3(s[9], s[10], s[11]);
  const float a4 = vmax3(s[12], s[13], s[14]);
  const float b0 = vmax3(a0, a1, a2), b1 = vmax3(a3, a4, s[15]);
  return vmax3(b0, b1, b1);
}

// Per-sequence data of the prefill kernels, loaded without a branch on the
// optional arrays (a branch would make the compiler wait for each load before
// the next one): a missing array reads a valid stand-in address (the first
// word of Q) and its default replaces the value. Uniform (b, hq) give scalar
// loads; per-lane ones give vector loads that all leave before one wait.

// Work list of the 128-row prefill grid, decided on the host from the shapes:
// item = (pair, q tile, head) where a pair is one (sequence, KV-head group) of
// `group` q heads with `ntq` q tiles each (PACKED: one (sequence, KV head) of
// ntq packed tiles, group 1). order 0: slot L runs item
// (L % 8) * per_xcd + L / 8 of the list ordered by (pair, q tile descending,
// head). order 1 and 2 (the pairs divide evenly over the XCDs): XCD x owns
// pairs x, x + 8, ..., kp of them; order 1 runs them four at a time with the
// items interleaved, order 2 one after another with only the last tp
// interleaved. rank: order the XCD's pairs by key count first.
struct PrefillGrid {
  int ntq, group, per_xcd, total;
  int order, kp, tp, head_items, rank;
  int per_pair, ngroups, band, gsz;
  FastDiv d_pair, d_group, d_ngroups, d_band, d_gsz;
};

struct SeqData {
  int kv_len, hk, qo, ko, qlen;
};

__device__ __forceinline__ int ld_or(const int32_t* ptr, int idx, int dflt, const void* any) {
  typedef const __attribute__((address_space(4))) int32_t cint;
  const int32_t* a = ptr != nullptr ? ptr + idx : reinterpret_cast<const int32_t*>(any);
  const int v = *(cint*)a;
  return ptr != nullptr ? v : dflt;
}

// dflt_hk: q head hq's KV head when there is no head map (the contiguous
// operator: hq / (Hq / Hk), which the caller knows from its work item).
__device__ __forceinline__ SeqData seq_data(const AttnParams& p, int b, int hq, int dflt_hk) {
  SeqData d;
  const int n = ld_or(p.seqlen, b, p.N, p.q) + (p.seqlen != nullptr ? p.app_advance : 0);
  d.kv_len = n < 0 ? 0 : n > p.N ? p.N : n;
  const int hk = ld_or(p.head_map, hq, dflt_hk, p.q);
  d.hk = (hk >= 0 && hk < p.Hk) ? hk : -1;
  d.qo = ld_or(p.q_offsets, b, p.q_offset, p.q);
  d.ko = ld_or(p.k_offsets, b, p.k_offset, p.q);
  const int ql = ld_or(p.q_lens, b, p.M, p.q);
  d.qlen = ql < 0 ? 0 : ql > p.M ? p.M : ql;
  return d;
}

// Index i of pair x + 8i among the kp pairs of XCD x, at position j when those
// pairs are ordered by key count, longest first, ties by index. Lane i holds
// n = key count of pair x + 8i (-1 for lanes >= kp) and ranks it against all
// kp (kp <= 64); the result is wave-uniform.
__device__ __forceinline__ int pair_by_length(int n, int kp, int j) {
  const int lane = threadIdx.x & 63;
  int rank = 0;
  for (int i = 0; i < kp; ++i) {
    const int m = __builtin_amdgcn_readlane(n, i);
    rank += (m > n || (m == n && i < lane)) ? 1 : 0;
  }
  const uint64_t hit = __ballot(lane < kp && rank == j);
  return __builtin_amdgcn_readfirstlane(__builtin_ctzll(hit));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           (int)kRsrcWord3);
}

// One 16-byte-per-lane LDS DMA: M0 holds the wave's LDS destination, the
// lanes' rows land one after another from there. Issued as inline asm so the
// compiler does not track it: it puts an `s_waitcnt vmcnt(0)` in front of
// every ds_read_b64_tr_b16 that follows a DMA it knows of, which would make
// each wave wait for its next tile's DMA before reading V of the current one.
// Ordering is explicit instead: every DMA is waited for (vmcnt) before the
// barrier that precedes the reads of its stage. The `s_nop 0` is the wait
// state an LDS DMA needs after an SALU write of M0. NT sets the non-temporal
// cache policy, for K/V that no other workgroup reads.
template <bool NT>
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voffset) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)lds;
  if constexpr (NT)
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen nt lds"
                 :: "v"(voffset), "s"(r), "{m0}"(m0) : "memory");
  else
    asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                 :: "v"(voffset), "s"(r), "{m0}"(m0) : "memory");
}

template <int D>
struct DmaCfg {
  static constexpr int ROWB = 2 * D;             // bytes per key row
  static constexpr int CH = D / 8;               // 16-byte chunks per row
  static constexpr int RPI = 1024 / ROWB;        // rows per wave-wide 16-byte load
  __device__ static int swz_k(int row) { return row % CH; }
  __device__ static int swz_v(int row) { return (4 * row) % CH; }
};

// Page part of one tile DMA: this wave's slab of keys lies in one page; `off`
// is its element offset (0 when nothing is valid) and `nbytes` the bytes of
// its valid rows (the buffer range: rows beyond read as zero).
struct QuarterSrc {
  int64_t off;
  uint32_t nbytes;
};

// V^T operand (8 keys of one d per lane) of PV step s, d block i, via two
// transposing reads; voff holds the lane's byte offset from `buf`.
template <int D>
__device__ __forceinline__ half8 ld_vt(const char* buf, const int* voff, int s, int i) {
  using C = DmaCfg<D>;
  const char* va = buf + voff[i] + 16 * s * C::ROWB;
  const half4 lo = __builtin_bit_cast(
      half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4v*)(va)));
  const half4 hi = __builtin_bit_cast(
      half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                 (__attribute__((address_space(3))) short4v*)(va + 8 * C::ROWB)));
  return half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// With NW waves per workgroup and BN-key tiles, wave w moves the slab of
// SLAB = BN / NW keys starting at k0 + SLAB * w (one page: pages hold a
// multiple of 16 tokens).
template <int D, int NW, int BN>
struct Slab {
  static constexpr int SLAB = BN / NW;                  // keys per wave and tile
  static constexpr int IPW = SLAB / DmaCfg<D>::RPI;     // 16-byte DMA loads per wave
  static_assert(IPW >= 1, "slab smaller than one wave-wide load");
};

// Per-wave page table in VGPR lanes: lane i holds the key-row index (element
// offset / D) of this wave's slab of tile base + i, or ~0u when the slab has
// no addressable row. One vector pass (block-table loads included) covers 64
// tiles; a tile's lookup is then one v_readlane, so the tile loop issues no
// scalar loads (whose lgkmcnt wait would also drain the LDS reads in flight).
// Row indices fit 32 bits: 2^32 rows of >= 128 bytes exceed the device memory.
template <int D, int NW, int BN>
struct SlabTable {
  static constexpr int SPAN = 64;
  uint32_t rows;     // pool row of the slab of tile base + lane, KV head 0 (~0u: none)
  int base;
  uint32_t hk_rows;  // rows between KV heads: hk * stride_hk / D

  // Page row of the slab of tile T for KV head 0, whether or not it holds
  // keys below kv_len (get() masks by kv_len): the table load needs only b,
  // so it leaves with the Q loads, before kv_len and the head map are known.
  // row_offset bounds the page by the block table width.
  // The same map as KVMap::row_offset (KV head 0), split into the table load
  // (row_load) and the arithmetic on its result (row_finish), with the
  // per-lane checks as selects around an always in-bounds load: no divergent
  // branch makes the compiler wait for the load where it is issued, and the
  // first fill can issue it, then other loads, then finish.
  struct RowReq {
    unsigned raw;   // physical page id (block table), logical page, or token
    unsigned slot;  // token within the page
    bool ok;
  };
  __device__ static RowReq row_load(const AttnParams& p, int b, int T, int wave) {
    const KVMap& kv = p.kv;
    const int g0 = T * BN + (BN / NW) * wave;
    RowReq r;
    r.ok = g0 >= 0 && g0 < p.N;
    const unsigned g = r.ok ? (unsigned)g0 : 0u;
    if (!kv.paged) {
      r.raw = g;
      r.slot = 0;
      return r;
    }
    unsigned page;
    if (kv.ps_shift >= 0) {
      page = g >> kv.ps_shift;
      r.slot = g & (unsigned)(kv.PS - 1);
    } else {
      page = g / (unsigned)kv.PS;
      r.slot = g - page * (unsigned)kv.PS;
    }
    r.ok = r.ok && page < (unsigned)kv.max_blocks;
    const unsigned pg = r.ok ? page : 0u;
    if (kv.block_table != nullptr) {
      typedef const __attribute__((address_space(4))) int32_t ctable;
      r.raw = (unsigned)((ctable*)kv.block_table)[(int64_t)b * kv.max_blocks + pg];
    } else {
      r.raw = pg;
    }
    return r;
  }
  __device__ static uint32_t row_finish(const AttnParams& p, int b, const RowReq& r) {
    const KVMap& kv = p.kv;
    if (!kv.paged)
      return r.ok ? (uint32_t)(((int64_t)b * kv.stride_nb + (int64_t)r.raw * kv.stride_tok) / D) : ~0u;
    bool ok = r.ok;
    unsigned nb, pp;
    if (kv.block_table != nullptr) {
      ok = ok && r.raw < (unsigned)kv.num_phys;
      nb = kv.num_phys <= kv.P ? 0u : r.raw / (unsigned)kv.P;
      pp = r.raw - nb * (unsigned)kv.P;
    } else {
      nb = (unsigned)b;
      pp = r.raw;
    }
    const int64_t off = (int64_t)nb * kv.stride_nb + (int64_t)pp * kv.stride_page + (int64_t)r.slot * D;
    return ok ? (uint32_t)(off / D) : ~0u;
  }
  __device__ void fill(const AttnParams& p, int b, int wave, int lane, int first) {
    // opaque to the compiler, so it keeps no per-tile induction variables for
    // the (rare) refill
    asm volatile("" : "+s"(first));
    base = first;
    rows = row_finish(p, b, row_load(p, b, first + lane, wave));
    // s_waitcnt vmcnt(0) (expcnt, lgkmcnt unconstrained) as an instruction
    // the compiler's wait insertion sees: the block-table load is then known
    // complete on every path out of the refill, so a later reuse of its
    // register in the tile loop needs no wait there.
    __builtin_amdgcn_s_waitcnt(0x0F70);
  }
  // Source of tile T (uniform, non-decreasing over the calls) for this wave.
  __device__ QuarterSrc get(const AttnParams& p, int b, int T, int kv_len, int wave, int lane) {
    if (T - base >= SPAN) fill(p, b, wave, lane, T);
    const uint32_t r = (uint32_t)__builtin_amdgcn_readlane((int)rows, T - base);
    const int valid = min(BN / NW, kv_len - (T * BN + (BN / NW) * wave));
    const bool ok = r != ~0u && valid > 0;
    return QuarterSrc{ok ? (int64_t)(r + hk_rows) * D : 0,
                      ok ? (uint32_t)(valid * DmaCfg<D>::ROWB) : 0u};
  }
};

template <int D, int NW, int BN>
struct SlabLane {
  uint32_t vk[Slab<D, NW, BN>::IPW];
  uint32_t vv[Slab<D, NW, BN>::IPW];
};

template <int D, int NW, int BN>
__device__ __forceinline__ SlabLane<D, NW, BN> slab_lane(int wave, int lane) {
  using C = DmaCfg<D>;
  SlabLane<D, NW, BN> d;
  const int pch = lane % C::CH;
#pragma unroll
  for (int i = 0; i < Slab<D, NW, BN>::IPW; ++i) {
    const int rq = C::RPI * i + lane / C::CH;            // row within the slab
    const int rt = Slab<D, NW, BN>::SLAB * wave + rq;    // row within the tile
    d.vk[i] = (uint32_t)(rq * C::ROWB + 16 * (pch ^ C::swz_k(rt)));
    d.vv[i] = (uint32_t)(rq * C::ROWB + 16 * (pch ^ C::swz_v(rt)));
  }
  return d;
}

template <int D, int NW, int BN, bool NT>
__device__ __forceinline__ void dma_slab(const QuarterSrc& q, const uint32_t* voffs,
                                         const char* base, int wave, char* dst_tile) {
  using C = DmaCfg<D>;
  const __amdgpu_buffer_rsrc_t r = make_rsrc(base + q.off * 2, q.nbytes);
#pragma unroll
  for (int i = 0; i < Slab<D, NW, BN>::IPW; ++i)
    lds_dma16<NT>(r, dst_tile + (Slab<D, NW, BN>::SLAB * wave + C::RPI * i) * C::ROWB, voffs[i]);
}

// ---------------------------------------------------------------------------
// Prefill on 32-key tiles: 16 KB of K and V per stage, two stages per
// workgroup (32 KB; three, 48 KB, for packed rows), at most 168 VGPRs, so
// three workgroups (three waves per SIMD) share a CU, whose waves hide each
// other's latency.
// ---------------------------------------------------------------------------
//
// PACKED: the 128 rows of a workgroup are (head, position) rows of one KV
// head instead of 128 positions of one q head. Row r of the (sequence, KV
// head) pair's packed list is position r % M of the (r / M)-th q head that
// reads the KV head (head-map order), so a pair's K/V streams once for all
// its q heads when M < 128 (e.g. 16 positions x 8 heads in one tile, where
// the per-head layout would fill 16 of 128 rows and stream the K/V once per
// q head). `ntq` is then the number of 128-row tiles per pair, `group` 1,
// and slot L runs pair L / ntq (consecutive pairs go to different XCDs).
template <int D, bool PACKED>
__global__ __launch_bounds__(kThreads, 3) void prefill_b32_kernel(AttnParams p, PrefillGrid g) {
  using C = DmaCfg<D>;
  constexpr int BN = 32;
  constexpr int NW = 4;
  constexpr int TILE = BN * C::ROWB;
  constexpr int KSTEPS = D / 16;
  constexpr int DBLK = D / 32;
  // PACKED tiles stream K/V that no other workgroup reads (one workgroup per
  // KV head and tile of its rows) from HBM, where the per-head layout's K/V
  // is shared through L2 by the q tiles and heads of one KV head. They load it
  // non-temporally (M = 16 over cfg4's pool: +6 %, M = 8: +10 %) through three
  // stages, each tile's DMA issued two tiles ahead (48 KB of LDS at D = 128,
  // still three workgroups per CU; +1-2 %). The per-head layout keeps two
  // stages: a third gained nothing there.
  constexpr int NST = PACKED ? 3 : 2;
  constexpr int kDmaPerTile = 2 * Slab<D, NW, BN>::IPW;  // DMA instructions per wave and tile
  __shared__ __attribute__((aligned(1024))) char smem[2 * NST * TILE];  // K0 V0 K1 V1 (K2 V2)
  // PACKED: the q heads of the pair's KV head in head-map order, and the
  // heads whose head-map entry is outside [0, Hk) (collected by the pairs of
  // KV head 0); s_pk_n holds both counts.
  constexpr int kPackList = PACKED ? kMaxPackHeads : 1;
  __shared__ int s_pk[kPackList];
  __shared__ int s_bad[kPackList];
  __shared__ int s_pk_n[2];

  const int slot = blockIdx.x;
  const int item = PACKED ? slot : (slot & 7) * g.per_xcd + (slot >> 3);
  if (item >= g.total) return;
  const int group = g.group;
  const int ngroups = g.ngroups;
  int pair, qt, head;
  // With `pre`, the sequence data of the chosen pair come from the loads that
  // ordered the pairs (kv_len_pre, hk_pre, qo_pre, ko_pre).
  bool pre = false;
  int kv_len_pre = 0, hk_pre = 0, qo_pre = 0, ko_pre = 0, qlen_pre = 0;
  if (PACKED || g.order == 0) {
    pair = fdiv(item, g.d_pair);
    const int rem = item - pair * g.per_pair;
    const int r = fdiv(rem, g.d_group);
    qt = g.ntq - 1 - r;
    head = rem - r * group;
  } else {
    // Each XCD owns whole (sequence, KV group) pairs: XCD x takes pairs x,
    // x + 8, x + 16, ..., so sequences of different lengths spread over all
    // XCDs.
    // When the K/V of four pairs (at the per-sequence capacity) fit one XCD's
    // 4 MB L2 (cfg2: 1 MB per pair), four pairs at a time run longest q tile
    // first across all four (order 1): the XCD's slots finish together and
    // the four pairs share the L2 (+1.5 % on cfg2 over two at a time). Longer
    // pairs (cfg5: up to 17 MB each) run one after another, longest q tile
    // first within each (order 2), so a pair's items start together and
    // stream its K/V through the L2 once; only the XCD's last two pairs
    // interleave, to keep the tail short. On cfg5 that fetches 1.03x the
    // algorithmic bytes against 2.0x with every two pairs interleaved, at
    // 0.4-0.6 % of time (same-process A/B on two boxes); interleaving the
    // last four fetched 1.22x and lost 1.6 %, and no interleave at all lost
    // 1.0 %.
    const int x = slot & 7, l = slot >> 3;
    int r, w, j;
    if (g.order == 1) {
      const int gi = fdiv(l, g.d_gsz), lg = l - gi * g.gsz;
      r = fdiv(lg, g.d_band);
      w = lg - r * g.band;
      j = gi * 4 + fdiv(w, g.d_group);
    } else if (l < g.head_items) {
      j = fdiv(l, g.d_pair);
      const int lg = l - j * g.per_pair;
      r = fdiv(lg, g.d_group);
      w = lg - r * group;
    } else {
      const int l2 = l - g.head_items;
      r = fdiv(l2, g.d_band);
      w = l2 - r * g.band;
      j = g.kp - g.tp + fdiv(w, g.d_group);
    }
    head = w - fdiv(w, g.d_group) * group;
    if (g.rank) {
      // Chunked prefill over cached context: a pair's work grows with its
      // sequence's key count, so the XCD runs its pairs longest first. One
      // round of per-lane loads gives every candidate's key count, head map
      // entry and offsets; the chosen pair's are then read from its lane. (A
      // plain prefill batch keeps the natural order and saves this round.)
      const int lane = threadIdx.x & 63;
      const int cpair = x + 8 * min(lane, g.kp - 1);
      const int cb = fdiv(cpair, g.d_ngroups), chk = cpair - cb * ngroups;
      const SeqData c = seq_data(p, cb, chk * group + head, chk);
      j = pair_by_length(lane < g.kp ? c.kv_len : -1, g.kp, j);
      kv_len_pre = __builtin_amdgcn_readlane(c.kv_len, j);
      hk_pre = __builtin_amdgcn_readlane(c.hk, j);
      qo_pre = __builtin_amdgcn_readlane(c.qo, j);
      ko_pre = __builtin_amdgcn_readlane(c.ko, j);
      qlen_pre = __builtin_amdgcn_readlane(c.qlen, j);
      pre = true;
    }
    pair = x + 8 * j;
    qt = g.ntq - 1 - r;
  }
  const int b = fdiv(pair, g.d_ngroups);
  const int hk_pair = pair - b * ngroups;  // PACKED: the pair's KV head
  const int hq = PACKED ? 0 : hk_pair * group + head;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31;
  const int half_id = lane >> 5;
  const int q0 = qt * kBM;
  // PACKED: wave 0 lists the q heads of KV head hk_pair in head-map order (64
  // heads per ballot); the pairs of KV head 0 also list the heads whose entry
  // is outside [0, Hk).
  int pk_count = 0, pk_rows = 0;
  if constexpr (PACKED) {
    if (wave == 0) {
      int count = 0, nbad = 0;
      for (int base = 0; base < p.Hq; base += 64) {
        const int h = base + lane;
        const int hm = h < p.Hq ? p.kv_head(h) : -2;
        const bool match = hm == hk_pair;
        const bool bad = hk_pair == 0 && hm == -1;
        const uint64_t below = (1ull << lane) - 1ull;
        const uint64_t mm = __ballot(match), mb = __ballot(bad);
        if (match) {
          const int pos = count + __popcll(mm & below);
          if (pos < kMaxPackHeads) s_pk[pos] = h;
        }
        if (bad) {
          const int pos = nbad + __popcll(mb & below);
          if (pos < kMaxPackHeads) s_bad[pos] = h;
        }
        count += __popcll(mm);
        nbad += __popcll(mb);
      }
      if (lane == 0) {
        s_pk_n[0] = min(count, kMaxPackHeads);
        s_pk_n[1] = min(nbad, kMaxPackHeads);
      }
    }
    __syncthreads();
    // Heads past pack_heads (a head map that sends more heads to one KV head
    // than the caller stated) get no packed rows: tile 0 writes them as NaN.
    pk_count = min(s_pk_n[0], p.pack_heads);
    pk_rows = pk_count * p.M;
  }
  // The wave's block of 32 rows. Under a causal mask the block with the last
  // rows computes up to three more tiles than the first; the per-head layout
  // rotates the blocks over the waves from item to item so that this work
  // does not always land on the same SIMD.
  const int rblk = PACKED ? wave : (wave + (slot >> 3)) & (NW - 1);
  // This lane's query row: position qrow of q head hq_row.
  const int prow = q0 + rblk * 32 + col;  // PACKED: row of the pair's packed list
  const int pj = PACKED ? prow / p.M : 0;
  const bool row_exists = PACKED ? prow < pk_rows : true;
  const int qrow = PACKED ? prow - pj * p.M : prow;
  const int hq_row = PACKED ? (row_exists ? s_pk[pj] : 0) : hq;
  f16* op = reinterpret_cast<f16*>(p.o) + ((int64_t)b * p.Hq + hq) * p.M * D;

  // The loads that need only (b, hq) leave first, together with the scalar
  // loads of the key count, head map entry and offsets: Q (rows past M read
  // row M-1 and are zeroed after the load) and the page rows of the first 64
  // tiles. No branch separates them from their uses, so the compiler keeps
  // them here; a head-map entry outside [0, Hk) runs no tiles and writes NaN
  // rows through the common epilogue.
  const f16* qp = reinterpret_cast<const f16*>(p.q) + ((int64_t)b * p.Hq + hq_row) * p.M * D;
  const int64_t qoff = (int64_t)min(qrow, p.M - 1) * D + 8 * half_id;
  const bool q_ok = qrow < p.M && row_exists;
  half8 qreg[KSTEPS];
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) {
    const half8 v = *reinterpret_cast<const half8*>(qp + qoff + 16 * ks);
    qreg[ks] = q_ok ? v : half8{0, 0, 0, 0, 0, 0, 0, 0};
  }
  using Table = SlabTable<D, NW, BN>;
  const typename Table::RowReq req0 = Table::row_load(p, b, lane, wave);
  const SeqData sd = seq_data(p, b, hq, hk_pair);
  const int hk = PACKED ? hk_pair : pre ? hk_pre : sd.hk;
  const int kv_len = pre ? kv_len_pre : sd.kv_len;
  const int qo = pre ? qo_pre : sd.qo;
  const int ko = pre ? ko_pre : sd.ko;
  const int qlen = pre ? qlen_pre : sd.qlen;  // rows at or past qlen: padding (zeros, no tiles)
  const bool head_ok = hk >= 0;
  Table pages;
  pages.base = 0;
  pages.rows = Table::row_finish(p, b, req0);
  pages.hk_rows = head_ok ? (uint32_t)((int64_t)hk * (p.kv.stride_hk / D)) : 0u;

  int wg_lim, wave_lim_max, wave_lim_min;
  if constexpr (PACKED) {
    // First and last position held by packed rows [r0, r1) that are not
    // padding (position < qlen), when there is such a row.
    auto positions = [&](int r0, int r1, int& pmin, int& pmax) {
      r1 = min(r1, pk_rows);
      if (r1 <= r0) return false;
      if (r1 - r0 >= p.M) {
        pmin = 0;
        pmax = p.M - 1;
      } else {
        const int s0 = r0 % p.M, s1 = (r1 - 1) % p.M;
        pmin = s0 <= s1 ? s0 : 0;
        pmax = s0 <= s1 ? s1 : p.M - 1;
      }
      if (pmin >= qlen) return false;
      pmax = min(pmax, qlen - 1);
      return true;
    };
    int pmin = 0, pmax = 0;
    wg_lim = positions(q0, q0 + kBM, pmin, pmax) ? row_key_limit(kv_len, p.causal, qo, ko, pmax) : 0;
    const bool any = positions(q0 + wave * 32, q0 + wave * 32 + 32, pmin, pmax);
    wave_lim_max = any ? row_key_limit(kv_len, p.causal, qo, ko, pmax) : 0;
    wave_lim_min = any ? row_key_limit(kv_len, p.causal, qo, ko, pmin) : 0;
  } else {
    const int last_row = min(q0 + kBM, qlen) - 1;
    wg_lim = head_ok && q0 < qlen ? row_key_limit(kv_len, p.causal, qo, ko, last_row) : 0;
    const int wrow0 = q0 + rblk * 32;
    const int wrow1 = min(wrow0 + 31, qlen - 1);
    const bool wave_rows = wrow0 < qlen;
    wave_lim_max = wave_rows ? row_key_limit(kv_len, p.causal, qo, ko, wrow1) : 0;
    wave_lim_min = wave_rows ? row_key_limit(kv_len, p.causal, qo, ko, wrow0) : 0;
  }
  const int ntiles = (wg_lim + BN - 1) / BN;
  const int lim = row_key_limit(kv_len, p.causal, qo, ko, qrow);

  const char* kp = reinterpret_cast<const char*>(p.k);
  const char* vp = reinterpret_cast<const char*>(p.v);
  const SlabLane<D, NW, BN> dl = slab_lane<D, NW, BN>(wave, lane);
  if (ntiles > 0) {
    const QuarterSrc s0 = pages.get(p, b, 0, kv_len, wave, lane);
    dma_slab<D, NW, BN, PACKED>(s0, dl.vk, kp, wave, smem);
    dma_slab<D, NW, BN, PACKED>(s0, dl.vv, vp, wave, smem + TILE);
  }
  if constexpr (NST == 3) {
    if (ntiles > 1) {
      const QuarterSrc s1 = pages.get(p, b, 1, kv_len, wave, lane);
      dma_slab<D, NW, BN, PACKED>(s1, dl.vk, kp, wave, smem + 2 * TILE);
      dma_slab<D, NW, BN, PACKED>(s1, dl.vv, vp, wave, smem + 3 * TILE);
    }
  }
  QuarterSrc next_src = pages.get(p, b, NST - 1, kv_len, wave, lane);

  if (p.rope_cos != nullptr && q_ok) rope_fragment<KSTEPS, 16>(qreg, p, qo + qrow, 8 * half_id);

  // LDS byte offsets of the lane's operands. K: row col, logical chunk
  // 2*ks + half_id at chunk ^ swz_k(col); the chunk bits of 2*ks and half_id
  // are disjoint, so the k-step ks offset is kbase ^ (32 * ks). V (transposing
  // read, d = 32*i + 16*(gq%2) + 4*(sl%4)): likewise vbase ^ (64 * i). All of
  // them are held in registers for the whole loop rather than recomputed per
  // tile: the XORs are VALU work the MFMAs wait behind (+4 % on cfg2).
  const int gq = lane >> 4, sl = lane & 15;
  const int vrow = 4 * (gq >> 1) + (sl >> 2);
  int kbase = col * C::ROWB + 16 * (half_id ^ C::swz_k(col));
  int vbase;
  {
    const int d = 16 * (gq & 1) + 4 * (sl & 3);
    vbase = TILE + vrow * C::ROWB + 16 * ((d >> 3) ^ C::swz_v(vrow)) + 2 * (d & 7);
  }

  int kofs[KSTEPS], vofs[DBLK];  // operand byte offsets within a K/V stage
#pragma unroll
  for (int ks = 0; ks < KSTEPS; ++ks) kofs[ks] = kbase ^ (32 * ks);
#pragma unroll
  for (int i = 0; i < DBLK; ++i) vofs[i] = vbase ^ (64 * i);
  floatx16 acc_o[DBLK];
#pragma unroll
  for (int i = 0; i < DBLK; ++i) acc_o[i] = floatx16{};
  float m_ref = -INFINITY;
  float neg_m_use = 0.f;  // -(m_ref, or 0 while m_ref is -inf), kept with m_ref
  // (m_ref + 2^8) / c: a raw score above it needs the rescale (c > 0)
  float thr_raw = -INFINITY;
  float l_run = 0.f;
  const float c = p.scale_log2;
  const half2v ones = half2v{(f16)1.f, (f16)1.f};

  auto step = [&](auto par, int t) {
    constexpr int PB = decltype(par)::value;
    const int k0 = t * BN;
    // this wave's DMA of tile t has landed (with three stages, tile t + 1's
    // may still be in flight: vector loads complete in order); the barrier
    // then makes every wave's part visible and frees the stage of tile t - 1
    if constexpr (NST == 3) {
      if (t + 1 < ntiles)
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaPerTile) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();
    if (t + (NST - 1) < ntiles) {
      constexpr int NEXT = (PB + NST - 1) % NST;  // the stage tile t + NST - 1 goes to
      char* nbuf = smem + NEXT * 2 * TILE;
      dma_slab<D, NW, BN, PACKED>(next_src, dl.vk, kp, wave, nbuf);
      dma_slab<D, NW, BN, PACKED>(next_src, dl.vv, vp, wave, nbuf + TILE);
      if (t + NST < ntiles) next_src = pages.get(p, b, t + NST, kv_len, wave, lane);
    }
    if (k0 >= wave_lim_max) return;
    const char* buf = smem + PB * 2 * TILE;
    int koff[KSTEPS], voff[DBLK];
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) koff[ks] = kofs[ks];
#pragma unroll
    for (int i = 0; i < DBLK; ++i) voff[i] = vofs[i];

    constexpr int KA = 2;
    floatx16 s0 = floatx16{};
    half8 ka[KA];
#pragma unroll
    for (int i = 0; i < KA; ++i) ka[i] = *reinterpret_cast<const half8*>(buf + koff[i]);
    // Waves issuing MFMAs run at raised priority, so the SIMD's matrix unit is
    // fed first while other waves are in their softmax (+0.3 % on cfg2).
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      s0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[ks % KA], qreg[ks], s0, 0, 0, 0);
      if (ks + KA < KSTEPS) ka[ks % KA] = *reinterpret_cast<const half8*>(buf + koff[ks + KA]);
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
    constexpr int NMF = 2 * DBLK;
    constexpr int VA = 4;  // V operands read ahead (4: +1.2 % on cfg2 over 3; 5 and 6 no better)
    half8 va[VA];
#pragma unroll
    for (int m = 0; m < VA; ++m) va[m] = ld_vt<D>(buf, voff, m / DBLK, m % DBLK);
    if (k0 + BN > wave_lim_min) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + 8 * (r >> 2) + 4 * half_id + (r & 3);
        if (key >= lim) s0[r] = -INFINITY;
      }
    }
    // The lane's half of the row is tested on its own: the rescale branch,
    // taken for the whole wave when any lane's half exceeds the threshold,
    // takes the full row max (both halves agree on m_ref).
    float mx = max16(s0);
    if (__builtin_amdgcn_ballot_w64(mx > thr_raw) != 0) {
      {
        const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, mx),
                                                         __builtin_bit_cast(uint32_t, mx), false, false);
        mx = vmax3(__builtin_bit_cast(float, (uint32_t)sw[0]),
                   __builtin_bit_cast(float, (uint32_t)sw[1]),
                   __builtin_bit_cast(float, (uint32_t)sw[1])) * c;
      }
      const float m_new = fmaxf(m_ref, mx);
      const float alpha = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_ref - m_new);
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < DBLK; ++i) acc_o[i] = acc_o[i] * alpha;
      m_ref = m_new;
      neg_m_use = m_new == -INFINITY ? 0.f : -m_new;
      thr_raw = (m_new + kRescaleLog2) / c;
    }
    half8 pb[2];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pb[0][j] = (f16)__builtin_amdgcn_exp2f(__builtin_fmaf(s0[j], c, neg_m_use));
      pb[1][j] = (f16)__builtin_amdgcn_exp2f(__builtin_fmaf(s0[8 + j], c, neg_m_use));
    }
    // row sum from the fp16 values the PV product uses, one dot2 chain
#pragma unroll
    for (int st = 0; st < 2; ++st) {
#pragma unroll
      for (int j = 0; j < 8; j += 2)
        l_run = __builtin_amdgcn_fdot2(half2v{pb[st][j], pb[st][j + 1]}, ones, l_run, false);
    }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int m = 0; m < NMF; ++m) {
      const int st = m / DBLK, i = m % DBLK;
      acc_o[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[m % VA], pb[st], acc_o[i], 0, 0, 0);
      if (m + VA < NMF) va[m % VA] = ld_vt<D>(buf, voff, (m + VA) / DBLK, (m + VA) % DBLK);
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
  };
  for (int t = 0; t < ntiles; t += NST) {
    step(std::integral_constant<int, 0>{}, t);
    if (t + 1 < ntiles) step(std::integral_constant<int, 1>{}, t + 1);
    if constexpr (NST == 3) {
      if (t + 2 < ntiles) step(std::integral_constant<int, 2>{}, t + 2);
    }
  }

  // O leaves through LDS (128 rows x 2D bytes, the size of the two K/V
  // stages, with K's chunk swizzle): each wave writes its 32 rows as fp16,
  // then each thread stores whole 16-byte chunks, 16 threads per row, so one
  // store instruction writes 4 complete rows instead of a 16-byte piece of
  // each of 32 rows (with the non-temporal store below: +4.5 % on cfg2).
  // Lane (col, half) holds d = 32i + 8g + 4*half + 0..3 of its row, i.e.
  // half of 16-byte chunk 4i + g.
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = !head_ok ? __builtin_nanf("") : kv_len == 0 ? 0.f : 1.f / l_tot;
  const bool live = qrow < qlen && row_exists;  // padding rows are zeros whatever their Q held
  __syncthreads();  // every wave has finished reading the last K/V stage
  const int lrow = rblk * 32 + col;
#pragma unroll
  for (int i = 0; i < DBLK; ++i) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      half4 h = half4{(f16)(acc_o[i][4 * g + 0] * inv), (f16)(acc_o[i][4 * g + 1] * inv),
                      (f16)(acc_o[i][4 * g + 2] * inv), (f16)(acc_o[i][4 * g + 3] * inv)};
      if (!live) h = half4{0, 0, 0, 0};
      const int chunk = (4 * i + g) ^ C::swz_k(lrow);
      *reinterpret_cast<half4*>(smem + lrow * C::ROWB + 16 * chunk + 8 * half_id) = h;
    }
  }
  __syncthreads();
  const int rows = min(kBM, (PACKED ? pk_rows : p.M) - q0);
  f16* ob = op + (int64_t)q0 * D;
  for (int e = tid; e < rows * C::CH; e += kThreads) {
    const int r = e / C::CH, ch = e % C::CH;
    const half8 v = *reinterpret_cast<const half8*>(smem + r * C::ROWB + 16 * (ch ^ C::swz_k(r)));
    f16* dst;
    if constexpr (PACKED) {
      const int pr = q0 + r, j = pr / p.M;
      dst = reinterpret_cast<f16*>(p.o) + (((int64_t)b * p.Hq + s_pk[j]) * p.M + (pr - j * p.M)) * D;
    } else {
      dst = ob + (int64_t)r * D;
    }
    // O is not read again by this kernel: a non-temporal store keeps the
    // K/V lines that other workgroups still read in L2.
    __builtin_nontemporal_store(v, reinterpret_cast<half8*>(dst + 8 * ch));
  }
  if constexpr (PACKED) {
    // Tile 0 of each pair writes the rows no packed row covers: the pair's
    // heads past pack_heads and, for KV head 0, the heads whose head-map
    // entry is outside [0, Hk): NaN, padding positions zero, as the
    // per-head layout writes them.
    if (qt == 0) {
      const int extra = max(s_pk_n[0] - pk_count, 0);
      const int nh = extra + s_pk_n[1];
      const f16 qnan = (f16)__builtin_nanf("");
      const half8 nan8 = half8{qnan, qnan, qnan, qnan, qnan, qnan, qnan, qnan};
      for (int e = tid; e < nh * p.M * C::CH; e += kThreads) {
        const int ch = e % C::CH, rowi = e / C::CH;
        const int i = rowi / p.M, pos = rowi - i * p.M;
        const int h = i < extra ? s_pk[pk_count + i] : s_bad[i - extra];
        const half8 v = pos < qlen ? nan8 : half8{0, 0, 0, 0, 0, 0, 0, 0};
        f16* d = reinterpret_cast<f16*>(p.o) + (((int64_t)b * p.Hq + h) * p.M + pos) * D;
        *reinterpret_cast<half8*>(d + 8 * ch) = v;
      }
    }
  }
}

// fp32 contiguous attention (the reference's CPU path accepts fp32,
// flashattention_custom/ops.py:19-31), in fp32 arithmetic on the vector ALUs.
// A workgroup takes kF32Rows query rows of one (sequence, q head). Within a
// wave, the four lanes of a row split the head dimension (lane = 4 * row +
// part) and sum their partial dot products with two lane exchanges, so all
// four hold the same score. The eight waves split every LDS tile of 4096/D
// keys (8 keys each at D = 64, 4 at D = 128), and each keeps its own online
// softmax state; the eight states are merged in LDS at the end. So a row's
// keys run on 32 lanes at once (the causal rows at the end of a sequence set
// the kernel's duration), and a 512-row head spreads over 32 workgroups. The
// next tile's K and V rows are loaded into registers while the current tile
// is computed (8 + 8 floats per thread).
constexpr int kF32Rows = 16;
constexpr int kF32Waves = 8;

template <int D>
__global__ __launch_bounds__(64 * kF32Waves) void prefill_f32_kernel(AttnParams p) {
  constexpr int BN = 4096 / D;    // keys per LDS tile
  constexpr int NW = kF32Waves;
  constexpr int NT = 64 * NW;
  constexpr int KPW = BN / NW;    // keys per wave and tile
  constexpr int EPT = BN * D / NT;  // K (and V) elements per thread and tile
  constexpr int DP = D / 4;       // head dims per lane
  __shared__ float sK[BN][D];
  __shared__ float sV[BN][D];
  __shared__ float sM[NW][kF32Rows];
  __shared__ float sL[NW][kF32Rows];
  __shared__ float sO[NW][kF32Rows][D + 1];  // +1: the 16 rows x 4 parts hit 64 banks
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane >> 2;
  const int part = lane & 3;
  const int q0 = blockIdx.x * kF32Rows;
  const int hq = blockIdx.y;
  const int b = blockIdx.z;
  const int qrow = q0 + r;
  const float* qp = reinterpret_cast<const float*>(p.q) + ((int64_t)b * p.Hq + hq) * p.M * D;
  float* op = reinterpret_cast<float*>(p.o) + ((int64_t)b * p.Hq + hq) * p.M * D;
  const float* kp = reinterpret_cast<const float*>(p.k);
  const float* vp = reinterpret_cast<const float*>(p.v);
  const int hk = p.kv_head(hq);
  const int kv_len = p.kv_len(b);
  const int qo = p.q_off(b);
  const int ko = p.k_off(b);

  float q[DP];
#pragma unroll
  for (int i = 0; i < DP; ++i) q[i] = qrow < p.M ? qp[(int64_t)qrow * D + part * DP + i] : 0.f;
  const int last_row = min(q0 + kF32Rows, p.M) - 1;
  const int wg_lim = hk < 0 ? 0 : row_key_limit(kv_len, p.causal, qo, ko, last_row);
  const int lim = row_key_limit(kv_len, p.causal, qo, ko, qrow);
  const float scale = p.scale_log2 / kLog2e;  // 1/sqrt(D)

  float o[DP];
#pragma unroll
  for (int i = 0; i < DP; ++i) o[i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  // Element i of a thread's share of a tile is (key row, dim) = divmod(tid +
  // NT i, D): consecutive threads read consecutive dims of a row.
  float nk[EPT], nv[EPT];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int e = tid + NT * i;
      const int j = k0 + e / D;
      const int64_t off = j < kv_len ? p.kv.row_offset(b, hk, j) : -1;
      nk[i] = off >= 0 ? kp[off + e % D] : 0.f;
      nv[i] = off >= 0 ? vp[off + e % D] : 0.f;
    }
  };
  if (wg_lim > 0) fetch(0);
  for (int k0 = 0; k0 < wg_lim; k0 += BN) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < EPT; ++i) {
      const int e = tid + NT * i;
      sK[e / D][e % D] = nk[i];
      sV[e / D][e % D] = nv[i];
    }
    __syncthreads();
    if (k0 + BN < wg_lim) fetch(k0 + BN);
    float s[KPW];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int kr = wave * KPW + i;
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < DP; ++d) acc = __builtin_fmaf(q[d], sK[kr][part * DP + d], acc);
      // a + b == b + a exactly, so the four lanes of the row agree bit for bit
      acc += __shfl_xor(acc, 1);
      acc += __shfl_xor(acc, 2);
      s[i] = (k0 + kr < lim) ? acc * scale : -INFINITY;
      mx = fmaxf(mx, s[i]);
    }
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = expf(m_run - m_use);
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      s[i] = expf(s[i] - m_use);
      psum += s[i];
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int d = 0; d < DP; ++d) {
      float acc = o[d] * alpha;
#pragma unroll
      for (int i = 0; i < KPW; ++i) acc = __builtin_fmaf(s[i], sV[wave * KPW + i][part * DP + d], acc);
      o[d] = acc;
    }
  }

  // Merge the waves' states per row, then write O (consecutive threads,
  // consecutive dims).
  if (part == 0) {
    sM[wave][r] = m_run;
    sL[wave][r] = l_run;
  }
#pragma unroll
  for (int d = 0; d < DP; ++d) sO[wave][r][part * DP + d] = o[d];
  __syncthreads();
  for (int e = tid; e < kF32Rows * D; e += NT) {
    const int row = e / D, d = e % D;
    if (q0 + row >= p.M) break;
    float val;
    if (hk < 0) {
      val = __builtin_nanf("");
    } else if (kv_len == 0) {
      val = 0.f;  // no keys: zeros (flashattention_custom/ops.py:39, 52-59 with slen == 0)
    } else {
      float m_all = sM[0][row];
#pragma unroll
      for (int w = 1; w < NW; ++w) m_all = fmaxf(m_all, sM[w][row]);
      float l = 0.f, acc = 0.f;
      if (m_all != -INFINITY) {
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const float c = expf(sM[w][row] - m_all);  // a wave with no visible key: 0
          l += c * sL[w][row];
          acc += c * sO[w][row][d];
        }
      }
      val = acc * (1.f / l);  // no visible key: 0 * inf = NaN, the fully masked row
    }
    op[(int64_t)(q0 + row) * D + d] = val;
  }
}

}  // namespace

// The packed layout serves calls with fewer than 128 rows per q head and at
// least two q heads per KV head (pack_heads, from the caller's heads_per_kv),
// on the tile-DMA kernel: it fills 128-row tiles with the (head, position)
// rows of a KV head, where one q head per tile would leave rows empty and
// stream the KV head's pages once per q head.
static bool use_packed_rows(const AttnParams& p) {
  return p.pack_heads >= 2 && p.M < kBM && p.Hq <= kMaxPackHeads && p.Hk > 0;
}

// The work list of prefill_b32_kernel (see PrefillGrid): ntq tiles per pair,
// `group` q heads per pair, `ngroups` pairs per sequence, `total` items.
static PrefillGrid prefill_grid(const AttnParams& p, int D, int ntq, int group, int ngroups,
                                int total, bool packed) {
  PrefillGrid g{};
  g.ntq = ntq;
  g.group = group;
  g.ngroups = ngroups;
  g.total = total;
  g.per_pair = ntq * group;
  g.per_xcd = packed ? 0 : (total + 7) / 8;
  g.order = 0;
  g.tp = 1;
  g.band = group;
  g.gsz = g.per_pair;
  if (!packed && g.per_xcd % g.per_pair == 0 && total == 8 * g.per_xcd) {
    g.kp = g.per_xcd / g.per_pair;
    const bool four_fit = (int64_t)p.N * D * 2 * 2 * 4 <= ((int64_t)4 << 20);
    if (four_fit && g.kp % 4 == 0) {
      g.order = 1;
      g.gsz = 4 * g.per_pair;
      g.band = 4 * group;
    } else {
      g.order = 2;
      g.tp = g.kp >= 2 ? 2 : 1;
      g.head_items = (g.kp - g.tp) * g.per_pair;
      g.band = g.tp * group;
    }
    g.rank = p.seqlen != nullptr && p.q_offsets != nullptr && g.kp > 1 && g.kp <= 64;
  }
  g.d_pair = make_fastdiv(g.per_pair);
  g.d_group = make_fastdiv(group);
  g.d_ngroups = make_fastdiv(ngroups);
  g.d_band = make_fastdiv(g.band);
  g.d_gsz = make_fastdiv(g.gsz);
  return g;
}

hipError_t launch_prefill(const AttnParams& p, int D, int dtype, hipStream_t stream) {
  if (dtype == 1) {
    const dim3 grid((unsigned)((p.M + kF32Rows - 1) / kF32Rows), (unsigned)p.Hq, (unsigned)p.B);
    if (D == 128)
      hipLaunchKernelGGL(prefill_f32_kernel<128>, grid, dim3(64 * kF32Waves), 0, stream, p);
    else
      hipLaunchKernelGGL(prefill_f32_kernel<64>, grid, dim3(64 * kF32Waves), 0, stream, p);
    return hipGetLastError();
  }
  const bool aligned = p.kv.paged ? (p.kv.PS % 16) == 0 : p.kv.stride_tok == p.kv.D;
  const int ntq = (p.M + kBM - 1) / kBM;
  if (!aligned) {
    const dim3 grid((unsigned)ntq, (unsigned)p.Hq, (unsigned)p.B);
    if (D == 128)
      hipLaunchKernelGGL((prefill_f16_kernel<128, false>), grid, dim3(kThreads), 0, stream, p);
    else
      hipLaunchKernelGGL((prefill_f16_kernel<64, false>), grid, dim3(kThreads), 0, stream, p);
    return hipGetLastError();
  }
  if (use_packed_rows(p)) {
    // (head, position) rows of each KV head packed into 128-row tiles
    const int ntp = (int)(((int64_t)p.pack_heads * p.M + kBM - 1) / kBM);
    const PrefillGrid g = prefill_grid(p, D, ntp, 1, p.Hk, ntp * p.Hk * p.B, true);
    const dim3 grid((unsigned)g.total);
    if (D == 128)
      hipLaunchKernelGGL((prefill_b32_kernel<128, true>), grid, dim3(kThreads), 0, stream, p, g);
    else
      hipLaunchKernelGGL((prefill_b32_kernel<64, true>), grid, dim3(kThreads), 0, stream, p, g);
    return hipGetLastError();
  }
  const int group = (p.Hk > 0 && p.Hq % p.Hk == 0) ? p.Hq / p.Hk : 1;
  const PrefillGrid g = prefill_grid(p, D, ntq, group, p.Hq / group, ntq * p.Hq * p.B, false);
  const dim3 grid((unsigned)(8 * g.per_xcd));
  if (D == 128)
    hipLaunchKernelGGL((prefill_b32_kernel<128, false>), grid, dim3(kThreads), 0, stream, p, g);
  else
    hipLaunchKernelGGL((prefill_b32_kernel<64, false>), grid, dim3(kThreads), 0, stream, p, g);
  return hipGetLastError();
}

}  // namespace fa
