// Paged KV append for gfx950.
//
// Semantics follow the reference's paged_kv_append_kernel
// (csrc/flash_attn_sm75.cu:528-555) and its CPU twin
// (flashattention_custom/ops.py:63-72): token t of sequence b goes to position
// start + t, i.e. page (start+t)/PS, slot (start+t)%PS, for every KV head.
// Positions whose page is out of range are skipped (reference :548).
// With per-token positions ([B, T], the general path of the reference's
// cache, engine/llama_tp.py:80-99), token t of sequence b goes to
// positions[b*T + t] instead; negative positions are skipped.
//
// Each lane's source loads are issued first (every index below total_chunks is
// in bounds), so their round trip overlaps the dependent position and
// block-table loads that give the destination.
//
// Layout of the work: one lane moves one 16-byte chunk (8 fp16) of K and the
// same chunk of V. Consecutive lanes take consecutive chunks of a token row,
// then consecutive tokens, so both the source rows [B,Hk,T,D] and the
// destination slots (consecutive within a page) are written as whole 64-byte
// segments per quarter-wave. Work is split as (b, hk, t, chunk); when the chunk
// count D/8 is a power of two (D = 64, 128) the chunk index is a mask and a
// shift, otherwise a division. The index arithmetic is 32-bit (I = uint32_t)
// whenever the lane count fits, since 64-bit division is a long software
// sequence ahead of every load; the 64-bit form serves larger appends.
#include "fa_common.h"

namespace fa {

// row = (b*Hk + hk)*T + t
template <typename I>
__device__ __forceinline__ void split_row(I row, int T, int Hk, int& b, int& hk, int& t) {
  const I bh = row / (I)T;
  t = (int)(row - bh * (I)T);
  const I bq = bh / (I)Hk;
  hk = (int)(bh - bq * (I)Hk);
  b = (int)bq;
}

template <typename I>
__global__ __launch_bounds__(256) void paged_append_kernel(
    f16* __restrict__ k_pages, f16* __restrict__ v_pages,
    const f16* __restrict__ k_new, const f16* __restrict__ v_new,
    KVMap map, int B, int Hk, int T, int chunks_per_row, int chunk_shift, int start_pos,
    const int32_t* __restrict__ start_positions, const int32_t* __restrict__ token_positions,
    int64_t total_chunks) {
  const I idx = (I)blockIdx.x * (I)blockDim.x + (I)threadIdx.x;
  if ((int64_t)idx >= total_chunks) return;
  int chunk;
  I row;
  if (chunk_shift >= 0) {
    chunk = (int)(idx & (I)((1 << chunk_shift) - 1));
    row = idx >> chunk_shift;
  } else {
    row = idx / (I)chunks_per_row;
    chunk = (int)(idx - row * (I)chunks_per_row);
  }
  int b, hk, t;
  split_row<I>(row, T, Hk, b, hk, t);

  const int64_t src = (int64_t)row * map.D + chunk * 8;
  const u32x4 kv = *reinterpret_cast<const u32x4*>(k_new + src);
  const u32x4 vv = *reinterpret_cast<const u32x4*>(v_new + src);

  const int pos = token_positions ? token_positions[(int64_t)b * T + t]
                                  : (start_positions ? start_positions[b] : start_pos) + t;
  if (pos < 0) return;
  const int64_t dst_row = map.row_offset(b, hk, pos);
  if (dst_row < 0) return;

  const int64_t dst = dst_row + chunk * 8;
  *reinterpret_cast<u32x4*>(k_pages + dst) = kv;
  *reinterpret_cast<u32x4*>(v_pages + dst) = vv;
}

// Append with the rotary embedding of K fused in (the reference applies
// engine/rope.py:15-24 to K before llama_tp.py:74 appends it). One lane takes
// the 8-element chunk c < D/16 of a row together with its rotary partner
// c + D/16: it rotates and writes both K chunks and copies both V chunks.
// A position outside the rotary table writes NaN keys.
template <typename I>
__global__ __launch_bounds__(256) void paged_append_rope_kernel(
    f16* __restrict__ k_pages, f16* __restrict__ v_pages,
    const f16* __restrict__ k_new, const f16* __restrict__ v_new,
    KVMap map, int B, int Hk, int T, int pairs_per_row, int start_pos,
    const int32_t* __restrict__ start_positions, const int32_t* __restrict__ token_positions,
    const f16* __restrict__ rope_cos,
    const f16* __restrict__ rope_sin, int rope_len, int64_t total_pairs) {
  const I idx = (I)blockIdx.x * (I)blockDim.x + (I)threadIdx.x;
  if ((int64_t)idx >= total_pairs) return;
  const I row = idx / (I)pairs_per_row;
  const int pair = (int)(idx - row * (I)pairs_per_row);
  int b, hk, t;
  split_row<I>(row, T, Hk, b, hk, t);

  const int half = map.D / 2;
  const int64_t src = (int64_t)row * map.D + pair * 8;
  const half8 x1 = *reinterpret_cast<const half8*>(k_new + src);
  const half8 x2 = *reinterpret_cast<const half8*>(k_new + src + half);
  const u32x4 v1 = *reinterpret_cast<const u32x4*>(v_new + src);
  const u32x4 v2 = *reinterpret_cast<const u32x4*>(v_new + src + half);

  const int pos = token_positions ? token_positions[(int64_t)b * T + t]
                                  : (start_positions ? start_positions[b] : start_pos) + t;
  if (pos < 0) return;
  const int64_t dst_row = map.row_offset(b, hk, pos);
  if (dst_row < 0) return;
  const int64_t dst = dst_row + pair * 8;
  const bool ok = pos < rope_len;
  const int64_t trow = (int64_t)(ok ? pos : 0) * half + pair * 8;
  const half8 c = *reinterpret_cast<const half8*>(rope_cos + trow);
  const half8 s = *reinterpret_cast<const half8*>(rope_sin + trow);
  half8 y1, y2;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    f16 a, e;
    rope_pair(x1[j], x2[j], c[j], s[j], a, e);
    y1[j] = ok ? a : (f16)__builtin_nanf("");
    y2[j] = ok ? e : (f16)__builtin_nanf("");
  }
  *reinterpret_cast<half8*>(k_pages + dst) = y1;
  *reinterpret_cast<half8*>(k_pages + dst + half) = y2;
  *reinterpret_cast<u32x4*>(v_pages + dst) = v1;
  *reinterpret_cast<u32x4*>(v_pages + dst + half) = v2;
}

__global__ __launch_bounds__(256) void advance_lengths_kernel(int32_t* __restrict__ seqlen, int B) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < B) seqlen[b] += 1;
}

hipError_t launch_advance_lengths(int32_t* seqlen, int B, hipStream_t stream) {
  if (B <= 0) return hipSuccess;
  hipLaunchKernelGGL(advance_lengths_kernel, dim3((unsigned)((B + 255) / 256)), dim3(256), 0,
                     stream, seqlen, B);
  return hipGetLastError();
}

hipError_t launch_paged_append(void* k_pages, void* v_pages, const void* k_new, const void* v_new,
                               const KVMap& map, int B, int Hk, int T, int start_pos,
                               const int32_t* start_positions, const int32_t* token_positions,
                               const f16* rope_cos, const f16* rope_sin, int rope_len,
                               hipStream_t stream) {
  const int threads = 256;
  if (rope_cos != nullptr) {
    const int pairs_per_row = map.D / 16;
    const int64_t total = (int64_t)B * Hk * T * pairs_per_row;
    if (total == 0) return hipSuccess;
    const int64_t blocks = (total + threads - 1) / threads;
    auto fn = total + threads < ((int64_t)1 << 31) ? paged_append_rope_kernel<uint32_t>
                                                   : paged_append_rope_kernel<int64_t>;
    hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(threads), 0, stream,
                       reinterpret_cast<f16*>(k_pages), reinterpret_cast<f16*>(v_pages),
                       reinterpret_cast<const f16*>(k_new), reinterpret_cast<const f16*>(v_new),
                       map, B, Hk, T, pairs_per_row, start_pos, start_positions,
                       token_positions, rope_cos, rope_sin, rope_len, total);
    return hipGetLastError();
  }
  const int chunks_per_row = map.D / 8;
  int chunk_shift = 0;
  while ((1 << chunk_shift) < chunks_per_row) ++chunk_shift;
  if ((1 << chunk_shift) != chunks_per_row) chunk_shift = -1;
  const int64_t total = (int64_t)B * Hk * T * chunks_per_row;
  if (total == 0) return hipSuccess;
  const int64_t blocks = (total + threads - 1) / threads;
  auto fn = total + threads < ((int64_t)1 << 31) ? paged_append_kernel<uint32_t>
                                                 : paged_append_kernel<int64_t>;
  hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(threads), 0, stream,
                     reinterpret_cast<f16*>(k_pages), reinterpret_cast<f16*>(v_pages),
                     reinterpret_cast<const f16*>(k_new), reinterpret_cast<const f16*>(v_new), map,
                     B, Hk, T, chunks_per_row, chunk_shift, start_pos, start_positions,
                     token_positions, total);
  return hipGetLastError();
}

}  // namespace fa
