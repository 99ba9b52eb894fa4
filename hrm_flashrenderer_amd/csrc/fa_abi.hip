// extern "C" entry points of libfa_mi355x.so (declared in include/fa_mi355x.h).
//
// This layer replaces the reference's pybind module csrc/ext.cpp:30-116: it
// validates sizes (with the reference's messages where the same condition is
// checked), builds the kernel arguments and launches on the caller's stream.
// It never allocates device memory and never synchronises the host. Errors are
// returned as status codes; the message is kept per thread (fa_last_error).
#include "fa_mi355x.h"
#include "fa_common.h"

#include <limits.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>
#include <string>

// Decode scratch of fa_flash_attn_paged_fwd_noalloc: the same partial-result
// workspace that fa_flash_attn_paged_fwd takes from its caller, held in a
// static device array instead (one copy per GPU, for the life of the
// process). 32 MiB covers the decode workspace of (B*Hk + 1024) partial
// slots x 64 rows (e.g. B = 64 sequences of 64/8 heads at M = 8, or B = 2048
// at M = 1, 8 heads per KV head). In host code `scratch` names a host-side
// stand-in: only the address from hipGetSymbolAddress (scratch_base) reaches
// a kernel or a copy.
constexpr size_t kScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int launch_status(hipError_t e) {
  if (e == hipSuccess) return FA_OK;
  return fail(FA_ERR_LAUNCH, "HIP launch failed: %s", hipGetErrorString(e));
}

int ps_shift_of(int ps) {
  if (ps <= 0 || (ps & (ps - 1)) != 0) return -1;
  int s = 0;
  while ((1 << s) < ps) ++s;
  return s;
}

bool head_dim_ok(int D) { return D == 64 || D == 128; }

// Offsets are narrowed to int as the reference launcher does ((int)q_offset,
// csrc/flash_attn_sm75.cu:461, :519).
int narrow(int64_t v) { return (int)v; }

fa::KVMap paged_map(const int32_t* block_table, int max_blocks, int NB, int Hk, int P, int PS,
                    int D) {
  fa::KVMap m;
  m.block_table = block_table;
  m.stride_page = (int64_t)PS * D;
  m.stride_hk = (int64_t)P * m.stride_page;
  m.stride_nb = (int64_t)Hk * m.stride_hk;
  m.stride_tok = D;
  m.max_blocks = block_table ? max_blocks : P;
  m.P = P;
  const int64_t phys = (int64_t)NB * P;
  m.num_phys = phys > INT_MAX ? INT_MAX : (int)phys;
  m.PS = PS;
  m.ps_shift = ps_shift_of(PS);
  m.D = D;
  m.paged = 1;
  return m;
}

int capacity_tokens(int cap_pages, int PS) {
  const int64_t t = (int64_t)cap_pages * PS;
  return t > INT_MAX ? INT_MAX : (int)t;
}

// Shared validation of the paged pool arguments.
int check_pool(int B, int NB, int Hk, int P, int page_size, const int32_t* block_table,
               int max_blocks) {
  if (NB < 0 || Hk <= 0 || P < 0) return fail(FA_ERR_INVALID, "k_pages/v_pages [B,Hk,P,PS,D]");
  if (page_size <= 0) return fail(FA_ERR_INVALID, "page_size mismatch");
  if (block_table == nullptr && NB != B) return fail(FA_ERR_INVALID, "B mismatch");
  if (block_table != nullptr && max_blocks < 0)
    return fail(FA_ERR_INVALID, "block_table [B, max_blocks] required");
  return FA_OK;
}

// Device address of `scratch` on the current device, looked up once per
// device (hipGetSymbolAddress, with that device current) and kept.
std::mutex g_scratch_mu;
void* g_scratch_base[64] = {};

int scratch_base(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
    return fail(FA_ERR_LAUNCH, "no current HIP device for the static scratch");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_base[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(FA_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_base[dev] = ptr;
  }
  *out = g_scratch_base[dev];
  return FA_OK;
}

}  // namespace

extern "C" {

int fa_abi_version(void) { return FA_ABI_VERSION; }

const char* fa_last_error(void) { return g_last_error.c_str(); }

// Whether a contiguous call runs on the decode kernels: fp16, at most 32
// query rows per K/V head (the fused rows of a GQA group), and the paged
// entry's rule for the rest.
static bool contig_decode(int dtype, int B, int Hq, int Hk, int M, int N, int D) {
  if (dtype != FA_DTYPE_F16 || !head_dim_ok(D) || B <= 0 || Hk <= 0 || Hq % Hk != 0 || M <= 0 ||
      N <= 0)
    return false;
  const int group = Hq / Hk;
  return (int64_t)M * group <= 32 && fa::use_decode_path(B, M, Hq, Hk, group);
}

size_t fa_flash_attn_workspace_bytes(int dtype, int B, int Hq, int Hk, int M, int N, int D) {
  if (!contig_decode(dtype, B, Hq, Hk, M, N, D)) return 0;
  return fa::plan_decode(B, Hq, M, D, Hk, N, Hq / Hk).ws_bytes;
}

static int contig_fwd(const void* q, const void* k, const void* v, void* o, int dtype, int B,
                      int Hq, int Hk, int M, int N, int D, int causal, int64_t q_offset,
                      int64_t k_offset, const int32_t* q_offsets, const int32_t* k_offsets,
                      void* workspace, size_t workspace_bytes, bool decode_ok, void* stream);

int fa_flash_attn_fwd(const void* q, const void* k, const void* v, void* o, int dtype, int B,
                      int Hq, int Hk, int M, int N, int D, int causal, int64_t q_offset,
                      int64_t k_offset, const int32_t* q_offsets, const int32_t* k_offsets,
                      void* stream) {
  return contig_fwd(q, k, v, o, dtype, B, Hq, Hk, M, N, D, causal, q_offset, k_offset, q_offsets,
                    k_offsets, nullptr, 0, false, stream);
}

int fa_flash_attn_fwd_ws(const void* q, const void* k, const void* v, void* o, int dtype, int B,
                         int Hq, int Hk, int M, int N, int D, int causal, int64_t q_offset,
                         int64_t k_offset, const int32_t* q_offsets, const int32_t* k_offsets,
                         void* workspace, size_t workspace_bytes, void* stream) {
  return contig_fwd(q, k, v, o, dtype, B, Hq, Hk, M, N, D, causal, q_offset, k_offset, q_offsets,
                    k_offsets, workspace, workspace_bytes, true, stream);
}

static int contig_fwd(const void* q, const void* k, const void* v, void* o, int dtype, int B,
                      int Hq, int Hk, int M, int N, int D, int causal, int64_t q_offset,
                      int64_t k_offset, const int32_t* q_offsets, const int32_t* k_offsets,
                      void* workspace, size_t workspace_bytes, bool decode_ok, void* stream) {
  if (dtype != FA_DTYPE_F16 && dtype != FA_DTYPE_F32)
    return fail(FA_ERR_INVALID, "fp16 or fp32 required");
  if (B < 0 || Hq < 0 || Hk < 0 || M < 0 || N < 0 || D < 0)
    return fail(FA_ERR_INVALID, "q/k/v must be 4D");
  if (Hk == 0 ? Hq != 0 : (Hq % Hk) != 0) return fail(FA_ERR_INVALID, "H mismatch");
  if (!head_dim_ok(D)) return fail(FA_ERR_INVALID, "Supported head_dim: 64 or 128");
  if ((int64_t)B * Hq * M == 0) return FA_OK;
  if (q == nullptr || o == nullptr || (N > 0 && (k == nullptr || v == nullptr)))
    return fail(FA_ERR_INVALID, "null tensor pointer");

  fa::AttnParams p = {};
  p.q = q;
  p.k = k;
  p.v = v;
  p.o = o;
  p.seqlen = nullptr;
  p.head_map = nullptr;
  p.q_offsets = q_offsets;
  p.k_offsets = k_offsets;
  p.kv.block_table = nullptr;
  p.kv.stride_hk = (int64_t)N * D;
  p.kv.stride_nb = (int64_t)Hk * p.kv.stride_hk;
  p.kv.stride_page = 0;
  p.kv.stride_tok = D;
  p.kv.max_blocks = 0;
  p.kv.P = 0;
  p.kv.num_phys = 0;
  p.kv.PS = 1;
  p.kv.ps_shift = 0;
  p.kv.D = D;
  p.kv.paged = 0;
  p.B = B;
  p.Hq = Hq;
  p.Hk = Hk;
  p.M = M;
  p.N = N;
  p.group = Hq / Hk;
  p.pack_heads = p.group;  // rows of one KV head's q heads share 128-row tiles when M < 128
  p.causal = causal ? 1 : 0;
  p.q_offset = narrow(q_offset);
  p.k_offset = narrow(k_offset);
  p.scale_log2 = fa::kLog2e / sqrtf((float)D);
  (void)hipGetLastError();
  if (decode_ok && contig_decode(dtype, B, Hq, Hk, M, N, D)) {
    // split-K decode over the contiguous rows: one slot row per (q head of
    // the group, query position), seqlen = N for every sequence
    const fa::DecodePlan plan = fa::plan_decode(B, Hq, M, D, Hk, N, p.group);
    if (workspace == nullptr || workspace_bytes < plan.ws_bytes)
      return fail(FA_ERR_WORKSPACE, "workspace of %zu bytes required, got %zu", plan.ws_bytes,
                  workspace == nullptr ? (size_t)0 : workspace_bytes);
    char* ws = reinterpret_cast<char*>(workspace);
    hipError_t e = hipSuccess;
    for (int b0 = 0; b0 < B && e == hipSuccess; b0 += fa::kDecodeMaxBatch) {
      const int Bc = std::min(fa::kDecodeMaxBatch, B - b0);
      fa::AttnParams pc = p;
      const int64_t qrows = (int64_t)b0 * Hq * M * D;
      pc.q = reinterpret_cast<const fa::f16*>(q) + qrows;
      pc.o = reinterpret_cast<fa::f16*>(o) + qrows;
      pc.k = reinterpret_cast<const fa::f16*>(k) + b0 * p.kv.stride_nb;
      pc.v = reinterpret_cast<const fa::f16*>(v) + b0 * p.kv.stride_nb;
      if (q_offsets != nullptr) pc.q_offsets = q_offsets + b0;
      if (k_offsets != nullptr) pc.k_offsets = k_offsets + b0;
      pc.B = Bc;
      const fa::DecodePlan cplan = fa::plan_decode(Bc, Hq, M, D, Hk, N, p.group);
      pc.ws_o = reinterpret_cast<float*>(ws);
      pc.ws_ml = reinterpret_cast<float*>(ws + plan.o_bytes);
      pc.ws_units = reinterpret_cast<int*>(ws + plan.o_bytes + plan.ml_bytes);
      pc.ws_app = pc.ws_units + (Bc + 1);
      pc.dec_rows = cplan.rows;
      pc.dec_seg_cost = fa::kSegmentCost;
      pc.dec_wgs = fa::decode_launch_wgs(cplan, pc, D);
      e = fa::launch_decode(pc, D, (hipStream_t)stream);
    }
    return launch_status(e);
  }
  return launch_status(fa::launch_prefill(p, D, dtype, (hipStream_t)stream));
}

size_t fa_paged_workspace_bytes(int B, int Hq, int M, int D, int Hk, int capacity_pages,
                                int page_size, int heads_per_kv) {
  if (B <= 0 || Hq <= 0 || M <= 0 || Hk <= 0 || !head_dim_ok(D)) return 0;
  if (!fa::use_decode_path(B, M, Hq, Hk, heads_per_kv)) return 0;
  const int cap = capacity_tokens(capacity_pages < 0 ? 0 : capacity_pages,
                                  page_size < 1 ? 1 : page_size);
  return fa::plan_decode(B, Hq, M, D, Hk, cap, heads_per_kv).ws_bytes;
}

// The new token of fa_flash_attn_paged_append_fwd (k_new / v_new
// [B, Hk, 1, D]) and where it goes.
struct AppendArgs {
  const void* k_new;
  const void* v_new;
  int advance;                     // position seqlen[b]; seqlen[b] += 1 afterwards
  int64_t start_pos;               // position without advance, unless start_positions
  const int32_t* start_positions;  // nullable [B]
};

static int paged_fwd(const void* q, const void* k_pages, const void* v_pages,
                     const int32_t* seqlen, int page_size, const int32_t* head_map, void* o, int B,
                     int Hq, int M, int D, int NB, int Hk, int P, int causal, int64_t q_offset,
                     int64_t k_offset, const int32_t* q_offsets, const int32_t* k_offsets,
                     const int32_t* q_lens, const int32_t* block_table, int max_blocks,
                     int heads_per_kv, void* workspace,
                     size_t workspace_bytes, const void* rope_cos, const void* rope_sin,
                     int rope_len, void* stream, bool decode_ok = true,
                     const AppendArgs* app = nullptr) {
  if (B < 0 || Hq < 0 || M < 0 || D < 0) return fail(FA_ERR_INVALID, "q [B,Hq,M,D]");
  int rc = check_pool(B, NB, Hk, P, page_size, block_table, max_blocks);
  if (rc != FA_OK) return rc;
  if (!head_dim_ok(D)) return fail(FA_ERR_INVALID, "Supported head_dim: 64 or 128");
  if (app != nullptr && (int64_t)B * Hk > 0 &&
      (app->k_new == nullptr || app->v_new == nullptr || seqlen == nullptr ||
       k_pages == nullptr || v_pages == nullptr))
    return fail(FA_ERR_INVALID, "null tensor pointer");
  if (app == nullptr && (int64_t)B * Hq * M == 0) return FA_OK;
  if ((int64_t)B * Hq * M > 0 &&
      (q == nullptr || o == nullptr || seqlen == nullptr || head_map == nullptr ||
       ((int64_t)NB * P > 0 && (k_pages == nullptr || v_pages == nullptr))))
    return fail(FA_ERR_INVALID, "null tensor pointer");

  const int PS = page_size;
  fa::AttnParams p = {};
  p.q = q;
  p.k = k_pages;
  p.v = v_pages;
  p.o = o;
  p.seqlen = seqlen;
  p.head_map = head_map;
  p.q_offsets = q_offsets;
  p.k_offsets = k_offsets;
  p.q_lens = q_lens;
  p.kv = paged_map(block_table, max_blocks, NB, Hk, P, PS, D);
  p.B = B;
  p.Hq = Hq;
  p.Hk = Hk;
  p.M = M;
  p.N = capacity_tokens(p.kv.max_blocks, PS);
  p.group = 1;
  p.causal = causal ? 1 : 0;
  p.q_offset = narrow(q_offset);
  p.k_offset = narrow(k_offset);
  p.scale_log2 = fa::kLog2e / sqrtf((float)D);
  p.rope_cos = reinterpret_cast<const fa::f16*>(rope_cos);
  p.rope_sin = reinterpret_cast<const fa::f16*>(rope_sin);
  p.rope_len = rope_len;

  (void)hipGetLastError();
  const bool decode = decode_ok && fa::use_decode_path(B, M, Hq, Hk, heads_per_kv);
  if (app != nullptr) {
    p.app_advance = app->advance ? 1 : 0;
    // the decode kernels take the token in advance mode, where it is every
    // sequence's last key (its group comes last; fa_decode.hip). With rotary
    // tables the append kernel runs first instead: at cfg4 the step measured
    // 367.1 against 368.4 us fused (same-process A/B), the decode kernels
    // rotating q either way.
    if (decode && app->advance && rope_cos == nullptr &&
        fa::fused_append_ok(B, M, Hq, Hk, heads_per_kv)) {
      // the decode kernels take the new token (fa_decode.hip, APPEND)
      p.app_k = reinterpret_cast<const fa::f16*>(app->k_new);
      p.app_v = reinterpret_cast<const fa::f16*>(app->v_new);
    } else {
      // append kernel first (positions seqlen[b] with advance, read before
      // the advance below), then the attention over the appended pages
      hipError_t e = fa::launch_paged_append(
          const_cast<void*>(k_pages), const_cast<void*>(v_pages), app->k_new, app->v_new, p.kv,
          B, Hk, 1, narrow(app->start_pos), app->advance ? seqlen : app->start_positions,
          nullptr, p.rope_cos, p.rope_sin, rope_len, (hipStream_t)stream);
      if (e != hipSuccess) return launch_status(e);
    }
  }
  hipError_t e = hipSuccess;
  bool combine_advances = false;  // the decode path's combine kernel advances the lengths
  if ((int64_t)B * Hq * M == 0) {
    // nothing to attend: the append alone
    if (p.app_k != nullptr) {
      p.app_k = nullptr;
      e = fa::launch_paged_append(const_cast<void*>(k_pages), const_cast<void*>(v_pages),
                                  app->k_new, app->v_new, p.kv, B, Hk, 1,
                                  narrow(app->start_pos),
                                  app->advance ? seqlen : app->start_positions, nullptr,
                                  p.rope_cos, p.rope_sin, rope_len, (hipStream_t)stream);
    }
  } else if (decode) {
    // plan_decode sizes the workspace for one launch of at most
    // kDecodeMaxBatch sequences; a larger batch runs in such launches one
    // after another on the stream, each on the workspace the previous one
    // has finished with (its combine kernel runs before the next launch).
    const fa::DecodePlan plan = fa::plan_decode(B, Hq, M, D, Hk, p.N, heads_per_kv);
    if (workspace == nullptr || workspace_bytes < plan.ws_bytes)
      return fail(FA_ERR_WORKSPACE, "workspace of %zu bytes required, got %zu", plan.ws_bytes,
                  workspace == nullptr ? (size_t)0 : workspace_bytes);
    char* ws = reinterpret_cast<char*>(workspace);
    for (int b0 = 0; b0 < B && e == hipSuccess; b0 += fa::kDecodeMaxBatch) {
      const int Bc = std::min(fa::kDecodeMaxBatch, B - b0);
      fa::AttnParams pc = p;
      if (b0 > 0) {
        // the chunk's sequences: per-sequence arrays and rows from b0 on; the
        // pool rows too when the pages are per sequence (no block table)
        const int64_t qrows = (int64_t)b0 * Hq * M * D;
        pc.q = reinterpret_cast<const fa::f16*>(q) + qrows;
        pc.o = reinterpret_cast<fa::f16*>(o) + qrows;
        pc.seqlen = seqlen + b0;
        if (q_offsets != nullptr) pc.q_offsets = q_offsets + b0;
        if (k_offsets != nullptr) pc.k_offsets = k_offsets + b0;
        if (q_lens != nullptr) pc.q_lens = q_lens + b0;
        if (block_table != nullptr) {
          pc.kv.block_table = block_table + (int64_t)b0 * max_blocks;
        } else {
          pc.k = reinterpret_cast<const fa::f16*>(k_pages) + b0 * p.kv.stride_nb;
          pc.v = reinterpret_cast<const fa::f16*>(v_pages) + b0 * p.kv.stride_nb;
        }
        if (pc.app_k != nullptr) {
          pc.app_k += (int64_t)b0 * Hk * D;
          pc.app_v += (int64_t)b0 * Hk * D;
        }
      }
      pc.B = Bc;
      const fa::DecodePlan cplan = fa::plan_decode(Bc, Hq, M, D, Hk, p.N, heads_per_kv);
      pc.ws_o = reinterpret_cast<float*>(ws);
      pc.ws_ml = reinterpret_cast<float*>(ws + plan.o_bytes);
      pc.ws_units = reinterpret_cast<int*>(ws + plan.o_bytes + plan.ml_bytes);
      pc.ws_app = pc.ws_units + (Bc + 1);
      // every field decode_variant reads is set before the occupancy query
      pc.dec_rows = cplan.rows;
      pc.dec_seg_cost = PS % 16 == 0 ? fa::kSegmentCost : 0;
      pc.dec_wgs = fa::decode_launch_wgs(cplan, pc, D);
      e = fa::launch_decode(pc, D, (hipStream_t)stream);
    }
    combine_advances = true;
  } else {
    // the prefill kernel packs the rows of a KV head's q heads (at most
    // heads_per_kv of them) into shared 128-row tiles when M < 128
    p.pack_heads = heads_per_kv > 0 ? std::min(heads_per_kv, Hq) : 0;
    e = fa::launch_prefill(p, D, FA_DTYPE_F16, (hipStream_t)stream);
  }
  // the decode path's combine kernel advances the lengths itself (from the
  // copy the decode kernel published); the other paths need a launch
  if (e == hipSuccess && app != nullptr && app->advance && !combine_advances)
    e = fa::launch_advance_lengths(const_cast<int32_t*>(seqlen), B, (hipStream_t)stream);
  return launch_status(e);
}

int fa_flash_attn_paged_fwd(const void* q, const void* k_pages, const void* v_pages,
                            const int32_t* seqlen, int page_size, const int32_t* head_map, void* o,
                            int B, int Hq, int M, int D, int NB, int Hk, int P, int causal,
                            int64_t q_offset, int64_t k_offset, const int32_t* q_offsets,
                            const int32_t* k_offsets, const int32_t* q_lens,
                            const int32_t* block_table, int max_blocks, int heads_per_kv,
                            void* workspace, size_t workspace_bytes, void* stream) {
  return paged_fwd(q, k_pages, v_pages, seqlen, page_size, head_map, o, B, Hq, M, D, NB, Hk, P,
                   causal, q_offset, k_offset, q_offsets, k_offsets, q_lens, block_table,
                   max_blocks, heads_per_kv, workspace, workspace_bytes, nullptr, nullptr, 0,
                   stream);
}

int fa_flash_attn_paged_rope_fwd(const void* q, const void* k_pages, const void* v_pages,
                                 const int32_t* seqlen, int page_size, const int32_t* head_map,
                                 void* o, int B, int Hq, int M, int D, int NB, int Hk, int P,
                                 int causal, int64_t q_offset, int64_t k_offset,
                                 const int32_t* q_offsets, const int32_t* k_offsets,
                                 const int32_t* q_lens, const int32_t* block_table,
                                 int max_blocks, int heads_per_kv, void* workspace,
                                 size_t workspace_bytes, const void* rope_cos,
                                 const void* rope_sin, int rope_len, void* stream) {
  if (rope_cos == nullptr || rope_sin == nullptr || rope_len <= 0)
    return fail(FA_ERR_INVALID, "rotary tables cos/sin [L, D/2] required");
  return paged_fwd(q, k_pages, v_pages, seqlen, page_size, head_map, o, B, Hq, M, D, NB, Hk, P,
                   causal, q_offset, k_offset, q_offsets, k_offsets, q_lens, block_table,
                   max_blocks, heads_per_kv, workspace, workspace_bytes, rope_cos, rope_sin,
                   rope_len, stream);
}

int fa_flash_attn_paged_fwd_noalloc(const void* q, const void* k_pages, const void* v_pages,
                                    const int32_t* seqlen, int page_size,
                                    const int32_t* head_map, void* o, int B, int Hq, int M,
                                    int D, int NB, int Hk, int P, int causal, int64_t q_offset,
                                    int64_t k_offset, const int32_t* q_offsets,
                                    const int32_t* k_offsets, const int32_t* q_lens,
                                    const int32_t* block_table, int max_blocks,
                                    int heads_per_kv, void* stream) {
  const int cap_pages = block_table != nullptr ? max_blocks : P;
  size_t need = fa_paged_workspace_bytes(B, Hq, M, D, Hk, cap_pages, page_size, heads_per_kv);
  // More than 64 query rows per KV head also run on the prefill kernel, which
  // needs no scratch: it takes them when the decode kernels' passes would not
  // fit the scratch.
  const bool rows_gt_64 = Hk > 0 && (int64_t)M * ((Hq + Hk - 1) / Hk) > 64;
  const bool decode_ok = need <= kScratchBytes || !rows_gt_64;
  if (!decode_ok) need = 0;
  if (need > kScratchBytes)
    return fail(FA_ERR_WORKSPACE,
                "these shapes need %zu bytes of decode scratch; the allocation-free entry "
                "holds %zu (call fa_flash_attn_paged_fwd with a workspace)",
                need, kScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_base(&ws);
    if (rc != FA_OK) return rc;
  }
  return paged_fwd(q, k_pages, v_pages, seqlen, page_size, head_map, o, B, Hq, M, D, NB, Hk, P,
                   causal, q_offset, k_offset, q_offsets, k_offsets, q_lens, block_table,
                   max_blocks, heads_per_kv, ws, need > 0 ? kScratchBytes : 0, nullptr, nullptr,
                   0, stream, decode_ok);
}

int fa_flash_attn_paged_append_fwd(const void* q, void* k_pages, void* v_pages, int32_t* seqlen,
                                   int page_size, const int32_t* head_map, void* o, int B, int Hq,
                                   int M, int D, int NB, int Hk, int P, int causal,
                                   int64_t q_offset, const int32_t* q_offsets,
                                   const int32_t* block_table, int max_blocks, int heads_per_kv,
                                   const void* k_new, const void* v_new, int advance,
                                   int64_t start_pos, const int32_t* start_positions,
                                   const void* rope_cos, const void* rope_sin, int rope_len,
                                   void* workspace, size_t workspace_bytes, void* stream) {
  if (advance != 0 && advance != 1) return fail(FA_ERR_INVALID, "advance must be 0 or 1");
  if (advance && (start_positions != nullptr || start_pos != 0))
    return fail(FA_ERR_INVALID, "with advance the positions are the lengths: no start positions");
  if ((rope_cos == nullptr) != (rope_sin == nullptr) || (rope_cos != nullptr && rope_len <= 0))
    return fail(FA_ERR_INVALID, "rotary tables cos/sin [L, D/2] required");
  const AppendArgs app = {k_new, v_new, advance, start_pos, start_positions};
  return paged_fwd(q, k_pages, v_pages, seqlen, page_size, head_map, o, B, Hq, M, D, NB, Hk, P,
                   causal, q_offset, 0, q_offsets, nullptr, nullptr, block_table, max_blocks,
                   heads_per_kv, workspace, workspace_bytes, rope_cos, rope_sin,
                   rope_cos != nullptr ? rope_len : 0, stream, true, &app);
}

static int kv_append(void* k_pages, void* v_pages, const void* k_new, const void* v_new, int B,
                     int Hk, int T, int D, int NB, int P, int page_size, int64_t start_pos,
                     const int32_t* start_positions, const int32_t* token_positions,
                     const int32_t* block_table, int max_blocks, const void* rope_cos,
                     const void* rope_sin, int rope_len, void* stream) {
  if (B < 0 || T < 0 || D <= 0) return fail(FA_ERR_INVALID, "shape mismatch");
  int rc = check_pool(B, NB, Hk, P, page_size, block_table, max_blocks);
  if (rc != FA_OK) return rc;
  if (D % 8 != 0) return fail(FA_ERR_INVALID, "head_dim must be a multiple of 8");
  if (rope_cos != nullptr && D % 16 != 0)
    return fail(FA_ERR_INVALID, "rotary append needs head_dim a multiple of 16");
  if ((int64_t)B * Hk * T == 0) return FA_OK;
  if (k_pages == nullptr || v_pages == nullptr || k_new == nullptr || v_new == nullptr)
    return fail(FA_ERR_INVALID, "null tensor pointer");
  const fa::KVMap map = paged_map(block_table, max_blocks, NB, Hk, P, page_size, D);
  (void)hipGetLastError();
  return launch_status(fa::launch_paged_append(
      k_pages, v_pages, k_new, v_new, map, B, Hk, T, narrow(start_pos), start_positions,
      token_positions, reinterpret_cast<const fa::f16*>(rope_cos),
      reinterpret_cast<const fa::f16*>(rope_sin),
      rope_len, (hipStream_t)stream));
}

int fa_paged_kv_append(void* k_pages, void* v_pages, const void* k_new, const void* v_new, int B,
                       int Hk, int T, int D, int NB, int P, int page_size, int64_t start_pos,
                       const int32_t* start_positions, const int32_t* block_table, int max_blocks,
                       void* stream) {
  return kv_append(k_pages, v_pages, k_new, v_new, B, Hk, T, D, NB, P, page_size, start_pos,
                   start_positions, nullptr, block_table, max_blocks, nullptr, nullptr, 0, stream);
}

int fa_paged_kv_append_rope(void* k_pages, void* v_pages, const void* k_new, const void* v_new,
                            int B, int Hk, int T, int D, int NB, int P, int page_size,
                            int64_t start_pos, const int32_t* start_positions,
                            const int32_t* block_table, int max_blocks, const void* rope_cos,
                            const void* rope_sin, int rope_len, void* stream) {
  if (rope_cos == nullptr || rope_sin == nullptr || rope_len <= 0)
    return fail(FA_ERR_INVALID, "rotary tables cos/sin [L, D/2] required");
  return kv_append(k_pages, v_pages, k_new, v_new, B, Hk, T, D, NB, P, page_size, start_pos,
                   start_positions, nullptr, block_table, max_blocks, rope_cos, rope_sin, rope_len,
                   stream);
}

int fa_paged_kv_scatter(void* k_pages, void* v_pages, const void* k_new, const void* v_new, int B,
                        int Hk, int T, int D, int NB, int P, int page_size,
                        const int32_t* positions, const int32_t* block_table, int max_blocks,
                        const void* rope_cos, const void* rope_sin, int rope_len, void* stream) {
  if (positions == nullptr && (int64_t)B * Hk * T > 0)
    return fail(FA_ERR_INVALID, "positions [B, T] required");
  if ((rope_cos == nullptr) != (rope_sin == nullptr) || (rope_cos != nullptr && rope_len <= 0))
    return fail(FA_ERR_INVALID, "rotary tables cos/sin [L, D/2] required");
  return kv_append(k_pages, v_pages, k_new, v_new, B, Hk, T, D, NB, P, page_size, 0, nullptr,
                   positions, block_table, max_blocks, rope_cos, rope_sin, rope_len, stream);
}

// Most query heads one KV head serves: the engine's map h % KVH (no head
// map) gives at most ceil(H / KVH); an explicit head map states its own bound
// (<= 0: H, no assumption).
static int token_major_hpk(int H, int KVH, int heads_per_kv, bool engine_map) {
  if (engine_map) return (H + KVH - 1) / KVH;
  return heads_per_kv <= 0 || heads_per_kv > H ? H : heads_per_kv;
}

// The token-major step's decode plan. Its segments serve KV heads in pairs
// (AttnParams::kv_pair) when the head count is even and a pair's query rows
// fit one 16-row block (two heads of at most 8 query heads each): then Hk
// counts the pairs, a slot holds both heads' rows, and a segment has twice
// the 16-key groups (capacity passed as 32 keys per group of the sequence).
struct TokenMajorPlan {
  fa::DecodePlan plan;
  int pair;
};
static TokenMajorPlan token_major_plan(int H, int KVH, int Dh, int n_keys, int hpk) {
  TokenMajorPlan t;
  t.pair = KVH % 2 == 0 && 2 * hpk <= 16 ? 1 : 0;
  if (t.pair) {
    const int64_t cap = (int64_t)32 * ((n_keys + 15) / 16);
    t.plan = fa::plan_decode(1, H, 1, Dh, KVH / 2, cap > INT_MAX ? INT_MAX : (int)cap, 2 * hpk);
  } else {
    t.plan = fa::plan_decode(1, H, 1, Dh, KVH, n_keys, hpk);
  }
  return t;
}

size_t fa_decode_token_major_workspace_bytes(int H, int KVH, int Dh, int t_max,
                                             int heads_per_kv) {
  if (H <= 0 || KVH <= 0 || !head_dim_ok(Dh) || t_max < 0 || t_max >= INT_MAX) return 0;
  if (!fa::use_decode_path(1, 1, H, KVH, 0)) return 0;
  // the larger of the plans a launch may take (without a head map the bound
  // is ceil(H / KVH), which is at most the one assumed here)
  const int hpk = token_major_hpk(H, KVH, heads_per_kv, false);
  size_t need = token_major_plan(H, KVH, Dh, t_max + 1, hpk).plan.ws_bytes;
  if (heads_per_kv <= 0) {
    const int hpk_engine = token_major_hpk(H, KVH, 0, true);
    need = std::max(need, token_major_plan(H, KVH, Dh, t_max + 1, hpk_engine).plan.ws_bytes);
  }
  return need;
}

int fa_decode_token_major(float* out, const float* q, const void* k_cache, const void* v_cache,
                          int t, int H, int KVH, int Dh, float scale, const int32_t* head_map,
                          int heads_per_kv, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (H <= 0 || KVH <= 0) return fail(FA_ERR_INVALID, "H and KVH must be positive");
  if (!head_dim_ok(Dh)) return fail(FA_ERR_INVALID, "Supported head_dim: 64 or 128");
  if (t < 0 || t >= INT_MAX) return fail(FA_ERR_INVALID, "position t out of range");
  if (!isfinite(scale)) return fail(FA_ERR_INVALID, "scale must be finite");
  if (!fa::use_decode_path(1, 1, H, KVH, 0))
    return fail(FA_ERR_INVALID, "unsupported head counts H=%d KVH=%d", H, KVH);
  if (out == nullptr || q == nullptr || k_cache == nullptr || v_cache == nullptr)
    return fail(FA_ERR_INVALID, "null tensor pointer");

  fa::AttnParams p = {};
  p.q = q;
  p.q_f32 = 1;
  p.k = k_cache;
  p.v = v_cache;
  p.o = out;
  p.o_f32 = 1;
  p.seqlen = nullptr;  // all t + 1 rows
  p.head_map = head_map;
  p.head_mod = head_map == nullptr ? 1 : 0;
  p.kv.block_table = nullptr;
  p.kv.stride_nb = 0;
  p.kv.stride_hk = Dh;
  p.kv.stride_tok = (int64_t)KVH * Dh;
  p.kv.stride_page = 0;
  p.kv.max_blocks = 0;
  p.kv.P = 0;
  p.kv.num_phys = 0;
  p.kv.PS = 1;
  p.kv.ps_shift = 0;
  p.kv.D = Dh;
  p.kv.paged = 0;
  p.B = 1;
  p.Hq = H;
  p.Hk = KVH;
  p.M = 1;
  p.N = t + 1;
  p.group = H >= KVH ? H / KVH : 1;
  p.causal = 0;
  p.scale_log2 = scale * fa::kLog2e;

  (void)hipGetLastError();
  const TokenMajorPlan tp = token_major_plan(
      H, KVH, Dh, p.N, token_major_hpk(H, KVH, heads_per_kv, head_map == nullptr));
  const fa::DecodePlan& plan = tp.plan;
  p.kv_pair = tp.pair;
  p.Hk = KVH >> tp.pair;
  if (workspace == nullptr || workspace_bytes < plan.ws_bytes)
    return fail(FA_ERR_WORKSPACE, "workspace of %zu bytes required, got %zu", plan.ws_bytes,
                workspace == nullptr ? (size_t)0 : workspace_bytes);
  char* ws = reinterpret_cast<char*>(workspace);
  p.ws_o = reinterpret_cast<float*>(ws);
  p.ws_ml = reinterpret_cast<float*>(ws + plan.o_bytes);
  p.ws_units = reinterpret_cast<int*>(ws + plan.o_bytes + plan.ml_bytes);
  p.dec_rows = plan.rows;
  p.dec_seg_cost = 0;  // B = 1: a workgroup opens at most two segments
  p.dec_wgs = fa::decode_launch_wgs(plan, p, Dh);  // strided whole-group loads, fp32 query split
  return launch_status(fa::launch_decode(p, Dh, (hipStream_t)stream));
}

}  // extern "C"
