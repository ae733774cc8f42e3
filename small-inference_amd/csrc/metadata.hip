// Per-forward packed metadata built on the device from persistent block tables.
//
// Reference: engine/paged_cache.py:55-90 (build_metadata) builds, for a forward over sequences with n_s new tokens
// at positions start_s .. start_s + n_s - 1: query_starts (cumulative counts), positions, slot_mapping
// (slot = table[p // B] * B + p % B, engine/block_manager.py:118-123), slot // B, slot % B, the -1 padded int32
// block tables cut to ceil(context / B) blocks per sequence, context lengths (start + n) and the row of each
// sequence's last new token. Here the tables live on the device, one row per live sequence (kept current by the
// host from the block manager's changes), and one launch derives all of it for the forward.
#include "sipa_common.h"

namespace sipa {

struct MetaArgs {
  const int32_t* tables;  // [table_rows, table_stride] persistent block tables
  int64_t table_stride;
  int32_t table_rows, table_width;
  const int32_t* rows;    // [S] table row of each sequence
  const int32_t* starts;  // [S] position of each sequence's first new token
  const int32_t* qs;      // [S + 1] query starts
  int32_t S, T, B, W;     // sequences, tokens, block size, output table width
  int64_t* positions;     // [T]
  int64_t* slots;         // [T]
  int64_t* slot_blocks;   // [T]
  int64_t* slot_offsets;  // [T]
  int64_t* last_rows;     // [S]
  int32_t* bt;            // [S, W]
  int32_t* ctx;           // [S]
};

__device__ __forceinline__ int table_entry(const MetaArgs& a, int row, int col) {
  row = min(max(row, 0), a.table_rows - 1);
  col = min(max(col, 0), a.table_width - 1);
  return a.tables[(int64_t)row * a.table_stride + col];
}

// Threads [0, T): one token each; threads [T, T + S W): one entry of the packed tables each (the first column's
// thread also writes the sequence's context length and last row).
__global__ void __launch_bounds__(256) paged_metadata_kernel(const MetaArgs a) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < a.T) {
    const int t = (int)i;
    int lo = 0, hi = a.S;  // the sequence s with qs[s] <= t < qs[s + 1]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (a.qs[mid] <= t) lo = mid; else hi = mid;
    }
    const int s = lo;
    const int64_t p = (int64_t)a.starts[s] + (t - a.qs[s]);
    const int64_t blk = table_entry(a, a.rows[s], (int)(p / a.B));
    const int64_t slot = blk * a.B + p % a.B;
    a.positions[t] = p;
    a.slots[t] = slot;
    a.slot_blocks[t] = blk;
    a.slot_offsets[t] = p % a.B;
    return;
  }
  const int64_t j = i - a.T;
  if (j >= (int64_t)a.S * a.W) return;
  const int s = (int)(j / a.W), c = (int)(j % a.W);
  const int ctx = a.starts[s] + (a.qs[s + 1] - a.qs[s]);
  const int nb = (ctx + a.B - 1) / a.B;
  a.bt[(int64_t)s * a.W + c] = c < nb ? table_entry(a, a.rows[s], c) : -1;
  if (c == 0) {
    a.ctx[s] = ctx;
    a.last_rows[s] = a.qs[s + 1] - 1;
  }
}

}  // namespace sipa

using namespace sipa;

extern "C" int32_t sipa_paged_metadata(const int32_t* tables, int64_t table_stride, int32_t table_rows,
                                       int32_t table_width, const int32_t* seq_info, int32_t num_seqs,
                                       int32_t num_tokens, int32_t block_size, int32_t out_width,
                                       int64_t* positions, int64_t* slots, int64_t* slot_blocks,
                                       int64_t* slot_offsets, int64_t* last_rows, int32_t* block_tables,
                                       int32_t* context_lens, void* stream) {
  SIPA_CHECK(num_seqs > 0 && num_tokens >= num_seqs, SIPA_EINVAL, "%d sequences, %d tokens", num_seqs, num_tokens);
  SIPA_CHECK(block_size > 0 && out_width > 0 && table_rows > 0 && table_width > 0 && table_stride >= table_width,
             SIPA_EINVAL, "bad table or block sizes");
  SIPA_CHECK(tables && seq_info && positions && slots && slot_blocks && slot_offsets && last_rows && block_tables &&
                 context_lens, SIPA_EINVAL, "NULL pointer");
  MetaArgs a;
  a.tables = tables;
  a.table_stride = table_stride;
  a.table_rows = table_rows;
  a.table_width = table_width;
  a.rows = seq_info;
  a.starts = seq_info + num_seqs;
  a.qs = seq_info + 2 * num_seqs;
  a.S = num_seqs;
  a.T = num_tokens;
  a.B = block_size;
  a.W = out_width;
  a.positions = positions;
  a.slots = slots;
  a.slot_blocks = slot_blocks;
  a.slot_offsets = slot_offsets;
  a.last_rows = last_rows;
  a.bt = block_tables;
  a.ctx = context_lens;
  const int64_t threads = (int64_t)num_tokens + (int64_t)num_seqs * out_width;
  const int64_t grid = (threads + 255) / 256;
  SIPA_CHECK(grid <= 0x7fffffff, SIPA_EINVAL, "metadata grid too large");
  hipLaunchKernelGGL(paged_metadata_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SIPA_EHIP, "metadata launch failed: %s", hipGetErrorString(e));
  return SIPA_OK;
}
