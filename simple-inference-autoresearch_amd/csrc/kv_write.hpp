// Host/device description of one KV write (see kv_write.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sia {

struct KvWriteArgs {
  const char* src0; const char* src1;     // K and V sources (src1 unused when ntensors == 1)
  int64_t s_sb, s_sh, s_st;               // source byte strides (batch, head, token); head_dim contiguous
  char* dst0; char* dst1;                 // destinations: cache (B', H, S, D) or pool (pages, H, page, D)
  int64_t d_s0, d_sh, d_sn;               // destination byte strides
  char* sc0; char* sc1;                   // int8 scale destinations (same indexing without head_dim)
  int64_t c_s0, c_sh, c_sn;               // scale byte strides
  const int32_t* bt; int64_t bt_sb, bt_sl;   // block table (element strides); nullptr = contiguous cache
  int64_t num_pages;
  int32_t page;                           // tokens per page (paged)
  int32_t cap;                            // positions the destination holds (S, or max_blocks * page)
  const int32_t* start; int32_t start_per_seq; int32_t start_host;   // first position: start_host + start[b]
  int32_t B, H, T, D;
  int64_t rows;                           // B * H * T
  int32_t ntensors;
  int32_t scale_f32;
  float amax_floor;                       // 1e-8 rounded to the source dtype
  // rotary embedding of K (and q) on the way in; rope == 0 leaves the rows as they are
  int32_t rope;                           // 0 none, 1 split-half pairs (i, i + D/2), 2 interleaved (2i, 2i + 1)
  const char* cs; const char* sn;         // cos / sin tables (Tc, >= D/2), read at row `position`
  int64_t tab_rs;                         // table row stride (bytes)
  int32_t Tc, tab_dt;                     // table rows, table dtype code
  int32_t paged;                          // block table in use (bt valid otherwise too: a readable dummy)
  const char* q; char* qo;                // q (B, T, Hq, D) rotated into q_out; nullptr = no q
  int64_t q_sb, q_sh, q_st;               // q byte strides (batch, head, token)
  int64_t qo_sb, qo_sh, qo_st;            // q_out byte strides
  int32_t Hq;
  int64_t q_rows;                         // B * Hq * T
  uint32_t kv_blocks;                     // work-groups of the K/V part; the q part (one per token) follows
  int32_t log2_width;                     // log2(D / 8): lanes per row
  int32_t h_fast;                         // rows ordered (b, t, h) instead of (b, h, t)
};

int launch_kv_write(const KvWriteArgs& a, int src_dtype, int dst_dtype, hipStream_t stream);

}  // namespace sia
