// Float32 attention on the vector ALUs: the path for calls whose q or K/V are
// float32 (decode and prefill).
//
// The reference wrappers accept any float dtype and return q's dtype
// (kernels/flash_decode_kernel.py:119-160, kernels/attention_kernel.py:235-305);
// its decode kernel computes in fp32 on vector lanes, tl.sum(q * k) and
// tl.sum(p * v) with an online softmax (kernels/flash_decode_kernel.py:85-114).
// The MFMA kernels of this library take 16-bit or int8 operands, so float32
// inputs run here instead, in fp32 end to end: products, sums, exponentials
// and the output (rounded to q's dtype).
//
// Layout (gfx950, wave64):
//  * A work item is one (sequence, KV head), up to kF32Cols "columns" -- the
//    (query row, query head) pairs of that KV head -- and one split of the
//    key range.  The K/V rows of the item are read once for all of its
//    columns (GQA: the G query heads of a KV head; prefill: several query
//    rows too).  Column (i, g) sees keys [0, n_i): n = kv_len (decode) or
//    Tk, and with the causal mask n_i = min(n, Tk - Tq + i + 1) (bottom-right,
//    kernels/attention_kernel.py:184-226); n_i <= 0 writes zeros.
//  * D/4 lanes share a key row, 4 dimensions each (16-byte fp32 loads; 8 or 4
//    bytes for 16-bit and int8 K/V), so one load instruction of a wave reads
//    64/(D/4) whole rows.  Each lane group runs an online softmax over its
//    own keys (kF32Unroll keys per step); the dot products are completed
//    with cross-lane sums inside the group.  Groups are merged with shuffles,
//    waves through LDS.
//  * Split-K: the key range is cut into nsplit pieces of tps keys; with more
//    than one piece each item writes (m, l, acc) and attn_f32_merge combines
//    them.  The split is chosen on the host from the cache capacity (lengths
//    stay on the device), so one captured graph serves every length.
#pragma once

#include "sia_common.hpp"

namespace sia {

constexpr int kF32Cols = 8;     // columns (query row, head) per work item
constexpr int kF32Unroll = 4;   // keys per lane group per step

struct F32Args {
  const char* q; int64_t q_sb, q_sh, q_sm;           // byte strides; head_dim contiguous
  char* out; int64_t o_sb, o_sh, o_sm;
  const char* k; int64_t k_s0, k_sh, k_sn;           // s0: batch (contiguous) or page (paged)
  const char* v; int64_t v_s0, v_sh, v_sn;
  const char* ks; int64_t ks_s0, ks_sh, ks_sn;       // int8 scales (nullptr otherwise)
  const char* vs; int64_t vs_s0, vs_sh, vs_sn;
  const int32_t* bt; int64_t bt_sb, bt_sl;           // block table (element strides), nullptr = contiguous
  int64_t num_pages;
  int32_t page_size;
  const int32_t* kv_len; int32_t kv_per_seq;         // nullptr: every column sees `cap` keys (prefill)
  int32_t cap;                                       // keys addressable: S, max_blocks * page_size, or Tk
  int32_t B, Hq, Hkv, G, Tq, Tk, causal;
  int32_t ncol;                                      // Tq * G columns per (sequence, KV head)
  int32_t nchunk;                                    // ceil(ncol / kF32Cols)
  int32_t nsplit, tps;                               // key-range split: nsplit pieces of tps keys
  float qk_scale;                                    // sm_scale * log2(e)
  float* part;                                       // nsplit > 1: [row][split][D + 4] (acc, m, l)
};

struct F32Launch {
  F32Args a;
  int D;
  int q_dtype;       // also the output dtype
  int kv_dtype;
  int scale_dtype;   // int8 K/V only
  hipStream_t stream;
  hipEvent_t begin_event;   // optional, recorded around the main kernel
  hipEvent_t end_event;
};

// Launches attn_f32 (and attn_f32_merge when nsplit > 1); implemented in attn_f32.hip.
int launch_attn_f32(F32Launch& L);

// attn_f32_merge alone, for split-K partials written in its layout by another
// kernel: head_dim D, output dtype out_dtype (f16 / bf16 / f32).
int launch_attn_merge(const F32Args& a, int D, int out_dtype, hipStream_t stream);

// Bytes of split-K partials for `rows` output rows, `nsplit` pieces, head_dim D.
inline size_t f32_partial_bytes(int64_t rows, int64_t nsplit, int D) {
  return (size_t)rows * (size_t)nsplit * (size_t)(D + 4) * 4;
}

}  // namespace sia
