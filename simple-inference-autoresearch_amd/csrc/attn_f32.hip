// Float32 attention kernels (layout and semantics: attn_f32.hpp).
#include "attn_f32.hpp"
#include "host_util.hpp"

namespace sia {

// Four consecutive elements at p as fp32.
template <class T>
__device__ __forceinline__ f32x4 load4(const char* p);
template <>
__device__ __forceinline__ f32x4 load4<F32>(const char* p) {
  return __builtin_nontemporal_load((const f32x4*)p);
}
template <>
__device__ __forceinline__ f32x4 load4<F16>(const char* p) {
  const u32x2 w = __builtin_nontemporal_load((const u32x2*)p);
  return f32x4{lo_f32(F16{}, w[0]), hi_f32(F16{}, w[0]), lo_f32(F16{}, w[1]), hi_f32(F16{}, w[1])};
}
template <>
__device__ __forceinline__ f32x4 load4<BF16>(const char* p) {
  const u32x2 w = __builtin_nontemporal_load((const u32x2*)p);
  return f32x4{lo_f32(BF16{}, w[0]), hi_f32(BF16{}, w[0]), lo_f32(BF16{}, w[1]), hi_f32(BF16{}, w[1])};
}
template <>
__device__ __forceinline__ f32x4 load4<I8>(const char* p) {
  const uint32_t w = __builtin_nontemporal_load((const uint32_t*)p);
  return f32x4{(float)(int8_t)(w & 0xffu), (float)(int8_t)((w >> 8) & 0xffu), (float)(int8_t)((w >> 16) & 0xffu),
               (float)(int8_t)(w >> 24)};
}

template <class T>
__device__ __forceinline__ float scale_at(const char* p) {
  if constexpr (std::is_same<T, F32>::value) return *(const float*)p;
  else return (float)*(const _Float16*)p;
}

// Four outputs (fp32) stored as T at p.
__device__ __forceinline__ void store4(F32, char* p, f32x4 x) { *(f32x4*)p = x; }
__device__ __forceinline__ void store4(F16, char* p, f32x4 x) {
  *(u32x2*)p = u32x2{pack2(F16{}, x[0], x[1]), pack2(F16{}, x[2], x[3])};
}
__device__ __forceinline__ void store4(BF16, char* p, f32x4 x) {
  *(u32x2*)p = u32x2{pack2(BF16{}, x[0], x[1]), pack2(BF16{}, x[2], x[3])};
}

// 2^(x - mu) with mu = 0 standing in for a max of -inf (nothing seen yet).
__device__ __forceinline__ float exp2_from(float x, float mu) { return fast_exp2(x - mu); }

// Merge state (mb, lb, ab) into (m, l, acc): the larger max wins and each
// side is weighted by 2^(its max - the new max); an empty side (max -inf)
// weighs 0.
__device__ __forceinline__ void merge_state(float& m, float& l, f32x4& acc, float mb, float lb, f32x4 ab) {
  const float M = fmaxf(m, mb);
  const float mu = M == -INFINITY ? 0.f : M;
  const float wa = exp2_from(m, mu), wb = exp2_from(mb, mu);
  l = l * wa + lb * wb;
  acc = acc * wa + ab * wb;
  m = M;
}

template <int D, class QT, class KV, class ST>
__global__ __launch_bounds__(256) void attn_f32(const F32Args a) {
  constexpr int LPT = D / 4;            // lanes per key row
  constexpr int TPW = 64 / LPT;         // key rows per wave per load
  constexpr int U = kF32Unroll;
  constexpr int C = kF32Cols;
  constexpr int STEP = 4 * TPW * U;     // keys per work-group step
  constexpr bool kInt8 = std::is_same<KV, I8>::value;
  __shared__ __attribute__((aligned(16))) float sm[4][C][D + 4];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane / LPT, j4 = lane % LPT;
  int item = blockIdx.x;
  const int s = item % a.nsplit;
  item /= a.nsplit;
  const int chunk = item % a.nchunk;
  item /= a.nchunk;
  const int hkv = item % a.Hkv;
  const int b = item / a.Hkv;

  // columns of this item: keys visible to each, and the query slice
  int n_all = a.cap;
  if (a.kv_len != nullptr) {
    const int n = a.kv_len[a.kv_per_seq ? b : 0];
    n_all = n < 0 ? 0 : (n > a.cap ? a.cap : n);
  }
  int lim[C];
  f32x4 q[C];
  int nmax = 0;
#pragma unroll
  for (int c = 0; c < C; ++c) {
    const int col = chunk * C + c;
    const bool live = col < a.ncol;
    const int i = live ? col / a.G : 0;
    const int g = live ? col - i * a.G : 0;
    int n = live ? n_all : 0;
    if (a.causal) n = min(n, a.Tk - a.Tq + i + 1);
    lim[c] = n > 0 ? n : 0;
    nmax = max(nmax, lim[c]);
    const char* qp = a.q + b * a.q_sb + (int64_t)(hkv * a.G + g) * a.q_sh + (int64_t)i * a.q_sm +
                     j4 * 4 * QT::bytes;
    q[c] = live ? load4<QT>(qp) : f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const int lo = s * a.tps;
  const int hi = min(nmax, lo + a.tps);
  const int ncl = min(C, a.ncol - chunk * C);          // live columns (uniform)

  float m[C], l[C];
  f32x4 acc[C];
#pragma unroll
  for (int c = 0; c < C; ++c) {
    m[c] = -INFINITY;
    l[c] = 0.f;
    acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const bool paged = a.bt != nullptr;
  const int64_t seq_k = paged ? 0 : (int64_t)b * a.k_s0, seq_v = paged ? 0 : (int64_t)b * a.v_s0;
  const char* kb = a.k + seq_k + (int64_t)hkv * a.k_sh + j4 * 4 * KV::bytes;
  const char* vb = a.v + seq_v + (int64_t)hkv * a.v_sh + j4 * 4 * KV::bytes;
  const char* ksb = nullptr;
  const char* vsb = nullptr;
  if constexpr (kInt8) {
    ksb = a.ks + (paged ? 0 : (int64_t)b * a.ks_s0) + (int64_t)hkv * a.ks_sh;
    vsb = a.vs + (paged ? 0 : (int64_t)b * a.vs_s0) + (int64_t)hkv * a.vs_sh;
  }
  const int32_t* btrow = paged ? a.bt + (int64_t)b * a.bt_sb : nullptr;

  for (int t0 = lo + wave * TPW * U; t0 < hi; t0 += STEP) {
    f32x4 kk[U], vv[U];
    float ksc[U], vsc[U];
    int tt[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int t = t0 + u * TPW + r;
      tt[u] = t;
      const int tc = t < hi ? t : lo;                       // rows past the range reread a live one
      int64_t page = 0;
      int pos = tc;
      if (paged) {
        const int pg = btrow[(int64_t)(tc / a.page_size) * a.bt_sl];
        page = (unsigned)pg < (unsigned long long)a.num_pages ? pg : 0;   // never read outside the pool
        pos = tc - (tc / a.page_size) * a.page_size;
      }
      kk[u] = load4<KV>(kb + page * a.k_s0 + (int64_t)pos * a.k_sn);
      vv[u] = load4<KV>(vb + page * a.v_s0 + (int64_t)pos * a.v_sn);
      if constexpr (kInt8) {
        ksc[u] = scale_at<ST>(ksb + page * a.ks_s0 + (int64_t)pos * a.ks_sn);
        vsc[u] = scale_at<ST>(vsb + page * a.vs_s0 + (int64_t)pos * a.vs_sn);
      } else {
        ksc[u] = 1.0f;
        vsc[u] = 1.0f;
      }
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
      if (c >= ncl) break;
      float sc[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float d = q[c][0] * kk[u][0];
        d = __builtin_fmaf(q[c][1], kk[u][1], d);
        d = __builtin_fmaf(q[c][2], kk[u][2], d);
        d = __builtin_fmaf(q[c][3], kk[u][3], d);
#pragma unroll
        for (int o = LPT / 2; o > 0; o >>= 1) d += __shfl_xor(d, o);
        if constexpr (kInt8) d *= ksc[u];
        d *= a.qk_scale;
        sc[u] = tt[u] < hi && tt[u] < lim[c] ? d : -INFINITY;
      }
      float smax = sc[0];
#pragma unroll
      for (int u = 1; u < U; ++u) smax = fmaxf(smax, sc[u]);
      const float M = fmaxf(m[c], smax);
      const float mu = M == -INFINITY ? 0.f : M;
      const float alpha = exp2_from(m[c], mu);
      float psum = 0.f;
      f32x4 pv = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float p = exp2_from(sc[u], mu);
        psum += p;
        pv += (p * vsc[u]) * vv[u];
      }
      l[c] = l[c] * alpha + psum;
      acc[c] = acc[c] * alpha + pv;
      m[c] = M;
    }
  }

  // merge the lane groups of the wave (lanes LPT apart hold the same dims)
#pragma unroll
  for (int o = LPT; o < 64; o <<= 1) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      const float mb = __shfl_xor(m[c], o), lb = __shfl_xor(l[c], o);
      const f32x4 ab = {__shfl_xor(acc[c][0], o), __shfl_xor(acc[c][1], o), __shfl_xor(acc[c][2], o),
                        __shfl_xor(acc[c][3], o)};
      merge_state(m[c], l[c], acc[c], mb, lb, ab);
    }
  }
  if (r == 0) {
#pragma unroll
    for (int c = 0; c < C; ++c) {
      *(f32x4*)&sm[wave][c][4 * j4] = acc[c];
      if (j4 == 0) {
        sm[wave][c][D] = m[c];
        sm[wave][c][D + 1] = l[c];
      }
    }
  }
  __syncthreads();
  // the waves' states: thread (c, j4) of the group finishes column c
  for (int idx = threadIdx.x; idx < C * LPT; idx += 256) {
    const int c = idx / LPT, jj = idx - c * LPT;
    const int col = chunk * C + c;
    if (col >= a.ncol) continue;
    float M = sm[0][c][D], L = sm[0][c][D + 1];
    f32x4 A = *(const f32x4*)&sm[0][c][4 * jj];
#pragma unroll
    for (int w = 1; w < 4; ++w) merge_state(M, L, A, sm[w][c][D], sm[w][c][D + 1], *(const f32x4*)&sm[w][c][4 * jj]);
    const int i = col / a.G, g = col - i * a.G;
    const int hq = hkv * a.G + g;
    if (a.nsplit == 1) {
      const float inv = L == 0.f ? 0.f : 1.0f / L;     // no visible key: zeros (the reference's l_safe guard)
      char* op = a.out + b * a.o_sb + (int64_t)hq * a.o_sh + (int64_t)i * a.o_sm + jj * 4 * QT::bytes;
      store4(QT{}, op, A * inv);
    } else {
      const int64_t row = ((int64_t)b * a.Hq + hq) * a.Tq + i;
      float* dst = a.part + (row * a.nsplit + s) * (D + 4);
      *(f32x4*)(dst + 4 * jj) = A;
      if (jj == 0) {
        dst[D] = M;
        dst[D + 1] = L;
      }
    }
  }
}

// Combine the nsplit partials of each output row: D/4 lanes per row.
template <int D, class OT>
__global__ __launch_bounds__(256) void attn_f32_merge(const F32Args a) {
  constexpr int LPT = D / 4, RPW = 64 / LPT;
  const int lane = threadIdx.x & 63;
  const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / LPT;
  const int jj = lane % LPT;
  if (row >= (int64_t)a.B * a.Hq * a.Tq) return;
  const float* p = a.part + row * a.nsplit * (D + 4);
  float M = -INFINITY;
  for (int s = 0; s < a.nsplit; ++s) M = fmaxf(M, p[s * (D + 4) + D]);
  float L = 0.f;
  f32x4 A = {0.f, 0.f, 0.f, 0.f};
  if (M != -INFINITY) {
    for (int s = 0; s < a.nsplit; ++s) {
      const float ms = p[s * (D + 4) + D];
      const float w = ms == -INFINITY ? 0.f : fast_exp2(ms - M);
      L += w * p[s * (D + 4) + D + 1];
      A += w * *(const f32x4*)(p + s * (D + 4) + 4 * jj);
    }
  }
  const int i = (int)(row % a.Tq);
  const int64_t bh = row / a.Tq;
  const int hq = (int)(bh % a.Hq);
  const int b = (int)(bh / a.Hq);
  const float inv = L == 0.f ? 0.f : 1.0f / L;
  store4(OT{}, a.out + b * a.o_sb + (int64_t)hq * a.o_sh + (int64_t)i * a.o_sm + jj * 4 * OT::bytes, A * inv);
}

template <int D, class QT, class KV, class ST>
static int launch_f32_typed(F32Launch& L) {
  const F32Args& a = L.a;
  const int64_t items = (int64_t)a.B * a.Hkv * a.nchunk * a.nsplit;
  if (items > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "fp32 attention: too many work items");
  if (items == 0) {   // nothing to launch: the events mark an empty interval
    if ((L.begin_event && hipEventRecord(L.begin_event, L.stream) != hipSuccess) ||
        (L.end_event && hipEventRecord(L.end_event, L.stream) != hipSuccess))
      return fail(SIA_ERR_LAUNCH, "cannot record the main kernel's events");
  } else {
    const int rc = launch_kernel(attn_f32<D, QT, KV, ST>, dim3((unsigned)items), dim3(256), 0, L.stream,
                                 L.begin_event, L.end_event, "fp32 attention", a);
    if (rc != SIA_OK) return rc;
  }
  if (a.nsplit > 1) {
    constexpr int RPB = 4 * (64 / (D / 4));
    const int64_t rows = (int64_t)a.B * a.Hq * a.Tq;
    const int64_t blocks = (rows + RPB - 1) / RPB;
    if (blocks > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "fp32 attention: too many rows");
    hipLaunchKernelGGL((attn_f32_merge<D, QT>), dim3((unsigned)blocks), dim3(256), 0, L.stream, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(SIA_ERR_LAUNCH, "fp32 attention merge launch: %s", hipGetErrorString(e));
  }
  return SIA_OK;
}

template <class QT, class KV, class ST>
static int launch_f32_d(F32Launch& L) {
  switch (L.D) {
    case 16: return launch_f32_typed<16, QT, KV, ST>(L);
    case 32: return launch_f32_typed<32, QT, KV, ST>(L);
    case 64: return launch_f32_typed<64, QT, KV, ST>(L);
    case 128: return launch_f32_typed<128, QT, KV, ST>(L);
    case 256: return launch_f32_typed<256, QT, KV, ST>(L);
    default: return fail(SIA_ERR_UNSUPPORTED, "head_dim %d not supported (16, 32, 64, 128, 256)", L.D);
  }
}

template <int D>
static int launch_merge_d(const F32Args& a, int out_dtype, hipStream_t st) {
  constexpr int RPB = 4 * (64 / (D / 4));
  const int64_t rows = (int64_t)a.B * a.Hq * a.Tq;
  const int64_t blocks = (rows + RPB - 1) / RPB;
  if (blocks > 0x7fffffff) return fail(SIA_ERR_UNSUPPORTED, "split-K merge: too many rows");
  if (blocks == 0) return SIA_OK;
  if (out_dtype == SIA_F16) hipLaunchKernelGGL((attn_f32_merge<D, F16>), dim3((unsigned)blocks), dim3(256), 0, st, a);
  else if (out_dtype == SIA_BF16) hipLaunchKernelGGL((attn_f32_merge<D, BF16>), dim3((unsigned)blocks), dim3(256), 0, st, a);
  else hipLaunchKernelGGL((attn_f32_merge<D, F32>), dim3((unsigned)blocks), dim3(256), 0, st, a);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? SIA_OK : fail(SIA_ERR_LAUNCH, "split-K merge launch: %s", hipGetErrorString(e));
}

int launch_attn_merge(const F32Args& a, int D, int out_dtype, hipStream_t stream) {
  switch (D) {
    case 16: return launch_merge_d<16>(a, out_dtype, stream);
    case 32: return launch_merge_d<32>(a, out_dtype, stream);
    case 64: return launch_merge_d<64>(a, out_dtype, stream);
    case 128: return launch_merge_d<128>(a, out_dtype, stream);
    case 256: return launch_merge_d<256>(a, out_dtype, stream);
    default: return fail(SIA_ERR_UNSUPPORTED, "head_dim %d not supported (16, 32, 64, 128, 256)", D);
  }
}

int launch_attn_f32(F32Launch& L) {
  if (L.q_dtype == SIA_F32) {
    switch (L.kv_dtype) {
      case SIA_F32: return launch_f32_d<F32, F32, F32>(L);
      case SIA_F16: return launch_f32_d<F32, F16, F32>(L);
      case SIA_BF16: return launch_f32_d<F32, BF16, F32>(L);
      case SIA_I8:
        return L.scale_dtype == SIA_F16 ? launch_f32_d<F32, I8, F16>(L) : launch_f32_d<F32, I8, F32>(L);
      default: break;
    }
  } else if (L.kv_dtype == SIA_F32) {
    if (L.q_dtype == SIA_F16) return launch_f32_d<F16, F32, F32>(L);
    if (L.q_dtype == SIA_BF16) return launch_f32_d<BF16, F32, F32>(L);
  } else {
    // 16-bit q over a paged pool whose pages are not whole 16-token tiles
    // (page sizes 1-8 and the like): 16-bit or int8 K/V
    const bool h = L.q_dtype == SIA_F16;
    if (L.q_dtype != SIA_F16 && L.q_dtype != SIA_BF16) return fail(SIA_ERR_UNSUPPORTED, "q dtype not supported");
    switch (L.kv_dtype) {
      case SIA_F16: return h ? launch_f32_d<F16, F16, F32>(L) : launch_f32_d<BF16, F16, F32>(L);
      case SIA_BF16: return h ? launch_f32_d<F16, BF16, F32>(L) : launch_f32_d<BF16, BF16, F32>(L);
      case SIA_I8:
        if (L.scale_dtype == SIA_F16) return h ? launch_f32_d<F16, I8, F16>(L) : launch_f32_d<BF16, I8, F16>(L);
        return h ? launch_f32_d<F16, I8, F32>(L) : launch_f32_d<BF16, I8, F32>(L);
      default: break;
    }
  }
  return fail(SIA_ERR_UNSUPPORTED, "fp32 attention: q %s with K/V %s not supported", dtype_name(L.q_dtype),
              dtype_name(L.kv_dtype));
}

}  // namespace sia
