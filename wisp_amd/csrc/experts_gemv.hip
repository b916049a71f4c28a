// Decode-shape expert kernels (GEMV): w13 with fused SiLU*mul, then w2 with
// the routing-order combine.
//
// Replaces vLLM fused_experts as called by the reference with the slot
// remap (src/wisp/integrations/vllm/fused_moe.py:1106-1118, 1155-1167):
//   act[t,k] = silu(W13[s][:I] x[t]) * (W13[s][I:] x[t]),   s = slots[t,k]
//   out[t]   = sum_{k=0..K-1} w[t,k] * (W2[s] act[t,k])     (k ascending)
//
// Both kernels stream weight rows with 16-byte loads, one wavefront (or half
// of one) per row, and reduce in a fixed butterfly order, so the bytes of
// out[t] depend only on x[t], the routing of token t and the weights read -
// never on the slot numbers, on cap or on the other tokens of the launch.
// That is what makes paged output byte-identical to resident output.
#include "common.h"

namespace wisp {
namespace {

template <typename T>
struct Vec;
template <>
struct Vec<float> {
  static constexpr int N = 4;
  __device__ static inline void unpack(const uint4& u, float* f) {
    f[0] = __uint_as_float(u.x); f[1] = __uint_as_float(u.y);
    f[2] = __uint_as_float(u.z); f[3] = __uint_as_float(u.w);
  }
};
template <>
struct Vec<uint16_t> {  // bf16 bits
  static constexpr int N = 8;
  __device__ static inline void unpack(const uint4& u, float* f) {
    f[0] = __uint_as_float(u.x << 16); f[1] = __uint_as_float(u.x & 0xffff0000u);
    f[2] = __uint_as_float(u.y << 16); f[3] = __uint_as_float(u.y & 0xffff0000u);
    f[4] = __uint_as_float(u.z << 16); f[5] = __uint_as_float(u.z & 0xffff0000u);
    f[6] = __uint_as_float(u.w << 16); f[7] = __uint_as_float(u.w & 0xffff0000u);
  }
};

template <typename T>
__device__ inline void store_elem(T* p, float v);
template <>
__device__ inline void store_elem<float>(float* p, float v) { *p = v; }
template <>
__device__ inline void store_elem<uint16_t>(uint16_t* p, float v) { *p = bf16_rne(v); }

__device__ inline uint4 ld16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// Streaming load for weight rows: each byte is read once per launch, so the
// nontemporal hint keeps the rows from displacing cached data (measured on
// MI355X: w13 at the Qwen3 decode shape 9.2 us instead of 10.2 us).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ inline uint4 ld16_stream(const void* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ---------------------------------------------------------------------------
// Kernel A: act = silu(gate) * up.  Block = 4 waves, each wave owns RW
// consecutive i (gate row i and up row I + i) of one (token, k) pair; each
// lane covers CH chunks of 16 bytes of a row (chunk c*64 + lane).
// grid = (ceil(I / (4 * RW)), T * K).  One row pair per wave (RW = 1) gives
// the most waves in flight, which is what a pure weight stream needs.  FULL:
// a row is exactly CH chunks per lane, so the loads carry no bounds guard
// (a guarded load sits in its own exec-masked block, which costs ~0.7 us per
// launch at the Qwen3 shape by keeping the loads from issuing back to back).
// ---------------------------------------------------------------------------
template <typename T, int CH, int RW, bool FULL>
__global__ __launch_bounds__(256) void w13_silu_kernel(const T* __restrict__ x, int H, int I,
                                                        int K, const int32_t* __restrict__ slots,
                                                        const T* __restrict__ w13,
                                                        size_t w13_stride, T* __restrict__ act,
                                                        const int32_t* __restrict__ pair_filter,
                                                        int want) {
  constexpr int V = Vec<T>::N;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int pair = blockIdx.y;
  if (pair_filter && pair_filter[pair] != want) return;
  const int t = pair / K;
  const int i0 = (blockIdx.x * 4 + wave) * RW;
  if (i0 >= I) return;
  const int s = slots[pair];
  T* arow = act + (size_t)pair * I;
  if (s < 0) {
    if (lane < RW && i0 + lane < I) store_elem(arow + i0 + lane, 0.f);
    return;
  }
  const int nch = H / V;
  const T* W = w13 + (size_t)s * w13_stride;
  const T* xr = x + (size_t)t * H;

  uint4 wg[RW][CH], wu[RW][CH], xv[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int ch = c * 64 + lane;
    xv[c] = (FULL || ch < nch) ? ld16(xr + (size_t)ch * V) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int i = min(i0 + r, I - 1);
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int ch = c * 64 + lane;
      if (FULL || ch < nch) {
        wg[r][c] = ld16_stream(W + (size_t)i * H + (size_t)ch * V);
        wu[r][c] = ld16_stream(W + (size_t)(I + i) * H + (size_t)ch * V);
      } else {
        wg[r][c] = make_uint4(0, 0, 0, 0);
        wu[r][c] = make_uint4(0, 0, 0, 0);
      }
    }
  }
  float ag[RW], au[RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) { ag[r] = 0.f; au[r] = 0.f; }
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    float xf[V];
    Vec<T>::unpack(xv[c], xf);
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      float gf[V], uf[V];
      Vec<T>::unpack(wg[r][c], gf);
      Vec<T>::unpack(wu[r][c], uf);
#pragma unroll
      for (int q = 0; q < V; ++q) {
        ag[r] = fmaf(gf[q], xf[q], ag[r]);
        au[r] = fmaf(uf[q], xf[q], au[r]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    for (int off = 32; off > 0; off >>= 1) {
      ag[r] += __shfl_xor(ag[r], off);
      au[r] += __shfl_xor(au[r], off);
    }
  }
#pragma unroll
  for (int r = 0; r < RW; ++r)
    if (lane == r && i0 + r < I) store_elem(arow + i0 + r, silu(ag[r]) * au[r]);
}

// ---------------------------------------------------------------------------
// Kernel B: out[t, h] = sum_k w[t,k] * dot(W2[s_k][h, :], act[t,k,:]).
// Block = K waves, wave k computes the dot products of expert k for the
// 64/LPR rows of this block (LPR lanes per row, CH chunks per lane, or a
// runtime chunk loop when CH == 0); the partials meet in LDS and one lane
// per row sums them in routing order, with the routing weights staged in
// LDS by the waves at the start (0 for an absent slot).
// grid = (ceil(H / (64 / LPR)), T).
// ---------------------------------------------------------------------------
constexpr int kMaxKw2 = kGemvMaxTopK;

template <typename T, int LPR, int CH, bool FULL>
__global__ __launch_bounds__(1024) void w2_combine_kernel(const T* __restrict__ act, int H, int I,
                                                           int K, const float* __restrict__ topk_w,
                                                           const int32_t* __restrict__ slots,
                                                           const T* __restrict__ w2,
                                                           size_t w2_stride,
                                                           T* __restrict__ out,
                                                           const int32_t* __restrict__ skip_if) {
  constexpr int V = Vec<T>::N;
  constexpr int RPW = 64 / LPR;
  __shared__ float part[kMaxKw2][RPW];
  __shared__ float wk[kMaxKw2];
  if (skip_if && *skip_if != 0) return;
  const int k = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int sub = lane / LPR, l = lane % LPR;
  const int t = blockIdx.y;
  const int h = blockIdx.x * RPW + sub;
  const int s = slots[t * K + k];
  if (lane == 0) wk[k] = s >= 0 ? topk_w[t * K + k] : 0.f;
  const int nch = I / V;
  float d = 0.f;
  if (s >= 0 && h < H) {
    const T* wrow = w2 + (size_t)s * w2_stride + (size_t)h * I;
    const T* arow = act + ((size_t)t * K + k) * I;
    if (CH > 0) {
      uint4 wv[CH > 0 ? CH : 1], av[CH > 0 ? CH : 1];
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int ch = c * LPR + l;
        if (FULL || ch < nch) {
          wv[c] = ld16(wrow + (size_t)ch * V);
          av[c] = ld16(arow + (size_t)ch * V);
        } else {
          wv[c] = make_uint4(0, 0, 0, 0);
          av[c] = make_uint4(0, 0, 0, 0);
        }
      }
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        float wf[V], af[V];
        Vec<T>::unpack(wv[c], wf);
        Vec<T>::unpack(av[c], af);
#pragma unroll
        for (int q = 0; q < V; ++q) d = fmaf(wf[q], af[q], d);
      }
    } else {
#pragma unroll 4
      for (int ch = l; ch < nch; ch += LPR) {
        float wf[V], af[V];
        Vec<T>::unpack(ld16(wrow + (size_t)ch * V), wf);
        Vec<T>::unpack(ld16(arow + (size_t)ch * V), af);
#pragma unroll
        for (int q = 0; q < V; ++q) d = fmaf(wf[q], af[q], d);
      }
    }
  }
  for (int off = LPR / 2; off > 0; off >>= 1) d += __shfl_xor(d, off);
  if (l == 0) part[k][sub] = d;
  __syncthreads();
  if (threadIdx.x < RPW) {
    const int r = threadIdx.x;
    const int hh = blockIdx.x * RPW + r;
    if (hh < H) {
      float acc = 0.f;
      for (int kk = 0; kk < K; ++kk) acc = fmaf(wk[kk], part[kk][r], acc);
      store_elem(out + (size_t)t * H + hh, acc);
    }
  }
}

// Optional controls of a launch: kernel timing events, the pair filter of
// the w13 kernel (run only pairs with pair_filter[p] == want) and the skip
// word of the w2 kernel (exit when *skip_if != 0).
struct LaunchCtl {
  hipEvent_t start = nullptr, stop = nullptr;
  const int32_t* pair_filter = nullptr;
  int want = 0;
  const int32_t* skip_if = nullptr;
};

template <typename T, int CH>
void launch_w13(const T* x, int T_, int H, int I, int K, const int32_t* slots, const T* w13,
                size_t w13_stride, T* act, hipStream_t st, const LaunchCtl& c) {
  constexpr int RW = 1;
  dim3 grid((I + 4 * RW - 1) / (4 * RW), T_ * K);
  if (H == CH * 64 * Vec<T>::N)
    launch_timed(w13_silu_kernel<T, CH, RW, true>, grid, dim3(256), st, c.start, c.stop, x, H, I,
                 K, slots, w13, w13_stride, act, c.pair_filter, c.want);
  else
    launch_timed(w13_silu_kernel<T, CH, RW, false>, grid, dim3(256), st, c.start, c.stop, x, H, I,
                 K, slots, w13, w13_stride, act, c.pair_filter, c.want);
}

template <typename T>
int dispatch_w13(const T* x, int T_, int H, int I, int K, const int32_t* slots, const T* w13,
                 size_t w13_stride, T* act, hipStream_t st, const LaunchCtl& c) {
  const int nch = H / Vec<T>::N;
  const int ch = (nch + 63) / 64;
  switch (ch) {
    case 1: launch_w13<T, 1>(x, T_, H, I, K, slots, w13, w13_stride, act, st, c); break;
    case 2: launch_w13<T, 2>(x, T_, H, I, K, slots, w13, w13_stride, act, st, c); break;
    case 3: launch_w13<T, 3>(x, T_, H, I, K, slots, w13, w13_stride, act, st, c); break;
    case 4: launch_w13<T, 4>(x, T_, H, I, K, slots, w13, w13_stride, act, st, c); break;
    case 5: case 6: launch_w13<T, 6>(x, T_, H, I, K, slots, w13, w13_stride, act, st, c); break;
    case 7: case 8: launch_w13<T, 8>(x, T_, H, I, K, slots, w13, w13_stride, act, st, c); break;
    default: return WISP_ERR_UNSUPPORTED;
  }
  return WISP_OK;
}

template <typename T, int LPR, int CH>
void launch_w2(const T* act, int T_, int H, int I, int K, const float* w, const int32_t* slots,
               const T* w2, size_t w2_stride, T* out, hipStream_t st, const LaunchCtl& c) {
  constexpr int RPW = 64 / LPR;
  dim3 grid((H + RPW - 1) / RPW, T_);
  if (CH > 0 && I == CH * LPR * Vec<T>::N)
    launch_timed(w2_combine_kernel<T, LPR, CH, true>, grid, dim3(64 * K), st, c.start, c.stop, act,
                 H, I, K, w, slots, w2, w2_stride, out, c.skip_if);
  else
    launch_timed(w2_combine_kernel<T, LPR, CH, false>, grid, dim3(64 * K), st, c.start, c.stop,
                 act, H, I, K, w, slots, w2, w2_stride, out, c.skip_if);
}

template <typename T>
int dispatch_w2(const T* act, int T_, int H, int I, int K, const float* w, const int32_t* slots,
                const T* w2, size_t w2_stride, T* out, hipStream_t st, const LaunchCtl& c) {
  if (K > kMaxKw2) return WISP_ERR_UNSUPPORTED;
  const int nch = I / Vec<T>::N;
  if (nch <= 32 * 4) {  // half a wave per row, up to 4 chunks per lane
    switch ((nch + 31) / 32) {
      case 1: launch_w2<T, 32, 1>(act, T_, H, I, K, w, slots, w2, w2_stride, out, st, c); break;
      case 2: launch_w2<T, 32, 2>(act, T_, H, I, K, w, slots, w2, w2_stride, out, st, c); break;
      case 3: launch_w2<T, 32, 3>(act, T_, H, I, K, w, slots, w2, w2_stride, out, st, c); break;
      default: launch_w2<T, 32, 4>(act, T_, H, I, K, w, slots, w2, w2_stride, out, st, c); break;
    }
  } else {
    launch_w2<T, 64, 0>(act, T_, H, I, K, w, slots, w2, w2_stride, out, st, c);
  }
  return WISP_OK;
}

}  // namespace

// Shapes the GEMV pair covers: the w13 kernel holds up to 8 chunks of 16
// bytes of a row per lane (H up to 4096 bf16 / 2048 fp32 elements), and the
// w2 kernel runs one wave per routed expert in a block of at most 16 waves.
bool gemv_supported(int dtype, int H, int K) {
  const int V = dtype == WISP_F32 ? 4 : 8;
  const int ch = (H / V + 63) / 64;
  return K >= 1 && K <= kMaxKw2 && ch >= 1 && ch <= 8;
}

int gemv_w13(const void* x, int dtype, int T_, int H, int I, int K, const int32_t* slots,
             const void* w13, size_t w13_stride, void* act, hipStream_t st,
             hipEvent_t ev_start, hipEvent_t ev_stop, const int32_t* pair_filter, int want) {
  if (T_ == 0) return WISP_OK;
  LaunchCtl c;
  c.start = ev_start;
  c.stop = ev_stop;
  c.pair_filter = pair_filter;
  c.want = want;
  const int rc = dtype == WISP_F32
      ? dispatch_w13<float>((const float*)x, T_, H, I, K, slots, (const float*)w13, w13_stride,
                            (float*)act, st, c)
      : dispatch_w13<uint16_t>((const uint16_t*)x, T_, H, I, K, slots, (const uint16_t*)w13,
                               w13_stride, (uint16_t*)act, st, c);
  if (rc != WISP_OK) {
    wisp_set_last_error("hidden size outside the GEMV kernels' coverage", "w13 kernel");
    return rc;
  }
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

int gemv_w2(const void* act, int dtype, int T_, int H, int I, int K, const float* topk_w,
            const int32_t* slots, const void* w2, size_t w2_stride, void* out, hipStream_t st,
            hipEvent_t ev_start, hipEvent_t ev_stop, const int32_t* skip_if) {
  if (T_ == 0) return WISP_OK;
  LaunchCtl c;
  c.start = ev_start;
  c.stop = ev_stop;
  c.skip_if = skip_if;
  const int rc = dtype == WISP_F32
      ? dispatch_w2<float>((const float*)act, T_, H, I, K, topk_w, slots, (const float*)w2,
                           w2_stride, (float*)out, st, c)
      : dispatch_w2<uint16_t>((const uint16_t*)act, T_, H, I, K, topk_w, slots,
                              (const uint16_t*)w2, w2_stride, (uint16_t*)out, st, c);
  if (rc != WISP_OK) {
    wisp_set_last_error("top_k above 16 is outside the GEMV kernels' coverage", "w2 kernel");
    return rc;
  }
  WISP_HIP_TRY(hipGetLastError());
  return WISP_OK;
}

int experts_gemv(const void* x, int dtype, int T_, int H, int I, int K, const float* topk_w,
                 const int32_t* slots, const void* w13, size_t w13_stride, const void* w2,
                 size_t w2_stride, void* act, void* out, hipStream_t st, const StageEvents* ev) {
  int rc = gemv_w13(x, dtype, T_, H, I, K, slots, w13, w13_stride, act, st,
                    ev ? ev->ev[0] : nullptr, ev ? ev->ev[1] : nullptr, nullptr, 0);
  if (rc != WISP_OK) return rc;
  return gemv_w2(act, dtype, T_, H, I, K, topk_w, slots, w2, w2_stride, out, st,
                 ev ? ev->ev[2] : nullptr, ev ? ev->ev[3] : nullptr, nullptr);
}

}  // namespace wisp
