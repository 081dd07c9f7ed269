// Depthwise causal short convolution over [shared prefix taps || beam suffix].
//
// Replaces src/kadllm/ops.py:166-226 and src/kadllm/kernels/causal_conv1d.py:10-78.
// HBM-bound: each output element reads its input once; the request-sized
// prefix taps (state[b, c, history-3 ..]) and the weights are read by every
// beam of the request and stay in L2.  Rounding follows the reference torch
// path: the convolution result is rounded to the tensor dtype, then SiLU is
// applied and rounded again (for fp32 both roundings are exact).  The bf16
// kernels (decode and prefill) take SiLU with the hardware reciprocal
// (silu_fast: they are VALU-bound and the result is rounded to bf16); fp16 and
// fp32 tensors keep the IEEE exp and divide.
//
// Three paths: a vectorised one when channels are contiguous in x and out
// (8 channels per thread, 16-byte accesses; the [rows, T, C] layout produced by
// the projection GEMM), a vectorised one for the reference's contiguous
// [BW, C, T] layout (8 channels x T tokens per thread), and a scalar one for
// any other strides, widths and dtypes.

#include "kad_common.h"

namespace {

template <typename T>
__device__ __forceinline__ float ld(const T* p) { return Elem<T>::to_f(*p); }

// SiLU in the dtype's precision: the hardware reciprocal for bf16 outputs, the
// IEEE exp and divide (torch's silu) for fp16 and fp32
template <typename T>
__device__ __forceinline__ float silu_for(float x) {
  if constexpr (Elem<T>::code == KAD_DTYPE_BF16) return silu_fast(x);
  else return x / (1.0f + expf(-x));
}

template <typename T>
__global__ __launch_bounds__(256) void conv_suffix_scalar(
    const T* __restrict__ x, int64_t sx_n, int64_t sx_c, int64_t sx_t,
    const T* __restrict__ state, int64_t ss_b, int64_t ss_c, int64_t ss_t, int history,
    const T* __restrict__ w, int width, const T* __restrict__ bias, T* __restrict__ out,
    int64_t so_n, int64_t so_c, int64_t so_t, int W, int C, int T_, int64_t total, int silu) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int c = (int)(idx % C);
  const int64_t n = idx / C;
  const int64_t b = n / W;
  if (width > 4) {
    // wide kernels: each output reads its window straight from the prefix
    // taps and the suffix, taps in weight order as the width-4 path
    const float bv = bias ? ld(bias + c) : 0.f;
    for (int t = 0; t < T_; ++t) {
      float acc = bv;
      for (int i = 0; i < width; ++i) {
        const int p = t + i - (width - 1);  // < 0: prefix tap history + p
        const float xv = p < 0 ? ld(state + b * ss_b + (int64_t)c * ss_c + (int64_t)(history + p) * ss_t)
                               : ld(x + n * sx_n + (int64_t)c * sx_c + (int64_t)p * sx_t);
        acc += ld(w + (int64_t)c * width + i) * xv;
      }
      float y = round_to_dtype(acc, Elem<T>::code);
      if (silu) y = silu_for<T>(y);
      out[n * so_n + (int64_t)c * so_c + (int64_t)t * so_t] = Elem<T>::from_f(y);
    }
    return;
  }
  float win[4] = {0.f, 0.f, 0.f, 0.f};  // win[3] is the newest tap
  float wt[4] = {0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < width; ++i) wt[4 - width + i] = ld(w + (int64_t)c * width + i);
  for (int i = 0; i < width - 1; ++i)
    win[4 - (width - 1) + i] = ld(state + b * ss_b + (int64_t)c * ss_c +
                                  (int64_t)(history - (width - 1) + i) * ss_t);
  const float bv = bias ? ld(bias + c) : 0.f;
  for (int t = 0; t < T_; ++t) {
    win[0] = win[1];
    win[1] = win[2];
    win[2] = win[3];
    win[3] = ld(x + n * sx_n + (int64_t)c * sx_c + (int64_t)t * sx_t);
    float acc = bv;
#pragma unroll
    for (int i = 0; i < 4; ++i) acc += wt[i] * win[i];
    float y = round_to_dtype(acc, Elem<T>::code);
    if (silu) y = silu_for<T>(y);
    out[n * so_n + (int64_t)c * so_c + (int64_t)t * so_t] = Elem<T>::from_f(y);
  }
}

// 8 contiguous bf16 channels per thread, kConvBeams beams of one request per
// thread (the request's weights and prefix taps are loaded once); width 4
// (3 taps), any T.  Grid: x = request x beam group, y = channel groups of 256
// threads.  The next (beam, token) row is loaded before the current one is
// computed so that every thread keeps one 16-byte load in flight.
constexpr int kConvBeams = 8;

// TT > 0: the suffix length fixed at compile time (the search's one- to
// four-token suffixes), so the (beam, token) of each step needs no division
template <int TT>
__global__ __launch_bounds__(256) void conv_suffix_vec_bf16(
    const bf16_t* __restrict__ x, int64_t sx_n, int64_t sx_t, const bf16_t* __restrict__ state,
    int64_t ss_b, int64_t ss_c, int64_t ss_t, int history, const bf16_t* __restrict__ w,
    bf16_t* __restrict__ out, int64_t so_n, int64_t so_t, int W, int C, int T_rt, int nbg,
    int silu) {
  const int T_ = TT > 0 ? TT : T_rt;
  const int c8 = blockIdx.y * 256 + threadIdx.x;
  if (c8 >= C / 8) return;
  const int c0 = c8 * 8;
  const int b = blockIdx.x / nbg;
  const int j0 = (blockIdx.x % nbg) * kConvBeams;
  const int nj = min(W - j0, kConvBeams);
  float wt[8][4];
  {
    const u32x4* wp = (const u32x4*)(w + (int64_t)c0 * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4 r = wp[j];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int flat = j * 8 + e * 2;  // channel c0 + flat/4, tap flat%4
        wt[flat / 4][flat % 4] = __uint_as_float(r[e] << 16);
        wt[(flat + 1) / 4][(flat + 1) % 4] = __uint_as_float(r[e] & 0xffff0000u);
      }
    }
  }
  // prefix taps: the last 3 of the request's state, per channel
  float tap[8][3];
  const bf16_t* sb = state + (int64_t)b * ss_b;
  if (ss_t == 1 && ss_c == 4 && history == 4 && (((uintptr_t)sb) % 16) == 0) {
    const u32x4* sp = (const u32x4*)(sb + (int64_t)c0 * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4 r = sp[j];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int flat = j * 8 + e * 2;  // channel flat/4, slot flat%4 (slots 1..3 are taps)
        if (flat % 4 != 0) tap[flat / 4][flat % 4 - 1] = __uint_as_float(r[e] << 16);
        tap[(flat + 1) / 4][(flat + 1) % 4 - 1] = __uint_as_float(r[e] & 0xffff0000u);
      }
    }
  } else {
#pragma unroll
    for (int ch = 0; ch < 8; ++ch)
#pragma unroll
      for (int i = 0; i < 3; ++i)
        tap[ch][i] = bf2f(sb[(int64_t)(c0 + ch) * ss_c + (int64_t)(history - 3 + i) * ss_t]);
  }

  const int64_t n0 = (int64_t)b * W + j0;
  const int steps = nj * T_;
  auto row = [&](int k) {
    const int j = k / T_, t = k - (k / T_) * T_;
    return x + (n0 + j) * sx_n + (int64_t)t * sx_t + c0;
  };
  u32x4 next = *(const u32x4*)row(0);
  float win[8][4];
  for (int k = 0, t = 0; k < steps; ++k) {
    const u32x4 r = next;
    if (k + 1 < steps) next = *(const u32x4*)row(k + 1);
    if (t == 0) {
#pragma unroll
      for (int ch = 0; ch < 8; ++ch) {
        win[ch][1] = tap[ch][0];
        win[ch][2] = tap[ch][1];
        win[ch][3] = tap[ch][2];
      }
    }
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float xv[2] = {__uint_as_float(r[e] << 16), __uint_as_float(r[e] & 0xffff0000u)};
      float acc[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int ch = e * 2 + hh;
        win[ch][0] = win[ch][1];
        win[ch][1] = win[ch][2];
        win[ch][2] = win[ch][3];
        win[ch][3] = xv[hh];
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) s += wt[ch][i] * win[ch][i];
        acc[hh] = s;
      }
      // the pair's roundings as one packed conversion each (the same bits)
      uint32_t packed = pack_bf16x2(acc[0], acc[1]);
      if (silu)
        packed = pack_bf16x2(silu_fast(__uint_as_float(packed << 16)),
                             silu_fast(__uint_as_float(packed & 0xffff0000u)));
      o[e] = packed;
    }
    const int j = k / T_;
    *(u32x4*)(out + (n0 + j) * so_n + (int64_t)t * so_t + c0) = o;
    if (++t == T_) t = 0;
  }
}


// The reference's contiguous [BW, C, T] layout (each beam's block of C * T
// elements is one contiguous run, tokens fastest): 8 channels x TT tokens per
// thread are TT consecutive 16-byte words, so a beam streams through with
// vector loads and stores exactly as the token-major kernel does.  Same grid
// and arithmetic as conv_suffix_vec_bf16 (kConvBeams beams of one request per
// thread, the next beam's words loaded before the current one is computed).
template <int TT>
__global__ __launch_bounds__(256) void conv_suffix_ct_bf16(
    const bf16_t* __restrict__ x, int64_t sx_n, const bf16_t* __restrict__ state, int64_t ss_b,
    int64_t ss_c, int64_t ss_t, int history, const bf16_t* __restrict__ w,
    bf16_t* __restrict__ out, int64_t so_n, int W, int C, int nbg, int silu) {
  const int c8 = blockIdx.y * 256 + threadIdx.x;
  if (c8 >= C / 8) return;
  const int c0 = c8 * 8;
  const int b = blockIdx.x / nbg;
  const int j0 = (blockIdx.x % nbg) * kConvBeams;
  const int nj = min(W - j0, kConvBeams);
  float wt[8][4];
  {
    const u32x4* wp = (const u32x4*)(w + (int64_t)c0 * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4 r = wp[j];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int flat = j * 8 + e * 2;
        wt[flat / 4][flat % 4] = __uint_as_float(r[e] << 16);
        wt[(flat + 1) / 4][(flat + 1) % 4] = __uint_as_float(r[e] & 0xffff0000u);
      }
    }
  }
  float tap[8][3];
  const bf16_t* sb = state + (int64_t)b * ss_b;
#pragma unroll
  for (int ch = 0; ch < 8; ++ch)
#pragma unroll
    for (int i = 0; i < 3; ++i)
      tap[ch][i] = bf2f(sb[(int64_t)(c0 + ch) * ss_c + (int64_t)(history - 3 + i) * ss_t]);

  const int64_t n0 = (int64_t)b * W + j0;
  const int64_t off = (int64_t)c0 * TT;  // this thread's 8 * TT elements in a beam's block
  u32x4 next[TT];
#pragma unroll
  for (int k = 0; k < TT; ++k) next[k] = ((const u32x4*)(x + n0 * sx_n + off))[k];
  for (int j = 0; j < nj; ++j) {
    u32x4 cur[TT];
#pragma unroll
    for (int k = 0; k < TT; ++k) cur[k] = next[k];
    if (j + 1 < nj) {
#pragma unroll
      for (int k = 0; k < TT; ++k) next[k] = ((const u32x4*)(x + (n0 + j + 1) * sx_n + off))[k];
    }
    u32x4 o[TT];
#pragma unroll
    for (int k = 0; k < TT; ++k) o[k] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int ch = 0; ch < 8; ++ch) {
      float w0 = tap[ch][0], w1 = tap[ch][1], w2 = tap[ch][2];
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const int e = ch * TT + t;  // element index within the thread's run
        const uint32_t word = cur[e / 8][(e % 8) / 2];
        const float xv = __uint_as_float((e & 1) ? (word & 0xffff0000u) : (word << 16));
        float acc = 0.f;
        acc += wt[ch][0] * w0;
        acc += wt[ch][1] * w1;
        acc += wt[ch][2] * w2;
        acc += wt[ch][3] * xv;
        w0 = w1;
        w1 = w2;
        w2 = xv;
        float y = round_bf(acc);
        if (silu) y = silu_fast(y);
        o[e / 8][(e % 8) / 2] |= (uint32_t)f2bf(y) << (16 * (e & 1));
      }
    }
#pragma unroll
    for (int k = 0; k < TT; ++k) ((u32x4*)(out + (n0 + j) * so_n + off))[k] = o[k];
  }
}

// Prefill: causal width-4 conv + SiLU over whole prompts with zero history
// (transformers causal_conv1d_fn, modeling_qwen3_5.py:220-239), and the conv
// state the decode path reads: the last 4 pre-conv inputs of each sequence
// (cache_utils.py:1032-1070), zero-padded on the left for prompts shorter
// than 4.  Rows are tokens (row = b * L + t) with channels contiguous; each
// thread owns 8 channels of a run of kRun tokens and reads a 3-token halo.
constexpr int kRun = 16;

__global__ __launch_bounds__(256) void conv_prefill_bf16(
    const bf16_t* __restrict__ x, int64_t ldx, const bf16_t* __restrict__ w,
    bf16_t* __restrict__ out, int64_t ldo, bf16_t* __restrict__ state, int B, int L, int C,
    int silu) {
  const int C8 = C / 8;
  const int runs = (L + kRun - 1) / kRun;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)B * runs * C8) return;
  const int c0 = (int)(idx % C8) * 8;
  const int64_t br = idx / C8;
  const int run = (int)(br % runs);
  const int b = (int)(br / runs);
  const int t0 = run * kRun;
  float wt[8][4];
  {
    const u32x4* wp = (const u32x4*)(w + (int64_t)c0 * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      u32x4 r = wp[j];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int flat = j * 8 + e * 2;
        wt[flat / 4][flat % 4] = __uint_as_float(r[e] << 16);
        wt[(flat + 1) / 4][(flat + 1) % 4] = __uint_as_float(r[e] & 0xffff0000u);
      }
    }
  }
  float win[8][4];
#pragma unroll
  for (int ch = 0; ch < 8; ++ch) win[ch][0] = win[ch][1] = win[ch][2] = win[ch][3] = 0.f;
  // halo: tokens t0-3 .. t0-1 (zero before the sequence start)
  for (int h = 3; h >= 1; --h) {
    const int t = t0 - h;
    float xv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (t >= 0) {
      const u32x4 r = *(const u32x4*)(x + ((int64_t)b * L + t) * ldx + c0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xv[2 * e] = __uint_as_float(r[e] << 16);
        xv[2 * e + 1] = __uint_as_float(r[e] & 0xffff0000u);
      }
    }
#pragma unroll
    for (int ch = 0; ch < 8; ++ch) {
      win[ch][0] = win[ch][1];
      win[ch][1] = win[ch][2];
      win[ch][2] = win[ch][3];
      win[ch][3] = xv[ch];
    }
  }
  const int t_end = min(L, t0 + kRun);
  // the run's rows are all loaded before any is used (kRun loads in flight)
  u32x4 rows_in[kRun];
#pragma unroll
  for (int i = 0; i < kRun; ++i)
    rows_in[i] = *(const u32x4*)(x + ((int64_t)b * L + min(t0 + i, L - 1)) * ldx + c0);
#pragma unroll
  for (int i = 0; i < kRun; ++i) {
    const int t = t0 + i;
    if (t >= t_end) break;
    const u32x4 r = rows_in[i];
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float xv[2] = {__uint_as_float(r[e] << 16), __uint_as_float(r[e] & 0xffff0000u)};
      float acc[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int ch = e * 2 + hh;
        win[ch][0] = win[ch][1];
        win[ch][1] = win[ch][2];
        win[ch][2] = win[ch][3];
        win[ch][3] = xv[hh];
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) s += wt[ch][i] * win[ch][i];
        acc[hh] = s;
      }
      // the pair's bf16 roundings (the conv output, then the SiLU output) as
      // one packed conversion each; SiLU with the hardware reciprocal, as in
      // the decode conv kernels (within one bf16 ulp of torch's silu)
      uint32_t packed = pack_bf16x2(acc[0], acc[1]);
      if (silu)
        packed = pack_bf16x2(silu_fast(__uint_as_float(packed << 16)),
                             silu_fast(__uint_as_float(packed & 0xffff0000u)));
      o[e] = packed;
    }
    *(u32x4*)(out + ((int64_t)b * L + t) * ldo + c0) = o;
  }
  // conv state [B, C, 4]: inputs at positions L-4 .. L-1 (the run holding L-1 writes it)
  if (state && t_end == L) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int t = L - 4 + j;
#pragma unroll
      for (int ch = 0; ch < 8; ++ch) {
        const float v = t >= 0 ? bf2f(x[((int64_t)b * L + t) * ldx + c0 + ch]) : 0.f;
        state[((int64_t)b * C + c0 + ch) * 4 + j] = f2bf(v);
      }
    }
  }
}

template <typename T>
int launch_scalar(const void* x, int64_t sx_n, int64_t sx_c, int64_t sx_t, const void* state,
                  int64_t ss_b, int64_t ss_c, int64_t ss_t, int history, const void* w,
                  int width, const void* bias, void* out, int64_t so_n, int64_t so_c,
                  int64_t so_t, int B, int W, int C, int T_, int silu, hipStream_t s) {
  const int64_t total = (int64_t)B * W * C;
  hipLaunchKernelGGL((conv_suffix_scalar<T>), dim3((unsigned)kad_cdiv(total, 256)), dim3(256), 0,
                     s, (const T*)x, sx_n, sx_c, sx_t, (const T*)state, ss_b, ss_c, ss_t,
                     history, (const T*)w, width, (const T*)bias, (T*)out, so_n, so_c, so_t, W,
                     C, T_, total, silu);
  return kad_launch_status("conv_suffix_scalar");
}

}  // namespace

extern "C" int kad_causal_conv_suffix(const void* x, int64_t sx_n, int64_t sx_c, int64_t sx_t,
                                      const void* state, int64_t ss_b, int64_t ss_c,
                                      int64_t ss_t, int history, const void* weight, int width,
                                      const void* bias, void* out, int64_t so_n, int64_t so_c,
                                      int64_t so_t, int B, int W, int C, int T, int dtype,
                                      int activation_silu, kad_stream_t stream) {
  KAD_REQUIRE(x && state && weight && out, "null pointer argument");
  KAD_REQUIRE(B > 0 && W > 0 && C > 0 && T > 0 && width > 0, "dimensions must be positive");
  if (width > 64) KAD_UNSUPPORTED("causal conv supports width <= 64, got %d", width);
  KAD_REQUIRE(history >= width - 1, "state history %d shorter than width-1", history);
  KAD_REQUIRE((int64_t)B * W * C < ((int64_t)1 << 40), "problem too large");
  hipStream_t s = (hipStream_t)stream;
  const bool vec = dtype == KAD_DTYPE_BF16 && width == 4 && bias == nullptr && sx_c == 1 &&
                   so_c == 1 && C % 8 == 0 && sx_n % 8 == 0 && sx_t % 8 == 0 && so_n % 8 == 0 &&
                   so_t % 8 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)out % 16) == 0 &&
                   ((uintptr_t)weight % 16) == 0;
  if (vec) {
    const int nbg = (int)kad_cdiv(W, kConvBeams);
    KAD_REQUIRE((int64_t)B * nbg < 2147483647, "too many beams for the grid");
    const dim3 grid((unsigned)(B * nbg), (unsigned)kad_cdiv(C / 8, 256));
#define KAD_CONV_VEC(TTV)                                                                    \
  hipLaunchKernelGGL((conv_suffix_vec_bf16<TTV>), grid, dim3(256), 0, s, (const bf16_t*)x,   \
                     sx_n, sx_t, (const bf16_t*)state, ss_b, ss_c, ss_t, history,             \
                     (const bf16_t*)weight, (bf16_t*)out, so_n, so_t, W, C, T, nbg,           \
                     activation_silu)
    switch (T) {
      case 1: KAD_CONV_VEC(1); break;
      case 2: KAD_CONV_VEC(2); break;
      case 3: KAD_CONV_VEC(3); break;
      case 4: KAD_CONV_VEC(4); break;
      default: KAD_CONV_VEC(0); break;
    }
#undef KAD_CONV_VEC
    return kad_launch_status("conv_suffix_vec_bf16");
  }
  // [BW, C, T] with each beam's C * T block contiguous (the reference's layout)
  const bool ct = dtype == KAD_DTYPE_BF16 && width == 4 && bias == nullptr && T <= 4 &&
                  sx_t == 1 && sx_c == T && so_t == 1 && so_c == T && C % 8 == 0 &&
                  sx_n % 8 == 0 && so_n % 8 == 0 && ((uintptr_t)x % 16) == 0 &&
                  ((uintptr_t)out % 16) == 0 && ((uintptr_t)weight % 16) == 0;
  if (ct) {
    const int nbg = (int)kad_cdiv(W, kConvBeams);
    KAD_REQUIRE((int64_t)B * nbg < 2147483647, "too many beams for the grid");
    const dim3 grid((unsigned)(B * nbg), (unsigned)kad_cdiv(C / 8, 256));
#define KAD_CONV_CT(TTV)                                                                     \
  hipLaunchKernelGGL((conv_suffix_ct_bf16<TTV>), grid, dim3(256), 0, s, (const bf16_t*)x,    \
                     sx_n, (const bf16_t*)state, ss_b, ss_c, ss_t, history,                   \
                     (const bf16_t*)weight, (bf16_t*)out, so_n, W, C, nbg, activation_silu)
    switch (T) {
      case 1: KAD_CONV_CT(1); break;
      case 2: KAD_CONV_CT(2); break;
      case 3: KAD_CONV_CT(3); break;
      default: KAD_CONV_CT(4); break;
    }
#undef KAD_CONV_CT
    return kad_launch_status("conv_suffix_ct_bf16");
  }
  if (dtype == KAD_DTYPE_BF16)
    return launch_scalar<bf16_t>(x, sx_n, sx_c, sx_t, state, ss_b, ss_c, ss_t, history, weight,
                                 width, bias, out, so_n, so_c, so_t, B, W, C, T,
                                 activation_silu, s);
  if (dtype == KAD_DTYPE_F32)
    return launch_scalar<float>(x, sx_n, sx_c, sx_t, state, ss_b, ss_c, ss_t, history, weight,
                                width, bias, out, so_n, so_c, so_t, B, W, C, T, activation_silu,
                                s);
  if (dtype == KAD_DTYPE_F16)
    return launch_scalar<_Float16>(x, sx_n, sx_c, sx_t, state, ss_b, ss_c, ss_t, history, weight,
                                   width, bias, out, so_n, so_c, so_t, B, W, C, T,
                                   activation_silu, s);
  KAD_UNSUPPORTED("causal conv supports bf16, fp16 and fp32, got dtype %d", dtype);
}

extern "C" int kad_causal_conv_prefill(const void* x, int64_t ldx, const void* weight, void* out,
                                       int64_t ldo, void* state, int B, int L, int C,
                                       int activation_silu, kad_stream_t stream) {
  KAD_REQUIRE(x && weight && out, "null pointer argument");
  KAD_REQUIRE(B > 0 && L > 0 && C > 0 && C % 8 == 0, "bad dimensions (C %% 8 == 0 required)");
  KAD_REQUIRE(ldx % 8 == 0 && ldo % 8 == 0 && ((uintptr_t)x % 16) == 0 &&
                  ((uintptr_t)out % 16) == 0 && ((uintptr_t)weight % 16) == 0,
              "16-byte aligned rows required");
  const int runs = (L + kRun - 1) / kRun;
  const int64_t total = (int64_t)B * runs * (C / 8);
  hipLaunchKernelGGL(conv_prefill_bf16, dim3((unsigned)kad_cdiv(total, 256)), dim3(256), 0,
                     (hipStream_t)stream, (const bf16_t*)x, ldx, (const bf16_t*)weight,
                     (bf16_t*)out, ldo, (bf16_t*)state, B, L, C, activation_silu);
  return kad_launch_status("conv_prefill_bf16");
}
