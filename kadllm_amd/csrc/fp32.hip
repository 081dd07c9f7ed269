// fp32 model kernels (gfx950): the projections and row-wise layer ops of a
// Qwen3.5 model held in fp32.
//
// The reference adapter runs any float model (src/kadllm/adapters/qwen3_5.py
// wraps whatever dtype the transformers model has), and its fp32 runs are
// where it states its fixed-history accuracy (README.md:152).  The bf16 path
// of this library rounds where the transformers bf16 modules round; these
// kernels are the same layer math with no rounding at all, fp32 throughout:
//   kad_gemm_f32           C = A W^T on v_mfma_f32_16x16x4_f32 (exact fp32
//                          products, fp32 accumulation), store / residual /
//                          SwiGLU epilogues as kad_gemm_bf16
//   kad_rmsnorm_f32        x rsqrt(mean x^2 + eps) (w_offset + w)
//   kad_rmsnorm_gated_f32  w (x rsqrt(mean x^2 + eps)) silu(z) per head
//   kad_gdn_gates_f32      g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b)
//   kad_qk_norm_rope_f32   per-head RMSNorm(1 + w), then rotate-half RoPE on
//                          the first `rot` dims with fp32 cos/sin
//   kad_embedding_f32      row gather
// They serve small fp32 models (the reference's CPU-plumbing configuration);
// the bf16 kernels serve the headline model.

#include "kad_common.h"

namespace {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma16x16x4f32(float a, float b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// torch's fp32 silu and sigmoid: IEEE exp and divide
__device__ __forceinline__ float silu_exact(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float sigmoid_exact(float x) { return 1.0f / (1.0f + expf(-x)); }

// ---------------------------------------------------------------------------
// GEMM: 64 x 64 output tile per workgroup of 4 waves, each wave a 32 x 32
// block of four 16 x 16 MFMA tiles.  K moves in 16-deep slices through LDS
// (rows padded to 17 floats: the 16 lanes of an MFMA operand read 16 rows of
// one column, conflict free).  Operand layout of v_mfma_f32_16x16x4_f32:
// lane l holds A[l % 16][l / 16] and B[l / 16][l % 16]; the accumulator's
// element r of lane l is C[(l / 16) * 4 + r][l % 16].
constexpr int kBM = 64, kBN = 64, kBK = 16, kLd = kBK + 1, kCld = kBN + 1;

__global__ __launch_bounds__(256) void gemm_f32_kernel(
    const float* __restrict__ A, int64_t lda, const float* __restrict__ Wt, int64_t ldw,
    float* C, int64_t ldc, const float* R, int64_t ldr, int M, int N, int K, int epilogue) {
  __shared__ float As[kBM * kLd], Ws[kBN * kLd];
  __shared__ float Cs[kBM * kCld];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.y * kBM;
  const int n0 = blockIdx.x * kBN;
  f32x4_t acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < K; k0 += kBK) {
    // 64 x 16 of A and of W: 1024 elements each, 4 per thread, zero outside
    for (int e = tid; e < kBM * kBK; e += 256) {
      const int r = e / kBK, c = e % kBK;
      const int64_t gm = m0 + r;
      const int gk = k0 + c, gn = n0 + r;
      As[r * kLd + c] = (gm < M && gk < K) ? A[gm * lda + gk] : 0.f;
      Ws[r * kLd + c] = (gn < N && gk < K) ? Wt[(int64_t)gn * ldw + gk] : 0.f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 4) {
      const int k = kk + lane / 16;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float a = As[(wm * 32 + i * 16 + lane % 16) * kLd + k];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float b = Ws[(wn * 32 + j * 16 + lane % 16) * kLd + k];
          acc[i][j] = mfma16x16x4f32(a, b, acc[i][j]);
        }
      }
    }
    __syncthreads();
  }
  // stage the tile, then write it out row by row with the epilogue
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        Cs[(wm * 32 + i * 16 + (lane / 16) * 4 + r) * kCld + wn * 32 + j * 16 + lane % 16] =
            acc[i][j][r];
  __syncthreads();
  if (epilogue == KAD_EPI_SWIGLU) {
    // the tile's 64 columns are one [gate 32 | up 32] block of W rows
    const int oc0 = n0 / 2;
    for (int e = tid; e < kBM * 32; e += 256) {
      const int r = e / 32, c = e % 32;
      const int64_t gm = m0 + r;
      if (gm < M && n0 + c < N)
        C[gm * ldc + oc0 + c] = silu_exact(Cs[r * kCld + c]) * Cs[r * kCld + 32 + c];
    }
    return;
  }
  for (int e = tid; e < kBM * kBN; e += 256) {
    const int r = e / kBN, c = e % kBN;
    const int64_t gm = m0 + r;
    const int gn = n0 + c;
    if (gm < M && gn < N) {
      float v = Cs[r * kCld + c];
      if (epilogue == KAD_EPI_RESIDUAL) v += R[gm * ldr + gn];
      C[gm * ldc + gn] = v;
    }
  }
}

// ---------------------------------------------------------------------------
// Row-wise ops: one wave per row (or per head group), elements lane, lane+64, ...
__global__ __launch_bounds__(256) void rmsnorm_f32_kernel(const float* __restrict__ x,
                                                          int64_t ldx, const float* __restrict__ w,
                                                          float w_offset, float* __restrict__ y,
                                                          int64_t ldy, int64_t rows, int D,
                                                          float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const float* xr = x + row * ldx;
  float ss = 0.f;
  for (int d = lane; d < D; d += 64) ss += xr[d] * xr[d];
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)D + eps);
  for (int d = lane; d < D; d += 64) y[row * ldy + d] = (xr[d] * r) * (w_offset + w[d]);
}

__global__ __launch_bounds__(256) void rmsnorm_gated_f32_kernel(
    const float* __restrict__ x, int64_t ldx, const float* __restrict__ z, int64_t ldz,
    const float* __restrict__ w, float* __restrict__ y, int64_t ldy, int64_t groups, int heads,
    int D, float eps) {
  const int64_t g = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x & 63;
  if (g >= groups) return;
  const int64_t tok = g / heads;
  const int hh = (int)(g % heads);
  const float* xr = x + tok * ldx + (int64_t)hh * D;
  const float* zr = z + tok * ldz + (int64_t)hh * D;
  float ss = 0.f;
  for (int d = lane; d < D; d += 64) ss += xr[d] * xr[d];
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)D + eps);
  for (int d = lane; d < D; d += 64)
    y[tok * ldy + (int64_t)hh * D + d] = (w[d] * (xr[d] * r)) * silu_exact(zr[d]);
}

__global__ __launch_bounds__(256) void gdn_gates_f32_kernel(
    const float* __restrict__ a, int64_t lda, const float* __restrict__ b, int64_t ldb,
    const float* __restrict__ A_log, const float* __restrict__ dt_bias, float* __restrict__ g,
    float* __restrict__ beta, int64_t rows, int HV) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * HV) return;
  const int64_t r = idx / HV;
  const int h = (int)(idx % HV);
  g[idx] = -expf(A_log[h]) * softplus_f(a[r * lda + h] + dt_bias[h]);
  beta[idx] = sigmoid_exact(b[r * ldb + h]);
}

// one wave per (token, head); output layout as kad_qk_norm_rope
__global__ __launch_bounds__(256) void qk_norm_rope_f32_kernel(
    const float* __restrict__ src, int64_t ld_src, int64_t src_head_stride, int heads,
    const float* __restrict__ w, float* __restrict__ dst, int64_t period, int64_t s_b,
    int64_t s_t, int64_t s_h, int64_t rows, int D, int rot, const float* __restrict__ inv_freq,
    int64_t pos0, int64_t pos_period, float eps, int do_norm) {
  const int64_t gw = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x & 63;
  if (gw >= rows * heads) return;
  const int64_t tok = gw / heads;
  const int hh = (int)(gw % heads);
  const float* s = src + tok * ld_src + hh * src_head_stride;
  float ss = 0.f;
  for (int d = lane; d < D; d += 64) ss += s[d] * s[d];
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)D + eps);
  auto normed = [&](int d) { return do_norm ? (s[d] * r) * (1.0f + w[d]) : s[d]; };
  const int half = rot / 2;
  const float pos = (float)(pos0 + tok % pos_period);
  float* o = dst + (tok / period) * s_b + (tok % period) * s_t + hh * s_h;
  for (int d = lane; d < D; d += 64) {
    float v = normed(d);
    if (d < rot) {
      const float ang = pos * inv_freq[d % half];
      const int pd = d < half ? d + half : d - half;
      const float partner = normed(pd);
      v = v * cosf(ang) + (d < half ? -partner : partner) * sinf(ang);
    }
    o[d] = v;
  }
}

__global__ __launch_bounds__(256) void embedding_f32_kernel(const int64_t* __restrict__ ids,
                                                            const float* __restrict__ table,
                                                            float* __restrict__ out, int64_t rows,
                                                            int D, int64_t vocab) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * D) return;
  const int64_t r = idx / D;
  int64_t id = ids[r];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  out[idx] = table[id * D + idx % D];
}

__global__ __launch_bounds__(64) void selftest_f32(const float* a, const float* b, float* c) {
  const int l = threadIdx.x;
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  // A[16][4]: lane l holds A[l % 16][l / 16]; B[4][16]: lane l holds B[l / 16][l % 16]
  acc = mfma16x16x4f32(a[(l % 16) * 4 + l / 16], b[(l / 16) * 16 + l % 16], acc);
  for (int r = 0; r < 4; ++r) c[((l / 16) * 4 + r) * 16 + (l % 16)] = acc[r];
}

}  // namespace

extern "C" int kad_gemm_f32(const float* A, int64_t lda, const float* W, int64_t ldw, float* C,
                            int64_t ldc, const float* R, int64_t ldr, int M, int N, int K,
                            int epilogue, kad_stream_t stream) {
  KAD_REQUIRE(A && W && C, "null pointer argument");
  KAD_REQUIRE(M > 0 && N > 0 && K > 0, "bad dimensions");
  KAD_REQUIRE(epilogue == KAD_EPI_STORE || epilogue == KAD_EPI_RESIDUAL ||
                  epilogue == KAD_EPI_SWIGLU,
              "unknown epilogue %d", epilogue);
  KAD_REQUIRE(epilogue != KAD_EPI_RESIDUAL || R, "residual epilogue needs R");
  KAD_REQUIRE(epilogue != KAD_EPI_SWIGLU || N % 64 == 0, "SwiGLU needs N %% 64 == 0");
  KAD_REQUIRE(lda >= K && ldw >= K, "row strides too small");
  const int n_out = epilogue == KAD_EPI_SWIGLU ? N / 2 : N;
  KAD_REQUIRE(ldc >= n_out && (epilogue != KAD_EPI_RESIDUAL || ldr >= N), "row strides too small");
  dim3 grid((unsigned)kad_cdiv(N, kBN), (unsigned)kad_cdiv(M, kBM));
  KAD_REQUIRE(grid.y < 65536, "too many rows for one launch");
  hipLaunchKernelGGL(gemm_f32_kernel, grid, dim3(256), 0, (hipStream_t)stream, A, lda, W, ldw, C,
                     ldc, R, ldr, M, N, K, epilogue);
  return kad_launch_status("gemm_f32_kernel");
}

extern "C" int kad_rmsnorm_f32(const float* x, int64_t ldx, const float* w, float w_offset,
                               float* y, int64_t ldy, int64_t rows, int D, float eps,
                               kad_stream_t stream) {
  KAD_REQUIRE(x && w && y, "null pointer argument");
  KAD_REQUIRE(rows > 0 && D > 0 && ldx >= D && ldy >= D, "bad dimensions");
  hipLaunchKernelGGL(rmsnorm_f32_kernel, dim3((unsigned)kad_cdiv(rows, 4)), dim3(256), 0,
                     (hipStream_t)stream, x, ldx, w, w_offset, y, ldy, rows, D, eps);
  return kad_launch_status("rmsnorm_f32_kernel");
}

extern "C" int kad_rmsnorm_gated_f32(const float* x, int64_t ldx, const float* z, int64_t ldz,
                                     const float* w, float* y, int64_t ldy, int64_t rows,
                                     int heads, int D, float eps, kad_stream_t stream) {
  KAD_REQUIRE(x && z && w && y, "null pointer argument");
  KAD_REQUIRE(rows > 0 && heads > 0 && D > 0, "bad dimensions");
  const int64_t groups = rows * heads;
  hipLaunchKernelGGL(rmsnorm_gated_f32_kernel, dim3((unsigned)kad_cdiv(groups, 4)), dim3(256), 0,
                     (hipStream_t)stream, x, ldx, z, ldz, w, y, ldy, groups, heads, D, eps);
  return kad_launch_status("rmsnorm_gated_f32_kernel");
}

extern "C" int kad_gdn_gates_f32(const float* a, int64_t lda, const float* b, int64_t ldb,
                                 const float* A_log, const float* dt_bias, float* g, float* beta,
                                 int64_t rows, int HV, kad_stream_t stream) {
  KAD_REQUIRE(a && b && A_log && dt_bias && g && beta, "null pointer argument");
  KAD_REQUIRE(rows > 0 && HV > 0, "bad dimensions");
  hipLaunchKernelGGL(gdn_gates_f32_kernel, dim3((unsigned)kad_cdiv(rows * HV, 256)), dim3(256), 0,
                     (hipStream_t)stream, a, lda, b, ldb, A_log, dt_bias, g, beta, rows, HV);
  return kad_launch_status("gdn_gates_f32_kernel");
}

extern "C" int kad_qk_norm_rope_f32(const float* src, int64_t ld_src, int64_t src_head_stride,
                                    int heads, const float* w, float* dst, int64_t period,
                                    int64_t s_b, int64_t s_t, int64_t s_h, int64_t rows, int D,
                                    int rot, const float* inv_freq, int64_t pos0,
                                    int64_t pos_period, float eps, int do_norm,
                                    kad_stream_t stream) {
  KAD_REQUIRE(src && dst && inv_freq && (w || !do_norm), "null pointer argument");
  KAD_REQUIRE(rows > 0 && heads > 0 && D > 0, "bad dimensions");
  KAD_REQUIRE(rot >= 0 && rot <= D && rot % 2 == 0, "bad rotary dimension");
  KAD_REQUIRE(period > 0 && pos_period > 0, "bad periods");
  hipLaunchKernelGGL(qk_norm_rope_f32_kernel, dim3((unsigned)kad_cdiv(rows * heads, 4)),
                     dim3(256), 0, (hipStream_t)stream, src, ld_src, src_head_stride, heads, w,
                     dst, period, s_b, s_t, s_h, rows, D, rot, inv_freq, pos0, pos_period, eps,
                     do_norm);
  return kad_launch_status("qk_norm_rope_f32_kernel");
}

extern "C" int kad_embedding_f32(const int64_t* ids, const float* table, float* out,
                                 int64_t rows, int D, int64_t vocab, kad_stream_t stream) {
  KAD_REQUIRE(ids && table && out, "null pointer argument");
  KAD_REQUIRE(rows > 0 && D > 0 && vocab > 0, "bad dimensions");
  hipLaunchKernelGGL(embedding_f32_kernel, dim3((unsigned)kad_cdiv(rows * D, 256)), dim3(256), 0,
                     (hipStream_t)stream, ids, table, out, rows, D, vocab);
  return kad_launch_status("embedding_f32_kernel");
}

extern "C" int kad_selftest_mfma_f32(const float* a, const float* b, float* c,
                                     kad_stream_t stream) {
  KAD_REQUIRE(a && b && c, "null pointer argument");
  hipLaunchKernelGGL(selftest_f32, dim3(1), dim3(64), 0, (hipStream_t)stream, a, b, c);
  return kad_launch_status("selftest_f32");
}
