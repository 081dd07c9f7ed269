// Row-wise kernels of the Qwen3.5 hybrid layer (bf16 activations).
//
// Each reproduces the bf16 rounding points of the transformers modules the
// reference decode calls (src/kadllm/adapters/qwen3_5.py:161-176,184-189,
// 216-226,234-235):
//   rmsnorm        Qwen3_5RMSNorm: y = bf16(x * rsqrt(mean x^2 + eps) * (1 + w))
//   rmsnorm_gated  Qwen3_5RMSNormGated: y = bf16(bf16(w * bf16(x r)) * silu(z)), SiLU
//                  with the hardware reciprocal (the kernel is VALU-bound)
//   gdn_gates      g = -exp(A_log) softplus(a + dt_bias) (fp32); beta = bf16(sigmoid(b))
//   qk_norm_rope   per-head RMSNorm(1+w) then rotate-half RoPE on the first
//                  `rot` dims with bf16 cos/sin, every op rounded to bf16
//   embedding      row gather
// A row is spread over up to 64 lanes of one wave, 8 elements (16 bytes) per
// lane per step, so every access is a full 16-byte vector.

#include "kad_common.h"

namespace {

__device__ __forceinline__ void unpack8(u32x4 r, float* f) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    f[2 * e] = __uint_as_float(r[e] << 16);
    f[2 * e + 1] = __uint_as_float(r[e] & 0xffff0000u);
  }
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 r;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    r[e] = (uint32_t)f2bf(f[2 * e]) | ((uint32_t)f2bf(f[2 * e + 1]) << 16);
  return r;
}

// sum over the `lanes` lanes (power of two <= 64) that share a row
__device__ __forceinline__ float group_sum(float v, int lanes) {
  for (int o = lanes / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Rows of D elements; `lanes` lanes per row, each handling D/(8*lanes) chunks.
// LANES, CHUNKS > 0: the common shape fixed at compile time, the row's chunks
// held in registers between the two passes (0: the runtime form, which reads
// them again).
template <int LANES, int CHUNKS>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const bf16_t* __restrict__ x, int64_t ldx,
                                                      const bf16_t* __restrict__ w,
                                                      bf16_t* __restrict__ y, int64_t ldy,
                                                      int64_t rows, int D, int lanes_rt,
                                                      float eps, float w_offset) {
  constexpr bool kFixed = LANES > 0;
  const int lanes = kFixed ? LANES : lanes_rt;
  const int rows_per_block = 256 / lanes;
  const int64_t row = (int64_t)blockIdx.x * rows_per_block + threadIdx.x / lanes;
  const int li = threadIdx.x % lanes;
  const int chunks = kFixed ? CHUNKS : D / (8 * lanes);
  const bool live = row < rows;
  const bf16_t* xr = x + (live ? row : 0) * ldx;
  u32x4 xs[kFixed ? CHUNKS : 1];
  float ss = 0.f;
  for (int c = 0; c < chunks; ++c) {
    const u32x4 raw = *(const u32x4*)(xr + (c * lanes + li) * 8);
    if constexpr (kFixed) xs[c] = raw;
    float f[8];
    unpack8(raw, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += f[i] * f[i];
  }
  ss = group_sum(ss, lanes);
  const float r = 1.0f / sqrtf(ss / (float)D + eps);
  if (!live) return;
  for (int c = 0; c < chunks; ++c) {
    const int off = (c * lanes + li) * 8;
    float f[8], wv[8];
    if constexpr (kFixed)
      unpack8(xs[c], f);
    else
      unpack8(*(const u32x4*)(xr + off), f);
    unpack8(*(const u32x4*)(w + off), wv);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (f[i] * r) * (w_offset + wv[i]);
    *(u32x4*)(y + row * ldy + off) = pack8(f);
  }
}

// groups of D elements: x row stride ldx between tokens, `heads` groups per
// token at stride D; z likewise with ldz; y contiguous [rows, heads*D] (ldy)
template <int LANES, int CHUNKS>
__global__ __launch_bounds__(256) void rmsnorm_gated_kernel(
    const bf16_t* __restrict__ x, int64_t ldx, const bf16_t* __restrict__ z, int64_t ldz,
    const bf16_t* __restrict__ w, bf16_t* __restrict__ y, int64_t ldy, int64_t groups, int heads,
    int D, int lanes_rt, float eps) {
  constexpr bool kFixed = LANES > 0;
  const int lanes = kFixed ? LANES : lanes_rt;
  const int per_block = 256 / lanes;
  const int64_t gidx = (int64_t)blockIdx.x * per_block + threadIdx.x / lanes;
  const int li = threadIdx.x % lanes;
  const int chunks = kFixed ? CHUNKS : D / (8 * lanes);
  const bool live = gidx < groups;
  const int64_t g = live ? gidx : 0;
  const int64_t tok = g / heads;
  const int hh = (int)(g % heads);
  const bf16_t* xr = x + tok * ldx + (int64_t)hh * D;
  const bf16_t* zr = z + tok * ldz + (int64_t)hh * D;
  u32x4 xs[kFixed ? CHUNKS : 1];
  float ss = 0.f;
  for (int c = 0; c < chunks; ++c) {
    const u32x4 raw = *(const u32x4*)(xr + (c * lanes + li) * 8);
    if constexpr (kFixed) xs[c] = raw;
    float f[8];
    unpack8(raw, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += f[i] * f[i];
  }
  ss = group_sum(ss, lanes);
  const float r = 1.0f / sqrtf(ss / (float)D + eps);
  if (!live) return;
  for (int c = 0; c < chunks; ++c) {
    const int off = (c * lanes + li) * 8;
    float f[8], wv[8], zv[8];
    if constexpr (kFixed)
      unpack8(xs[c], f);
    else
      unpack8(*(const u32x4*)(xr + off), f);
    unpack8(*(const u32x4*)(w + off), wv);
    unpack8(*(const u32x4*)(zr + off), zv);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float nrm = round_bf(f[i] * r);
      const float wn = round_bf(wv[i] * nrm);
      f[i] = wn * silu_fast(zv[i]);
    }
    *(u32x4*)(y + tok * ldy + (int64_t)hh * D + off) = pack8(f);
  }
}

__global__ __launch_bounds__(256) void gdn_gates_kernel(const bf16_t* __restrict__ a, int64_t lda,
                                                        const bf16_t* __restrict__ b, int64_t ldb,
                                                        const bf16_t* __restrict__ A_log,
                                                        const bf16_t* __restrict__ dt_bias,
                                                        float* __restrict__ g,
                                                        bf16_t* __restrict__ beta, int64_t rows,
                                                        int HV) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * HV) return;
  const int64_t r = idx / HV;
  const int h = (int)(idx % HV);
  const float av = bf2f(a[r * lda + h]);
  const float bv = bf2f(b[r * ldb + h]);
  const float sp = softplus_f(av + bf2f(dt_bias[h]));
  g[idx] = -expf(bf2f(A_log[h])) * sp;
  beta[idx] = f2bf(1.0f / (1.0f + expf(-bv)));
}

// One wave per (token, head) of q or k.  Input row: src + tok*ld_src + head*src_head_stride,
// D elements.  Output: dst + (tok / period)*s_b + (tok % period)*s_t + head*s_h.
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const bf16_t* __restrict__ src, int64_t ld_src, int64_t src_head_stride, int heads,
    const bf16_t* __restrict__ w, bf16_t* __restrict__ dst, int64_t period, int64_t s_b,
    int64_t s_t, int64_t s_h, int64_t rows, int D, int rot, const float* __restrict__ inv_freq,
    int64_t pos0, int64_t pos_period, float eps, int do_norm) {
  const int64_t gw = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;  // global wave = (tok, head)
  const int lane = threadIdx.x & 63;
  if (gw >= rows * heads) return;
  const int64_t tok = gw / heads;
  const int hh = (int)(gw % heads);
  const bf16_t* s = src + tok * ld_src + hh * src_head_stride;
  // each lane handles elements lane, lane+64, ... (D <= 512)
  float v[8];
  const int per = D / 64;
  float ss = 0.f;
  for (int i = 0; i < per; ++i) {
    v[i] = bf2f(s[lane + 64 * i]);
    ss += v[i] * v[i];
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)D + eps);
  if (do_norm)
    for (int i = 0; i < per; ++i) v[i] = round_bf((v[i] * r) * (1.0f + bf2f(w[lane + 64 * i])));
  // rotate-half RoPE on dims [0, rot): pair (d, d + rot/2)
  const int half = rot / 2;
  const float pos = (float)(pos0 + tok % pos_period);
  float outv[8];
  for (int i = 0; i < per; ++i) {
    const int d = lane + 64 * i;
    outv[i] = v[i];
    if (d < rot) {
      const int fi = d % half;
      const float ang = pos * inv_freq[fi];
      const float c = round_bf(cosf(ang)), sn = round_bf(sinf(ang));
      // partner element value (rotate_half): -x[d+half] for d<half, x[d-half] otherwise
      const int pd = d < half ? d + half : d - half;
      float partner = bf2f(s[pd]);
      if (do_norm) partner = round_bf((partner * r) * (1.0f + bf2f(w[pd])));
      const float rh = d < half ? -partner : partner;
      outv[i] = round_bf(round_bf(v[i] * c) + round_bf(rh * sn));
    }
  }
  bf16_t* o = dst + (tok / period) * s_b + (tok % period) * s_t + hh * s_h;
  for (int i = 0; i < per; ++i) o[lane + 64 * i] = f2bf(outv[i]);
}

// The same operation with 16-byte accesses: one wave per token, LPH = D/8
// lanes per head (8 consecutive elements each), 64/LPH heads per pass.  The
// rotary cos/sin are computed once per token (lane l evaluates frequency
// l % (rot/2)) and reused by every head; the rotate-half partner (dim d +- rot/2, P = rot/16 lanes
// away) comes from a lane exchange.  Needs rot/16 a power of two (or rot 0).
// DT, ROTT > 0: the model's head (d 256, rotary 64, normed) fixed at compile
// time, so the lane arithmetic, shuffles and loops are constants; 0: runtime
template <int DT, int ROTT>
__global__ __launch_bounds__(256) void qk_norm_rope_vec_kernel(
    const bf16_t* __restrict__ src, int64_t ld_src, int64_t src_head_stride, int heads,
    const bf16_t* __restrict__ w, bf16_t* __restrict__ dst, int64_t period, int64_t s_b,
    int64_t s_t, int64_t s_h, int64_t rows, int D_rt, int rot_rt,
    const float* __restrict__ inv_freq, int64_t pos0, int64_t pos_period, float eps,
    int do_norm_rt) {
  constexpr bool kFixed = DT > 0;
  const int D = kFixed ? DT : D_rt;
  const int rot = kFixed ? ROTT : rot_rt;
  const bool do_norm = kFixed ? true : do_norm_rt != 0;
  const int64_t tok = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;
  const int lane = threadIdx.x & 63;
  if (tok >= rows) return;
  const int lph = D / 8, hpp = 64 / lph;
  const int m = lane % lph, d0 = m * 8;
  const int half = rot / 2, P = rot / 16;
  const bool in_rot = d0 < rot;
  float wv[8];
  if (do_norm) {
    unpack8(*(const u32x4*)(w + d0), wv);
#pragma unroll
    for (int i = 0; i < 8; ++i) wv[i] += 1.0f;
  }
  float cs[8], sn[8];
  const float pos = (float)(pos0 + tok % pos_period);
  if (half <= 64) {
    // lane l evaluates frequency l % half once; lanes fetch their 8
    float c1 = 0.f, s1 = 0.f;
    if (half) {
      const float ang = pos * inv_freq[lane % half];
      c1 = round_bf(cosf(ang));
      s1 = round_bf(sinf(ang));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int src_lane = half ? (d0 + i) % half : 0;
      cs[i] = __shfl(c1, src_lane, 64);
      sn[i] = __shfl(s1, src_lane, 64);
    }
  } else if (in_rot) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float ang = pos * inv_freq[(d0 + i) % half];
      cs[i] = round_bf(cosf(ang));
      sn[i] = round_bf(sinf(ang));
    }
  }
  const bf16_t* srow = src + tok * ld_src;
  bf16_t* drow = dst + (tok / period) * s_b + (tok % period) * s_t;
  for (int h0 = 0; h0 < heads; h0 += hpp) {
    const int hh = h0 + lane / lph;
    const bool live = hh < heads;
    float v[8];
    unpack8(*(const u32x4*)(srow + (int64_t)(live ? hh : h0) * src_head_stride + d0), v);
    if (do_norm) {
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
      ss = group_sum(ss, lph);
      const float r = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = round_bf((v[i] * r) * wv[i]);
    }
    if (rot) {
      // every lane takes part in the exchange; lanes outside [0, rot) keep v
      float pr[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) pr[i] = __shfl_xor(v[i], P, 64);
      if (in_rot) {
        const bool lo = d0 < half;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float rh = lo ? -pr[i] : pr[i];
          v[i] = round_bf(round_bf(v[i] * cs[i]) + round_bf(rh * sn[i]));
        }
      }
    }
    if (live) *(u32x4*)(drow + (int64_t)hh * s_h + d0) = pack8(v);
  }
}

// copy [rows, heads, D] head rows into a strided destination (prefill V
// cache); IDX: 32-bit index arithmetic whenever the chunk count fits
template <typename IDX>
__global__ __launch_bounds__(256) void scatter_heads_kernel(const bf16_t* __restrict__ src,
                                                            int64_t ld_src, int heads, int D,
                                                            bf16_t* __restrict__ dst,
                                                            int64_t period, int64_t s_b,
                                                            int64_t s_t, int64_t s_h,
                                                            int64_t rows) {
  const int chunks = D / 8;
  const IDX idx = (IDX)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (IDX)rows * heads * chunks) return;
  const int c = (int)(idx % (IDX)chunks);
  const IDX gh = idx / (IDX)chunks;
  const int hh = (int)(gh % (IDX)heads);
  const IDX tok = gh / (IDX)heads;
  const int64_t tb = (int64_t)(tok / (IDX)period), tt = (int64_t)(tok % (IDX)period);
  const u32x4 v = *(const u32x4*)(src + (int64_t)tok * ld_src + (int64_t)hh * D + c * 8);
  *(u32x4*)(dst + tb * s_b + tt * s_t + hh * s_h + c * 8) = v;
}

__global__ __launch_bounds__(256) void embedding_kernel(const int64_t* __restrict__ ids,
                                                        const bf16_t* __restrict__ table,
                                                        bf16_t* __restrict__ out, int64_t rows,
                                                        int D, int64_t vocab) {
  const int chunks = D / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= rows * chunks) return;
  const int64_t r = idx / chunks;
  const int c = (int)(idx % chunks);
  int64_t id = ids[r];
  // clamped so that the table read stays in bounds whatever the caller passes;
  // the model adapters reject out-of-range ids on the host before launching
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);
  *(u32x4*)(out + r * D + c * 8) = *(const u32x4*)(table + id * D + c * 8);
}

int lanes_for(int D) {
  int chunks = D / 8, lanes = 1;
  while (lanes * 2 <= 64 && chunks % (lanes * 2) == 0) lanes *= 2;
  return lanes;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" int kad_rmsnorm(const void* x, int64_t ldx, const void* w, float w_offset, void* y,
                           int64_t ldy, int64_t rows, int D, float eps, kad_stream_t stream) {
  KAD_REQUIRE(x && w && y, "null pointer argument");
  KAD_REQUIRE(rows > 0 && D > 0 && D % 8 == 0, "rows > 0 and D %% 8 == 0 required");
  KAD_REQUIRE(ldx % 8 == 0 && ldy % 8 == 0 && aligned16(x) && aligned16(y) && aligned16(w),
              "16-byte aligned rows required");
  const int lanes = lanes_for(D);
  const int64_t per_block = 256 / lanes;
  const dim3 grid((unsigned)kad_cdiv(rows, per_block));
  if (lanes == 64 && D == 1024)   // the model's hidden size
    hipLaunchKernelGGL((rmsnorm_kernel<64, 2>), grid, dim3(256), 0, (hipStream_t)stream,
                       (const bf16_t*)x, ldx, (const bf16_t*)w, (bf16_t*)y, ldy, rows, D, lanes,
                       eps, w_offset);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<0, 0>), grid, dim3(256), 0, (hipStream_t)stream,
                       (const bf16_t*)x, ldx, (const bf16_t*)w, (bf16_t*)y, ldy, rows, D, lanes,
                       eps, w_offset);
  return kad_launch_status("rmsnorm_kernel");
}

extern "C" int kad_rmsnorm_gated(const void* x, int64_t ldx, const void* z, int64_t ldz,
                                 const void* w, void* y, int64_t ldy, int64_t rows, int heads,
                                 int D, float eps, kad_stream_t stream) {
  KAD_REQUIRE(x && z && w && y, "null pointer argument");
  KAD_REQUIRE(rows > 0 && heads > 0 && D > 0 && D % 8 == 0, "bad dimensions");
  KAD_REQUIRE(ldx % 8 == 0 && ldz % 8 == 0 && ldy % 8 == 0 && aligned16(x) && aligned16(z) &&
                  aligned16(y) && aligned16(w),
              "16-byte aligned rows required");
  const int lanes = lanes_for(D);
  const int64_t groups = rows * heads, per_block = 256 / lanes;
  const dim3 grid((unsigned)kad_cdiv(groups, per_block));
  if (lanes == 16 && D == 128)   // the GDN value head
    hipLaunchKernelGGL((rmsnorm_gated_kernel<16, 1>), grid, dim3(256), 0, (hipStream_t)stream,
                       (const bf16_t*)x, ldx, (const bf16_t*)z, ldz, (const bf16_t*)w, (bf16_t*)y,
                       ldy, groups, heads, D, lanes, eps);
  else
    hipLaunchKernelGGL((rmsnorm_gated_kernel<0, 0>), grid, dim3(256), 0, (hipStream_t)stream,
                       (const bf16_t*)x, ldx, (const bf16_t*)z, ldz, (const bf16_t*)w, (bf16_t*)y,
                       ldy, groups, heads, D, lanes, eps);
  return kad_launch_status("rmsnorm_gated_kernel");
}

extern "C" int kad_gdn_gates(const void* a, int64_t lda, const void* b, int64_t ldb,
                             const void* A_log, const void* dt_bias, float* g, void* beta,
                             int64_t rows, int HV, kad_stream_t stream) {
  KAD_REQUIRE(a && b && A_log && dt_bias && g && beta, "null pointer argument");
  KAD_REQUIRE(rows > 0 && HV > 0, "bad dimensions");
  const int64_t total = rows * HV;
  hipLaunchKernelGGL(gdn_gates_kernel, dim3((unsigned)kad_cdiv(total, 256)), dim3(256), 0,
                     (hipStream_t)stream, (const bf16_t*)a, lda, (const bf16_t*)b, ldb,
                     (const bf16_t*)A_log, (const bf16_t*)dt_bias, g, (bf16_t*)beta, rows, HV);
  return kad_launch_status("gdn_gates_kernel");
}

extern "C" int kad_qk_norm_rope(const void* src, int64_t ld_src, int64_t src_head_stride,
                                int heads, const void* w, void* dst, int64_t period, int64_t s_b,
                                int64_t s_t, int64_t s_h, int64_t rows, int D, int rot,
                                const float* inv_freq, int64_t pos0, int64_t pos_period,
                                float eps, int do_norm, kad_stream_t stream) {
  KAD_REQUIRE(src && dst && inv_freq && (w || !do_norm), "null pointer argument");
  KAD_REQUIRE(rows > 0 && heads > 0 && D % 64 == 0 && D <= 512, "D must be a multiple of 64, <= 512");
  KAD_REQUIRE(rot >= 0 && rot <= D && rot % 2 == 0, "bad rotary dimension");
  KAD_REQUIRE(period > 0 && pos_period > 0, "bad periods");
  const int P = rot / 16;
  const bool vec = D % 8 == 0 && D / 8 <= 64 && (64 % (D / 8)) == 0 &&
                   (rot == 0 || (rot % 16 == 0 && (P & (P - 1)) == 0)) &&
                   aligned16(src) && aligned16(dst) && (!do_norm || aligned16(w)) &&
                   ld_src % 8 == 0 && src_head_stride % 8 == 0 && s_b % 8 == 0 && s_t % 8 == 0 &&
                   s_h % 8 == 0;
  if (vec) {
    const dim3 grid((unsigned)kad_cdiv(rows, 4));
    if (D == 256 && rot == 64 && do_norm)   // Qwen3.5's attention heads
      hipLaunchKernelGGL((qk_norm_rope_vec_kernel<256, 64>), grid, dim3(256), 0,
                         (hipStream_t)stream, (const bf16_t*)src, ld_src, src_head_stride, heads,
                         (const bf16_t*)w, (bf16_t*)dst, period, s_b, s_t, s_h, rows, D, rot,
                         inv_freq, pos0, pos_period, eps, do_norm);
    else
      hipLaunchKernelGGL((qk_norm_rope_vec_kernel<0, 0>), grid, dim3(256), 0,
                         (hipStream_t)stream, (const bf16_t*)src, ld_src, src_head_stride, heads,
                         (const bf16_t*)w, (bf16_t*)dst, period, s_b, s_t, s_h, rows, D, rot,
                         inv_freq, pos0, pos_period, eps, do_norm);
    return kad_launch_status("qk_norm_rope_vec_kernel");
  }
  const int64_t waves = rows * heads;
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned)kad_cdiv(waves, 4)), dim3(256), 0,
                     (hipStream_t)stream, (const bf16_t*)src, ld_src, src_head_stride, heads,
                     (const bf16_t*)w, (bf16_t*)dst, period, s_b, s_t, s_h, rows, D, rot, inv_freq,
                     pos0, pos_period, eps, do_norm);
  return kad_launch_status("qk_norm_rope_kernel");
}

extern "C" int kad_scatter_heads(const void* src, int64_t ld_src, int heads, int D, void* dst,
                                 int64_t period, int64_t s_b, int64_t s_t, int64_t s_h,
                                 int64_t rows, kad_stream_t stream) {
  KAD_REQUIRE(src && dst, "null pointer argument");
  KAD_REQUIRE(rows > 0 && heads > 0 && D % 8 == 0 && period > 0, "bad dimensions");
  KAD_REQUIRE(aligned16(src) && aligned16(dst) && ld_src % 8 == 0 && s_b % 8 == 0 &&
                  s_t % 8 == 0 && s_h % 8 == 0,
              "16-byte aligned rows required");
  const int64_t total = rows * heads * (D / 8);
  if (total + 256 < ((int64_t)1 << 31) && period < ((int64_t)1 << 31))
    hipLaunchKernelGGL(scatter_heads_kernel<uint32_t>, dim3((unsigned)kad_cdiv(total, 256)),
                       dim3(256), 0, (hipStream_t)stream, (const bf16_t*)src, ld_src, heads, D,
                       (bf16_t*)dst, period, s_b, s_t, s_h, rows);
  else
    hipLaunchKernelGGL(scatter_heads_kernel<int64_t>, dim3((unsigned)kad_cdiv(total, 256)),
                       dim3(256), 0, (hipStream_t)stream, (const bf16_t*)src, ld_src, heads, D,
                       (bf16_t*)dst, period, s_b, s_t, s_h, rows);
  return kad_launch_status("scatter_heads_kernel");
}

extern "C" int kad_embedding(const int64_t* ids, const void* table, void* out, int64_t rows,
                             int D, int64_t vocab, kad_stream_t stream) {
  KAD_REQUIRE(ids && table && out, "null pointer argument");
  KAD_REQUIRE(rows > 0 && D % 8 == 0 && vocab > 0, "bad dimensions");
  KAD_REQUIRE(aligned16(table) && aligned16(out), "16-byte aligned rows required");
  const int64_t total = rows * (D / 8);
  hipLaunchKernelGGL(embedding_kernel, dim3((unsigned)kad_cdiv(total, 256)), dim3(256), 0,
                     (hipStream_t)stream, ids, (const bf16_t*)table, (bf16_t*)out, rows, D, vocab);
  return kad_launch_status("embedding_kernel");
}
