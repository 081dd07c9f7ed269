// Chunked gated delta rule (gfx950): prefill state building and long suffixes.
//
// Replaces, for the prefill, transformers' torch_chunk_gated_delta_rule
// (modeling_qwen3_5.py:249-327) that the reference prefill runs through the
// native model forward (src/kadllm/adapters/qwen3_5.py:111), and, for the
// operator, src/kadllm/ops.py:139-163 when a suffix is longer than the replay
// kernel handles or a final state is requested (ops.py:119-122).
//
// One workgroup per (sequence n, value head hv) walks the sequence in chunks
// of 64 tokens; thread v owns column v of the fp32 state S [K, V] in
// registers.  Per chunk, with G the within-chunk cumulative log decay,
// D_ij = exp(G_i - G_j) and hats the normalised q (incl. scale) and k:
//   A_ij  = -beta_i (k^_i . k^_j) D_ij (j < i); T' = the routine's forward
//           substitution of A (rows i = 1..63); T = T' + I
//   Z_j   = beta_j (v_j - e^{G_j} k^_j S)          (so that v_new = T Z equals
//           U - W S with U = T beta v, W = T beta k^ e^G of the routine)
//   o_i   = e^{G_i} q^_i S + sum_{j<=i} (q^_i . k^_j) D_ij v_new_j
//   S    <- e^{G_last} S + sum_i e^{G_last - G_i} k^_i v_new_i^T
// The two 64 x 64 Gram matrices (k k^T, q k^T) run on bf16 MFMA from the bf16
// q/k rows staged in LDS (raw rows with fp32 norms applied afterwards, or,
// in the transformers prefill mode, rows normalised with its bf16 roundings,
// l2norm in modeling_qwen3_5.py:242-246); everything touching S is fp32.

#include "kad_common.h"

namespace {

constexpr int kC = 64;

template <int K>
struct ChunkSmem {
  static constexpr int ld = K + 8;  // bf16 row stride (16-byte padding)
};

template <int K, int V>
__global__ __launch_bounds__(V) void gdn_chunk_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, const bf16_t* __restrict__ v,
    int64_t ld_qk, int64_t ld_v, const void* __restrict__ g, int gdt,
    const void* __restrict__ beta, int bdt, int64_t ld_gate, const void* __restrict__ state0,
    int sdt, int beams_per_state, bf16_t* __restrict__ out, int64_t ld_out,
    float* __restrict__ final_state, int T, int H, int HV, float scale, int hf_norm) {
  constexpr int LD = ChunkSmem<K>::ld;
  constexpr int NW = V / 64;  // waves
  __shared__ __attribute__((aligned(16))) bf16_t kb[kC * LD];
  __shared__ __attribute__((aligned(16))) bf16_t qb[kC * LD];
  __shared__ float Am[kC][kC + 1];
  __shared__ float Tm[kC][kC + 1];
  __shared__ float In[kC][kC + 1];
  __shared__ float Gs[kC], eG[kC], bt[kC], kmul[kC], qmul[kC], wupd[kC];

  const int col = threadIdx.x;  // value column
  const int lane = col & 63, wave = col >> 6;
  const int n = blockIdx.x / HV, hv = blockIdx.x % HV;
  const int h = hv / (HV / H);

  float S[K];
  if (state0) {
    const int64_t base = ((int64_t)(n / beams_per_state) * HV + hv) * K * V + col;
#pragma unroll
    for (int kk = 0; kk < K; ++kk) S[kk] = load_as_float(state0, base + (int64_t)kk * V, sdt);
  } else {
#pragma unroll
    for (int kk = 0; kk < K; ++kk) S[kk] = 0.f;
  }

  const int nchunks = (T + kC - 1) / kC;
  for (int c = 0; c < nchunks; ++c) {
    const int t0 = c * kC;
    const int nt = min(kC, T - t0);
    __syncthreads();  // previous chunk done with LDS

    // ---- stage q/k rows (bf16) with their normalisation multipliers
    for (int i = wave; i < kC; i += NW) {
      float kv[K / 64], qv[K / 64];
      const bool live = i < nt;
      const int64_t row = ((int64_t)n * T + t0 + (live ? i : 0)) * ld_qk + (int64_t)h * K;
      float kss = 0.f, qss = 0.f;
#pragma unroll
      for (int e = 0; e < K / 64; ++e) {
        kv[e] = live ? bf2f(k[row + lane + 64 * e]) : 0.f;
        qv[e] = live ? bf2f(q[row + lane + 64 * e]) : 0.f;
        if (hf_norm) {
          kss += round_bf(kv[e] * kv[e]);
          qss += round_bf(qv[e] * qv[e]);
        } else {
          kss += kv[e] * kv[e];
          qss += qv[e] * qv[e];
        }
      }
      kss = wave_sum(kss);
      qss = wave_sum(qss);
      float km, qm;
      if (hf_norm) {
        // x * rsqrt(sum(x*x) + eps), every op rounded to bf16
        const float kr = round_bf(1.0f / sqrtf(round_bf(round_bf(kss) + 1e-6f)));
        const float qr = round_bf(1.0f / sqrtf(round_bf(round_bf(qss) + 1e-6f)));
#pragma unroll
        for (int e = 0; e < K / 64; ++e) {
          kv[e] = round_bf(kv[e] * kr);
          qv[e] = round_bf(qv[e] * qr);
        }
        km = 1.f;
        qm = scale;
      } else {
        km = 1.0f / sqrtf(kss + 1e-6f);
        qm = scale / sqrtf(qss + 1e-6f);
      }
#pragma unroll
      for (int e = 0; e < K / 64; ++e) {
        kb[i * LD + lane + 64 * e] = f2bf(kv[e]);
        qb[i * LD + lane + 64 * e] = f2bf(qv[e]);
      }
      if (lane == 0) {
        kmul[i] = km;
        qmul[i] = qm;
      }
    }
    if (col < kC) {
      const int i = col;
      const bool live = i < nt;
      const int64_t gi = ((int64_t)n * T + t0 + (live ? i : 0)) * ld_gate + hv;
      Gs[i] = live ? load_as_float(g, gi, gdt) : 0.f;
      bt[i] = live ? load_as_float(beta, gi, bdt) : 0.f;
    }
    __syncthreads();
    if (col == 0) {
      float acc = 0.f;
      for (int i = 0; i < kC; ++i) {  // sequential cumulative sum, as torch.cumsum
        acc += Gs[i];
        Gs[i] = acc;
      }
    }
    __syncthreads();
    if (col < kC) {
      eG[col] = expf(Gs[col]);
      wupd[col] = kmul[col] * expf(Gs[kC - 1] - Gs[col]);
    }

    // ---- Gram matrices on MFMA: wave 0 (or the only wave) k k^T, then q k^T
    for (int which = wave; which < 2; which += NW) {
      const bf16_t* rowsrc = which == 0 ? kb : qb;
      const int fr = lane & 31, fk = (lane >> 5) * 8;
#pragma unroll
      for (int ti = 0; ti < 2; ++ti)
#pragma unroll
        for (int tj = 0; tj < 2; ++tj) {
          f32x16 acc = f32x16{};
#pragma unroll
          for (int s = 0; s < K / 16; ++s) {
            const bf16x8 a = as_bf16x8(*(const u32x4*)(rowsrc + (ti * 32 + fr) * LD + s * 16 + fk));
            const bf16x8 b = as_bf16x8(*(const u32x4*)(kb + (tj * 32 + fr) * LD + s * 16 + fk));
            acc = mfma32x32x16(a, b, acc);
          }
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int i = ti * 32 + (e / 4) * 8 + (lane >> 5) * 4 + (e % 4);
            const int j = tj * 32 + fr;
            if (which == 0)
              Am[i][j] = j < i ? -bt[i] * (acc[e] * kmul[i] * kmul[j]) * expf(Gs[i] - Gs[j]) : 0.f;
            else
              In[i][j] = j <= i ? (acc[e] * qmul[i] * kmul[j]) * expf(Gs[i] - Gs[j]) : 0.f;
          }
        }
    }
    __syncthreads();

    // ---- forward substitution: T'[i][j] = A[i][j] + sum_{j<m<i} A[i][m] T'[m][j]
    if (col < kC) Tm[0][col] = 0.f;
    for (int i = 1; i < kC; ++i) {
      __syncthreads();
      if (col < i) {
        float acc = Am[i][col];
        for (int m = col + 1; m < i; ++m) acc += Am[i][m] * Tm[m][col];
        Tm[i][col] = acc;
      } else if (col < kC) {
        Tm[i][col] = 0.f;
      }
    }
    __syncthreads();

    // ---- Z_j = beta_j (v_j - e^{G_j} k^_j S), then v_new = (T' + I) Z (in place, i descending)
    float z[kC];
#pragma unroll
    for (int j = 0; j < kC; ++j) {
      float dot = 0.f;
#pragma unroll
      for (int k8 = 0; k8 < K; k8 += 8) {
        const u32x4 r = *(const u32x4*)(kb + j * LD + k8);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          dot += __uint_as_float(r[e] << 16) * S[k8 + 2 * e];
          dot += __uint_as_float(r[e] & 0xffff0000u) * S[k8 + 2 * e + 1];
        }
      }
      const float vj = j < nt ? bf2f(v[((int64_t)n * T + t0 + j) * ld_v + (int64_t)hv * V + col]) : 0.f;
      z[j] = bt[j] * (vj - eG[j] * (kmul[j] * dot));
    }
#pragma unroll
    for (int i = kC - 1; i > 0; --i) {
      float acc = z[i];
#pragma unroll
      for (int j = 0; j < i; ++j) acc += Tm[i][j] * z[j];
      z[i] = acc;
    }

    // ---- o_i = e^{G_i} q^_i S + sum_{j<=i} In[i][j] v_new_j
#pragma unroll
    for (int i = 0; i < kC; ++i) {
      float dot = 0.f;
#pragma unroll
      for (int k8 = 0; k8 < K; k8 += 8) {
        const u32x4 r = *(const u32x4*)(qb + i * LD + k8);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          dot += __uint_as_float(r[e] << 16) * S[k8 + 2 * e];
          dot += __uint_as_float(r[e] & 0xffff0000u) * S[k8 + 2 * e + 1];
        }
      }
      float o = eG[i] * (qmul[i] * dot);
#pragma unroll
      for (int j = 0; j <= i; ++j) o += In[i][j] * z[j];
      if (i < nt) out[((int64_t)n * T + t0 + i) * ld_out + (int64_t)hv * V + col] = f2bf(o);
    }

    // ---- S <- e^{G_last} S + sum_i (k^_i e^{G_last - G_i}) v_new_i
    const float eGl = eG[kC - 1];
#pragma unroll
    for (int kk = 0; kk < K; ++kk) S[kk] *= eGl;
#pragma unroll
    for (int i = 0; i < kC; ++i) {
      const float w = wupd[i] * z[i];
#pragma unroll
      for (int k8 = 0; k8 < K; k8 += 8) {
        const u32x4 r = *(const u32x4*)(kb + i * LD + k8);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          S[k8 + 2 * e] += __uint_as_float(r[e] << 16) * w;
          S[k8 + 2 * e + 1] += __uint_as_float(r[e] & 0xffff0000u) * w;
        }
      }
    }
  }
  if (final_state) {
    const int64_t base = ((int64_t)n * HV + hv) * K * V + col;
#pragma unroll
    for (int kk = 0; kk < K; ++kk) final_state[base + (int64_t)kk * V] = S[kk];
  }
}

template <int K, int V>
int launch_chunk(const void* q, const void* k, const void* v, int64_t ld_qk, int64_t ld_v,
                 const void* g, int gdt, const void* beta, int bdt, int64_t ld_gate,
                 const void* state0, int sdt, int bps, void* out, int64_t ld_out, float* fin,
                 int N, int T, int H, int HV, float scale, int hf_norm, hipStream_t s) {
  hipLaunchKernelGGL((gdn_chunk_kernel<K, V>), dim3((unsigned)((int64_t)N * HV)), dim3(V), 0, s,
                     (const bf16_t*)q, (const bf16_t*)k, (const bf16_t*)v, ld_qk, ld_v, g, gdt,
                     beta, bdt, ld_gate, state0, sdt, bps, (bf16_t*)out, ld_out, fin, T, H, HV,
                     scale, hf_norm);
  return kad_launch_status("gdn_chunk_kernel");
}

}  // namespace

extern "C" int kad_gdn_chunk(const void* q, const void* k, const void* v, int64_t ld_qk,
                             int64_t ld_v, int qkv_dtype, const void* log_decay, int gate_dtype,
                             const void* beta, int beta_dtype, int64_t ld_gate,
                             const void* initial_state, int state_dtype, int beams_per_state,
                             void* out, int64_t ld_out, float* final_state, int N, int T, int H,
                             int HV, int K, int V, float scale, int transformers_l2norm,
                             kad_stream_t stream) {
  KAD_REQUIRE(q && k && v && log_decay && beta && out, "null pointer argument");
  KAD_REQUIRE(N > 0 && T > 0 && H > 0 && HV > 0 && HV % H == 0, "bad dimensions");
  KAD_REQUIRE(!initial_state || (beams_per_state > 0 && N % beams_per_state == 0),
              "N must be a multiple of beams_per_state");
  KAD_REQUIRE(ld_qk >= (int64_t)H * K && ld_v >= (int64_t)HV * V && ld_out >= (int64_t)HV * V &&
                  ld_gate >= HV,
              "row strides smaller than a row");
  if (qkv_dtype != KAD_DTYPE_BF16) KAD_UNSUPPORTED("chunked gated delta takes bf16 q/k/v");
  hipStream_t s = (hipStream_t)stream;
#define KAD_CHUNK(KK, VV)                                                                     \
  if (K == KK && V == VV)                                                                     \
    return launch_chunk<KK, VV>(q, k, v, ld_qk, ld_v, log_decay, gate_dtype, beta, beta_dtype, \
                                ld_gate, initial_state, state_dtype, beams_per_state, out,    \
                                ld_out, final_state, N, T, H, HV, scale, transformers_l2norm, s);
  KAD_CHUNK(128, 128)
  KAD_CHUNK(64, 64)
  KAD_CHUNK(128, 64)
  KAD_CHUNK(64, 128)
#undef KAD_CHUNK
  KAD_UNSUPPORTED("chunked gated delta supports K, V in {64, 128}; got K=%d V=%d", K, V);
}
