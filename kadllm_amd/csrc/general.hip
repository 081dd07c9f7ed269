// General-shape kernels (gfx950): any head dimension up to 256, any suffix
// length, fp32 / bf16 / fp16 tensors, fp32 arithmetic.
//
// The specialised kernels (factored suffix replay, chunked GDN, prefix-shared
// MFMA attention) cover the Qwen3.5 shapes: head dims 64/128/256, suffixes of
// a few tokens, bf16.  The reference operators accept any shape and dtype
// (src/kadllm/ops.py:70-163,252-341), and its own toy model runs 8-wide heads
// in fp32 over whole prompts (src/kadllm/adapters/reference.py:56-91).  These
// kernels serve every shape outside the specialised set, with the arithmetic
// of the reference's torch path in fp32: the per-token recurrence of
// ops.py:152-158 and one softmax over the prefix and causal suffix keys
// (equal to the two-partition LSE merge of ops.py:229-249,340).
//
// Both are one wave per unit of work; neither is meant for the headline
// shapes, which the specialised kernels serve.

#include "kad_common.h"

namespace {

__device__ __forceinline__ void store_from_float(void* p, int64_t i, int dtype, float f) {
  if (dtype == KAD_DTYPE_F32)
    ((float*)p)[i] = f;
  else if (dtype == KAD_DTYPE_BF16)
    ((bf16_t*)p)[i] = f2bf(f);
  else
    ((_Float16*)p)[i] = (_Float16)f;
}

// 1 / (1 + e^-x) with the IEEE exp and divide (torch.sigmoid in fp32)
__device__ __forceinline__ float sigmoid_exact(float x) { return 1.0f / (1.0f + expf(-x)); }

// ---------------------------------------------------------------------------
// Gated delta recurrence, one wave per (sequence n, value head hv, 64 value
// columns).  The columns of the state evolve independently under
//   S <- S e^{g_t};  u = beta_t (v_t - S^T k_t);  S <- S + k_t u^T;  o_t = S^T q_t
// so lane j keeps column v0 + j of S (K values) in registers for all T tokens.
// q and k of each token are L2-normalised in fp32 as the reference does
// (q / sqrt(sum q^2 + 1e-6) * scale, ops.py:147-148) and shared through LDS.
template <int KMAX>
__global__ __launch_bounds__(64) void gdn_recurrent_kernel(
    const void* __restrict__ q, const void* __restrict__ k, const void* __restrict__ v,
    int64_t ld_qk, int64_t ld_v, int qkv_dtype, const void* __restrict__ gdecay,
    int gate_dtype, const void* __restrict__ beta, int beta_dtype, int64_t ld_gate,
    const void* __restrict__ init, int state_dtype, int beams_per_state, void* __restrict__ out,
    int64_t ld_out, float* __restrict__ final_state, int T, int H, int HV, int K, int V,
    float scale, int nvt) {
  __shared__ float qs[KMAX], ks[KMAX];
  const int lane = threadIdx.x;
  const int64_t bid = blockIdx.x;
  const int vt = (int)(bid % nvt);
  const int64_t nh = bid / nvt;
  const int hv = (int)(nh % HV);
  const int64_t n = nh / HV;
  const int h = hv / (HV / H);
  const int j = vt * 64 + lane;
  const bool active = j < V;

  float s[KMAX];
  const int64_t sbase = init ? (((n / beams_per_state) * HV + hv) * (int64_t)K) * V : 0;
#pragma unroll
  for (int i = 0; i < KMAX; ++i)
    s[i] = (init && active && i < K) ? load_as_float(init, sbase + (int64_t)i * V + j, state_dtype)
                                     : 0.f;

  for (int t = 0; t < T; ++t) {
    const int64_t row = n * T + t;
    float sq = 0.f, sk = 0.f;
    for (int i = lane; i < K; i += 64) {
      const float a = load_as_float(q, row * ld_qk + (int64_t)h * K + i, qkv_dtype);
      const float b = load_as_float(k, row * ld_qk + (int64_t)h * K + i, qkv_dtype);
      qs[i] = a;
      ks[i] = b;
      sq += a * a;
      sk += b * b;
    }
    sq = wave_sum(sq);
    sk = wave_sum(sk);
    const float dq = sqrtf(sq + 1e-6f), dk = sqrtf(sk + 1e-6f);
    for (int i = lane; i < K; i += 64) {
      qs[i] = qs[i] / dq * scale;
      ks[i] = ks[i] / dk;
    }
    __syncthreads();
    const float decay = expf(load_as_float(gdecay, row * ld_gate + hv, gate_dtype));
    const float bt = load_as_float(beta, row * ld_gate + hv, beta_dtype);
    const float vj = active ? load_as_float(v, row * ld_v + (int64_t)hv * V + j, qkv_dtype) : 0.f;
    float recall = 0.f;
#pragma unroll
    for (int i = 0; i < KMAX; ++i) {
      if (i < K) {
        s[i] *= decay;
        recall += s[i] * ks[i];
      }
    }
    const float u = bt * (vj - recall);
    float o = 0.f;
#pragma unroll
    for (int i = 0; i < KMAX; ++i) {
      if (i < K) {
        s[i] += ks[i] * u;
        o += s[i] * qs[i];
      }
    }
    if (active) store_from_float(out, row * ld_out + (int64_t)hv * V + j, qkv_dtype, o);
    __syncthreads();  // qs/ks are rewritten by the next token
  }
  if (final_state && active) {
    float* f = final_state + ((n * HV + hv) * (int64_t)K) * V + j;
#pragma unroll
    for (int i = 0; i < KMAX; ++i)
      if (i < K) f[(int64_t)i * V] = s[i];
  }
}

template <int KMAX>
int launch_recurrent(const void* q, const void* k, const void* v, int64_t ld_qk, int64_t ld_v,
                     int qkv_dtype, const void* g, int gate_dtype, const void* beta,
                     int beta_dtype, int64_t ld_gate, const void* init, int state_dtype,
                     int bps, void* out, int64_t ld_out, float* fin, int N, int T, int H, int HV,
                     int K, int V, float scale, hipStream_t s) {
  const int nvt = (V + 63) / 64;
  const int64_t blocks = (int64_t)N * HV * nvt;
  if (blocks > 0x7fffffffLL) KAD_UNSUPPORTED("too many (sequence, head) pairs for one launch");
  hipLaunchKernelGGL((gdn_recurrent_kernel<KMAX>), dim3((unsigned)blocks), dim3(64), 0, s, q, k,
                     v, ld_qk, ld_v, qkv_dtype, g, gate_dtype, beta, beta_dtype, ld_gate, init,
                     state_dtype, bps, out, ld_out, fin, T, H, HV, K, V, scale, nvt);
  return kad_launch_status("gdn_recurrent_kernel");
}

// ---------------------------------------------------------------------------
// Prefix + causal-suffix attention, one wave per query row (n, t, h).  Keys
// are visited in tiles of 64: lane j scores key j of the tile (the request's
// prefix keys first, then the beam's own suffix keys up to the query's
// position), an online softmax folds each tile in, and lane l accumulates
// output dims l, l + 64, ...  Masked prefix keys are skipped; a row with no
// visible key gives zeros (ops.py:229-240).  The output is rounded to the
// tensor dtype, then multiplied by the rounded sigmoid of the gate when one is
// given (src/kadllm/adapters/qwen3_5.py:199-201).
struct AttnArgs {
  const void *q, *pk, *pv, *sk, *sv, *gate;
  const uint8_t* mask;
  void* out;
  int64_t sq_n, sq_t, sq_h;
  int64_t sp_b, sp_l, sp_h;
  int64_t ssk_n, ssk_t, ssk_h, ssv_n, ssv_t, ssv_h;
  int64_t sg_n, sg_t, sg_h;
  int64_t so_n, so_t, so_h;
  int W, Tq, Tk, H, HK, L, D, dtype;
  float scale;
};

template <int DMAX>
__global__ __launch_bounds__(64) void attention_general_kernel(AttnArgs a) {
  constexpr int R = DMAX / 64;  // output dims per lane
  __shared__ float qv[DMAX];
  __shared__ float ps[64];
  const int lane = threadIdx.x;
  const int64_t rid = blockIdx.x;
  const int h = (int)(rid % a.H);
  const int t = (int)((rid / a.H) % a.Tq);
  const int64_t n = rid / ((int64_t)a.H * a.Tq);
  const int64_t b = n / a.W;
  const int hk = h / (a.H / a.HK);
  const int tpos = t + (a.Tk - a.Tq);  // suffix position of this query
  const int nkeys = a.L + tpos + 1;
  const int dt = a.dtype;

  for (int d = lane; d < a.D; d += 64)
    qv[d] = load_as_float(a.q, n * a.sq_n + (int64_t)t * a.sq_t + (int64_t)h * a.sq_h + d, dt);
  __syncthreads();

  // element offset of key `key`'s K row and V row
  auto krow = [&](int key, const void*& base) -> int64_t {
    if (key < a.L) {
      base = a.pk;
      return b * a.sp_b + (int64_t)key * a.sp_l + (int64_t)hk * a.sp_h;
    }
    base = a.sk;
    return n * a.ssk_n + (int64_t)(key - a.L) * a.ssk_t + (int64_t)hk * a.ssk_h;
  };
  auto vrow = [&](int key, const void*& base) -> int64_t {
    if (key < a.L) {
      base = a.pv;
      return b * a.sp_b + (int64_t)key * a.sp_l + (int64_t)hk * a.sp_h;
    }
    base = a.sv;
    return n * a.ssv_n + (int64_t)(key - a.L) * a.ssv_t + (int64_t)hk * a.ssv_h;
  };

  float m = -INFINITY, l = 0.f;
  float o[R];
#pragma unroll
  for (int r = 0; r < R; ++r) o[r] = 0.f;

  for (int k0 = 0; k0 < nkeys; k0 += 64) {
    const int key = k0 + lane;
    float sc = -INFINITY;
    if (key < nkeys && !(key < a.L && a.mask && a.mask[b * a.L + key] == 0)) {
      const void* base;
      const int64_t off = krow(key, base);
      float acc = 0.f;
      for (int d = 0; d < a.D; ++d) acc += qv[d] * load_as_float(base, off + d, dt);
      sc = acc * a.scale;
    }
    const float mt = wave_max(sc);
    const float mn = fmaxf(m, mt);
    if (mn == -INFINITY) continue;  // nothing visible yet (masked keys only)
    const float p = sc == -INFINITY ? 0.f : expf(sc - mn);
    const float alpha = m == -INFINITY ? 0.f : expf(m - mn);
    l = l * alpha + wave_sum(p);
    m = mn;
    ps[lane] = p;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) o[r] *= alpha;
    const int nk = min(64, nkeys - k0);
    for (int jj = 0; jj < nk; ++jj) {
      const float pj = ps[jj];
      if (pj == 0.f) continue;
      const void* base;
      const int64_t off = vrow(k0 + jj, base);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int d = lane + 64 * r;
        if (d < a.D) o[r] += pj * load_as_float(base, off + d, dt);
      }
    }
    __syncthreads();
  }
  const float inv = l > 0.f ? 1.0f / l : 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int d = lane + 64 * r;
    if (d >= a.D) continue;
    float y = round_to_dtype(o[r] * inv, dt);
    if (a.gate) {
      const float g = load_as_float(
          a.gate, n * a.sg_n + (int64_t)t * a.sg_t + (int64_t)h * a.sg_h + d, dt);
      y = round_to_dtype(y * round_to_dtype(sigmoid_exact(g), dt), dt);
    }
    store_from_float(a.out, n * a.so_n + (int64_t)t * a.so_t + (int64_t)h * a.so_h + d, dt, y);
  }
}

}  // namespace

extern "C" int kad_gdn_recurrent(const void* q, const void* k, const void* v, int64_t ld_qk,
                                 int64_t ld_v, int qkv_dtype, const void* log_decay,
                                 int gate_dtype, const void* beta, int beta_dtype,
                                 int64_t ld_gate, const void* initial_state, int state_dtype,
                                 int beams_per_state, void* out, int64_t ld_out,
                                 float* final_state, int N, int T, int H, int HV, int K, int V,
                                 float scale, kad_stream_t stream) {
  KAD_REQUIRE(q && k && v && log_decay && beta && out, "null pointer argument");
  KAD_REQUIRE(N > 0 && T > 0 && H > 0 && HV > 0 && K > 0 && V > 0 && HV % H == 0,
              "bad dimensions");
  KAD_REQUIRE(!initial_state || (beams_per_state > 0 && N % beams_per_state == 0),
              "beams_per_state must divide N");
  KAD_REQUIRE(ld_qk >= (int64_t)H * K && ld_v >= (int64_t)HV * V && ld_out >= (int64_t)HV * V &&
                  ld_gate >= HV,
              "row strides too small");
  for (int dt : {qkv_dtype, gate_dtype, beta_dtype})
    KAD_REQUIRE(dt == KAD_DTYPE_BF16 || dt == KAD_DTYPE_F16 || dt == KAD_DTYPE_F32,
                "unknown dtype code %d", dt);
  KAD_REQUIRE(!initial_state || state_dtype == KAD_DTYPE_F32 || state_dtype == KAD_DTYPE_BF16 ||
                  state_dtype == KAD_DTYPE_F16,
              "unknown state dtype code %d", state_dtype);
  const int bps = initial_state ? beams_per_state : 1;
  hipStream_t s = (hipStream_t)stream;
#define KAD_REC(KM)                                                                           \
  if (K <= KM)                                                                                \
    return launch_recurrent<KM>(q, k, v, ld_qk, ld_v, qkv_dtype, log_decay, gate_dtype, beta, \
                                beta_dtype, ld_gate, initial_state, state_dtype, bps, out,    \
                                ld_out, final_state, N, T, H, HV, K, V, scale, s);
  KAD_REC(16)
  KAD_REC(32)
  KAD_REC(64)
  KAD_REC(128)
  KAD_REC(256)
#undef KAD_REC
  KAD_UNSUPPORTED("gated delta recurrence supports key dims <= 256, got %d", K);
}

extern "C" int kad_attention_general(
    const void* q, int64_t sq_n, int64_t sq_t, int64_t sq_h, const void* prefix_k,
    const void* prefix_v, int64_t sp_b, int64_t sp_l, int64_t sp_h, const void* suffix_k,
    int64_t ssk_n, int64_t ssk_t, int64_t ssk_h, const void* suffix_v, int64_t ssv_n,
    int64_t ssv_t, int64_t ssv_h, const void* prefix_mask, const void* gate, int64_t sg_n,
    int64_t sg_t, int64_t sg_h, void* out, int64_t so_n, int64_t so_t, int64_t so_h, int B,
    int W, int Tq, int Tk, int H, int HK, int L, int D, int dtype, float scale,
    kad_stream_t stream) {
  KAD_REQUIRE(q && suffix_k && suffix_v && out, "null pointer argument");
  KAD_REQUIRE(L == 0 || (prefix_k && prefix_v), "null prefix K/V with L > 0");
  KAD_REQUIRE(B > 0 && W > 0 && Tq > 0 && Tq <= Tk && H > 0 && HK > 0 && H % HK == 0 &&
                  L >= 0 && D > 0,
              "bad dimensions");
  KAD_REQUIRE(dtype == KAD_DTYPE_BF16 || dtype == KAD_DTYPE_F16 || dtype == KAD_DTYPE_F32,
              "unknown dtype code %d", dtype);
  if (D > 256) KAD_UNSUPPORTED("attention supports head dims <= 256, got %d", D);
  const int64_t rows = (int64_t)B * W * Tq * H;
  if (rows > 0x7fffffffLL) KAD_UNSUPPORTED("too many query rows for one launch");
  AttnArgs a{q, prefix_k, prefix_v, suffix_k, suffix_v, gate, (const uint8_t*)prefix_mask, out,
             sq_n, sq_t, sq_h, sp_b, sp_l, sp_h, ssk_n, ssk_t, ssk_h, ssv_n, ssv_t, ssv_h,
             sg_n, sg_t, sg_h, so_n, so_t, so_h, W, Tq, Tk, H, HK, L, D, dtype, scale};
  hipStream_t s = (hipStream_t)stream;
  if (D <= 64)
    hipLaunchKernelGGL(attention_general_kernel<64>, dim3((unsigned)rows), dim3(64), 0, s, a);
  else if (D <= 128)
    hipLaunchKernelGGL(attention_general_kernel<128>, dim3((unsigned)rows), dim3(64), 0, s, a);
  else
    hipLaunchKernelGGL(attention_general_kernel<256>, dim3((unsigned)rows), dim3(64), 0, s, a);
  return kad_launch_status("attention_general_kernel");
}
