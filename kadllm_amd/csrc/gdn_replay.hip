// Gated DeltaNet suffix replay from a request-shared prefix state (gfx950).
//
// Replaces the per-beam / grouped recurrences of the reference
// (src/kadllm/ops.py:139-163, src/kadllm/kernels/gated_delta.py:14-142).
//
// Design.  One workgroup (4 waves) serves one (request b, value head hv) and a
// block of beams.  The request state S0 = state[b,hv] ([K,V] fp32) is read
// from HBM once per workgroup and kept for the whole kernel in registers as
// bf16 hi/lo MFMA A-fragments of S0^T (S0 ~= hi + lo to 2^-16 relative); wave
// w owns value rows [w*V/4, (w+1)*V/4).  Beams are the MFMA N dimension: for
// 16 beams at a time the raw bf16 q_t and k_t rows are loaded straight into
// B-fragments and v_mfma_f32_16x16x32_bf16 gives a_t = S0^T k_t and
// b_t = S0^T q_t exactly up to fp32 accumulation (two passes, hi and lo).
// No per-beam copy of S0 is ever formed.  The recurrence is then finished per
// beam in registers with the factored form (gamma_t = prod_{i<=t} e^{g_i},
// c_j(t) = gamma_t / gamma_j, hats = L2-normalised):
//   recall_t = gamma_t a^_t + sum_{j<t} c_j(t) (k^_j.k^_t) u_j
//   u_t      = beta_t (v_t - recall_t)
//   o_t      = gamma_t b^_t + sum_{j<t} c_j(t) (k^_j.q^_t) u_j + (k^_t.q^_t) u_t
// which is the reference recurrence S <- S e^g; u = beta (v - S^T k);
// S <- S + k u^T; o = S^T q expanded over the suffix (the reference's grouped
// kernel uses the t = T-1 row of the same identity, gated_delta.py:133-134).
// Norms and the T x T Gram terms come from the same fragments with two
// cross-lane reductions.

#include "kad_common.h"

namespace {

constexpr int kTLimit = 8;  // longest suffix the replay handles

template <typename TIN>
struct QKFrag;

template <>
struct QKFrag<bf16_t> {
  bf16x8 hi;
  __device__ __forceinline__ void load(const bf16_t* p, float* f) {
    u32x4 raw = *(const u32x4*)p;
    hi = as_bf16x8(raw);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)hi[i];
  }
};

template <>
struct QKFrag<float> {
  bf16x8 hi, lo;
  __device__ __forceinline__ void load(const float* p, float* f) {
    f32x4 a = *(const f32x4*)p;
    f32x4 b = *(const f32x4*)(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[i] = a[i];
      f[4 + i] = b[i];
    }
    split8(f, hi, lo);
  }
};

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// acc + sum_i a_i b_i over 8 bf16 pairs, as four v_dot2_f32_bf16
__device__ __forceinline__ float dot8_bf16(bf16x8 a, bf16x8 b, float acc) {
#pragma unroll
  for (int p = 0; p < 4; ++p)
    acc = __builtin_amdgcn_fdot2_f32_bf16(bf16x2_t{a[2 * p], a[2 * p + 1]},
                                          bf16x2_t{b[2 * p], b[2 * p + 1]}, acc, false);
  return acc;
}

template <typename TIN>
__device__ __forceinline__ void store4(TIN* p, const float* f);
template <>
__device__ __forceinline__ void store4<bf16_t>(bf16_t* p, const float* f) {
  u32x2 r;
  r[0] = (uint32_t)f2bf(f[0]) | ((uint32_t)f2bf(f[1]) << 16);
  r[1] = (uint32_t)f2bf(f[2]) | ((uint32_t)f2bf(f[3]) << 16);
  *(u32x2*)p = r;
}
template <>
__device__ __forceinline__ void store4<float>(float* p, const float* f) {
  f32x4 r = {f[0], f[1], f[2], f[3]};
  *(f32x4*)p = r;
}

// four consecutive v elements kept as loaded (the conversion waits for the
// load, so it happens only where the values are used)
template <typename TIN>
struct Raw4;
template <>
struct Raw4<bf16_t> {
  u32x2 r;
  __device__ __forceinline__ void load(const bf16_t* p) { r = *(const u32x2*)p; }
  __device__ __forceinline__ void unpack(float* f) const {
    f[0] = __uint_as_float(r[0] << 16);
    f[1] = __uint_as_float(r[0] & 0xffff0000u);
    f[2] = __uint_as_float(r[1] << 16);
    f[3] = __uint_as_float(r[1] & 0xffff0000u);
  }
};
template <>
struct Raw4<float> {
  f32x4 r;
  __device__ __forceinline__ void load(const float* p) { r = *(const f32x4*)p; }
  __device__ __forceinline__ void unpack(float* f) const {
    f[0] = r[0];
    f[1] = r[1];
    f[2] = r[2];
    f[3] = r[3];
  }
};

// one-token suffixes fit three workgroups per CU (150 registers), whose
// extra waves hide the per-group load latency (5% faster than two)
template <int KD, int VD, typename TIN, int kTMax>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kTMax == 1 ? 3 : 1, 8)))
void gdn_replay_kernel(
    const TIN* __restrict__ q, const TIN* __restrict__ k, const TIN* __restrict__ v,
    int64_t ld_qk, int64_t ld_v, const void* __restrict__ gdecay, int gate_dtype,
    const void* __restrict__ beta, int beta_dtype, int64_t ld_gate,
    const void* __restrict__ state, int state_dtype, TIN* __restrict__ out, int64_t ld_out,
    int W, int T_rt, int H, int HV, float scale, int beams_per_block, int nbb) {
  // each suffix length has its own instantiation (launched only with
  // T == kTMax), so the per-token tests and the row arithmetic see a constant
  constexpr int T = kTMax;
  (void)T_rt;
  constexpr int KSTEPS = KD / 32;
  constexpr int VROWS = VD / 4;
  constexpr int MT = VROWS / 16;
  constexpr bool kSplitB = sizeof(TIN) == 4;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lid = xcd_logical_id(blockIdx.x, gridDim.x);
  const int bb = lid % nbb;
  const int rh = lid / nbb;
  const int hv = rh % HV;
  const int b = rh / HV;
  const int h = hv / (HV / H);
  const int v0 = wave * VROWS;
  const int col = lane & 15;   // beam within the 16-beam group (MFMA N index)
  const int quad = lane >> 4;  // 0..3

  // ---- S0^T fragments, hi/lo bf16, held in registers for the whole kernel
  bf16x8 a_hi[MT][KSTEPS], a_lo[MT][KSTEPS];
  {
    const int64_t sbase = ((int64_t)b * HV + hv) * KD * VD;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const int vrow = v0 + mt * 16 + col;
        const int kc = ks * 32 + quad * 8;
        float x[8];
        if (state_dtype == KAD_DTYPE_F32) {
          // the common case without the per-element dtype branches, so that
          // all 64 loads go out back to back
#pragma unroll
          for (int i = 0; i < 8; ++i)
            x[i] = ((const float*)state)[sbase + (int64_t)(kc + i) * VD + vrow];
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i)
            x[i] = load_as_float(state, sbase + (int64_t)(kc + i) * VD + vrow, state_dtype);
        }
        split8(x, a_hi[mt][ks], a_lo[mt][ks]);
      }
    }
  }

  const int n_begin = bb * beams_per_block;
  const int n_end = min(W, n_begin + beams_per_block);

  for (int g0 = n_begin; g0 < n_end; g0 += 16) {
    const int nl = g0 + col;
    const bool valid = nl < n_end;
    const int64_t n = (int64_t)b * W + (valid ? nl : n_begin);

    // every load of the group goes out first (v, then q and k, then the
    // gates), so the group costs one memory round trip
    Raw4<TIN> vraw[kTMax][MT];
#pragma unroll
    for (int t = 0; t < kTMax; ++t)
      if (t < T)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          vraw[t][mt].load(v + (n * T + t) * ld_v + (int64_t)hv * VD + v0 + mt * 16 + quad * 4);

    f32x4 acc_q[kTMax][MT], acc_k[kTMax][MT];
#pragma unroll
    for (int t = 0; t < kTMax; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc_q[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc_k[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    float qq[kTMax], kk[kTMax], kkx[kTMax][kTMax], kqx[kTMax][kTMax];
#pragma unroll
    for (int t = 0; t < kTMax; ++t) {
      qq[t] = 0.f;
      kk[t] = 0.f;
#pragma unroll
      for (int j = 0; j < kTMax; ++j) {
        kkx[j][t] = 0.f;
        kqx[j][t] = 0.f;
      }
    }

    // q and k of every K step are loaded up front too where the registers
    // allow it (one token); longer suffixes load them step by step, which
    // keeps two waves per SIMD
    constexpr bool kHoistQK = kTMax == 1;
    constexpr int KSH = kHoistQK ? KSTEPS : 1;
    QKFrag<TIN> fq_all[KSH][kTMax], fk_all[KSH][kTMax];
    float xq_all[KSH][kTMax][8], xk_all[KSH][kTMax][8];
    auto load_qk = [&](int ks, int slot) {
#pragma unroll
      for (int t = 0; t < kTMax; ++t)
        if (t < T) {
          const int64_t row = (n * T + t) * ld_qk + (int64_t)h * KD + ks * 32 + quad * 8;
          fq_all[slot][t].load(q + row, xq_all[slot][t]);
          fk_all[slot][t].load(k + row, xk_all[slot][t]);
        }
    };
    if constexpr (kHoistQK) {
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) load_qk(ks, ks);
    }
    float et[kTMax], bt[kTMax];
#pragma unroll
    for (int t = 0; t < kTMax; ++t) {
      if (t < T) {
        const int64_t gi = (n * T + t) * ld_gate + hv;
        et[t] = load_as_float(gdecay, gi, gate_dtype);
        bt[t] = load_as_float(beta, gi, beta_dtype);
      } else {
        et[t] = 0.f;
        bt[t] = 0.f;
      }
    }

#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const int slot = kHoistQK ? ks : 0;
      if constexpr (!kHoistQK) load_qk(ks, 0);
      QKFrag<TIN>(&fq)[kTMax] = fq_all[slot];
      QKFrag<TIN>(&fk)[kTMax] = fk_all[slot];
      float(&xq)[kTMax][8] = xq_all[slot];
      float(&xk)[kTMax][8] = xk_all[slot];
#pragma unroll
      for (int t = 0; t < kTMax; ++t) {
        if (t < T) {
          if constexpr (!kSplitB) {
            // bf16 rows: packed dot2 (products exact, fp32 sums) on the raw fragments
            qq[t] = dot8_bf16(fq[t].hi, fq[t].hi, qq[t]);
            kk[t] = dot8_bf16(fk[t].hi, fk[t].hi, kk[t]);
#pragma unroll
            for (int j = 0; j <= t; ++j) {
              kqx[j][t] = dot8_bf16(fk[j].hi, fq[t].hi, kqx[j][t]);
              if (j < t) kkx[j][t] = dot8_bf16(fk[j].hi, fk[t].hi, kkx[j][t]);
            }
          } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              qq[t] += xq[t][i] * xq[t][i];
              kk[t] += xk[t][i] * xk[t][i];
            }
#pragma unroll
            for (int j = 0; j <= t; ++j) {
#pragma unroll
              for (int i = 0; i < 8; ++i) {
                kqx[j][t] += xk[j][i] * xq[t][i];
                if (j < t) kkx[j][t] += xk[j][i] * xk[t][i];
              }
            }
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            acc_k[t][mt] = mfma16x16x32(a_hi[mt][ks], fk[t].hi, acc_k[t][mt]);
            acc_k[t][mt] = mfma16x16x32(a_lo[mt][ks], fk[t].hi, acc_k[t][mt]);
            acc_q[t][mt] = mfma16x16x32(a_hi[mt][ks], fq[t].hi, acc_q[t][mt]);
            acc_q[t][mt] = mfma16x16x32(a_lo[mt][ks], fq[t].hi, acc_q[t][mt]);
            if constexpr (kSplitB) {
              acc_k[t][mt] = mfma16x16x32(a_hi[mt][ks], fk[t].lo, acc_k[t][mt]);
              acc_q[t][mt] = mfma16x16x32(a_hi[mt][ks], fq[t].lo, acc_q[t][mt]);
            }
          }
        }
      }
    }

    // full 128-element dot products: sum the 4 lanes (quad 0..3) of each beam
#pragma unroll
    for (int t = 0; t < kTMax; ++t) {
      qq[t] = add_xor32(add_xor16(qq[t]));
      kk[t] = add_xor32(add_xor16(kk[t]));
#pragma unroll
      for (int j = 0; j <= t; ++j) {
        kqx[j][t] = add_xor32(add_xor16(kqx[j][t]));
        if (j < t) kkx[j][t] = add_xor32(add_xor16(kkx[j][t]));
      }
    }

    float rk[kTMax], rq[kTMax];
#pragma unroll
    for (int t = 0; t < kTMax; ++t) {
      rk[t] = 1.0f / sqrtf(kk[t] + 1e-6f);
      rq[t] = scale / sqrtf(qq[t] + 1e-6f);
      et[t] = t < T ? expf(et[t]) : 1.f;
    }

    float u[kTMax][MT][4];
    float c[kTMax];
    float gam = 1.f;
#pragma unroll
    for (int t = 0; t < kTMax; ++t) {
      if (t < T) {
        gam *= et[t];
#pragma unroll
        for (int j = 0; j < t; ++j) c[j] *= et[t];
        const int64_t vrow_base = (n * T + t);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int vr = v0 + mt * 16 + quad * 4;
          float vt[4], ov[4];
          vraw[t][mt].unpack(vt);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float recall = gam * (acc_k[t][mt][i] * rk[t]);
#pragma unroll
            for (int j = 0; j < t; ++j) recall += c[j] * (kkx[j][t] * rk[j] * rk[t]) * u[j][mt][i];
            const float ut = bt[t] * (vt[i] - recall);
            u[t][mt][i] = ut;
            float o = gam * (acc_q[t][mt][i] * rq[t]);
#pragma unroll
            for (int j = 0; j < t; ++j) o += c[j] * (kqx[j][t] * rk[j] * rq[t]) * u[j][mt][i];
            o += (kqx[t][t] * rk[t] * rq[t]) * ut;
            ov[i] = o;
          }
          if (valid) store4<TIN>(out + vrow_base * ld_out + (int64_t)hv * VD + vr, ov);
        }
        c[t] = 1.f;
      }
    }
  }
}

// The same replay for the decode shapes (bf16, K = V = 128, up to 4 suffix
// tokens, 16-beam groups that are all full), with each group's q, k and v
// rows staged in LDS instead of loaded by every wave: one set of DMA loads
// (global_load_lds, 16 bytes per lane) per workgroup fills a stage, issued
// NS - 1 groups ahead of its use, so the groups' load latency overlaps the
// products of the groups before (an instrumented copy of the register-load
// kernel spent about 5,000 of 7,000 cycles per one-token group waiting for
// its loads).  Rows are 256 bytes with their 16-byte chunks XOR-swizzled by
// the beam index, so a fragment read of 16 beams touches 16 distinct bank
// groups.  The arithmetic is the register kernel's, operation for operation,
// so the outputs are bit-identical.
typedef __attribute__((address_space(1))) void replay_global_t;
typedef __attribute__((address_space(3))) void replay_lds_t;

// The fused form (CONV) takes q, k and v before the depthwise causal conv +
// SiLU of the decode (the column ranges of the projection rows) and applies
// the conv in LDS as each group's rows land, with the arithmetic of
// conv_suffix_vec_bf16 operation for operation (so the outputs are those of
// kad_causal_conv_suffix followed by the replay, bit for bit); the conv output
// never goes to HBM.  The prefix taps enter as per-channel partial sums: for
// token t the window is [x_{t-3} .. x_t] with x_{-3..-1} the prefix taps, and
// c_t is the chain of the window's tap terms (w_0 x_{t-3} + ..., in the conv
// kernel's order), which the suffix terms then continue.
struct ConvArgs {
  const bf16_t* state;     // prefix conv inputs [B, C, hist] (strides ss_b, ss_c, ss_t)
  int64_t ss_b, ss_c, ss_t;
  int hist;                // the taps are slots hist - 3 .. hist - 1
  const bf16_t* w;         // [C, 4], C the conv channels (q | k | v)
};
// per 8-channel chunk of the conv table: w_3 (bf16 x 8), then for T = 2 w_2;
// c_0 (fp32 x 8), then for T = 2 c_1
template <int T>
struct ConvTab {
  static constexpr int chunks = 48;                    // q, k and v of one head, 8 channels each
  static constexpr int w_bytes = 16 * T, c_bytes = 32 * T;
  static constexpr int chunk_bytes = w_bytes + c_bytes;
  static constexpr int bytes = chunks * chunk_bytes;
};

// The gated form (GATED, with CONV) passes each output row of a value head
// through the layer's gated RMSNorm on its way out, with the arithmetic of
// rmsnorm_gated_kernel<16, 1>: the row's 8-element pieces summed as one fma
// chain each (a piece spans two lanes here: the first four squares' chain is
// handed on by a lane shuffle), the 16 piece sums combined in that kernel's
// butterfly order through LDS, so y equals the replay followed by
// kad_rmsnorm_gated bit for bit.  Only the tokens from t_first on are
// normed and written (the last token only in the incremental decode, whose
// earlier tokens' outputs nothing reads): out row n * (T - t_first) + t - t_first.
struct GateOutArgs {
  const bf16_t* z;     // gate rows: (n, t) at z + (n*T + t) * ldz + hv*V
  int64_t ldz;
  const bf16_t* w;     // norm weight [V]
  float eps;
  int t_first;
};

// Parent-row form (PAR, with LAST): the earlier tokens' rows are read in
// place from the parent level's cached projection rows, through each beam's
// parent index, and the new token's from a compact buffer of one row per
// beam, so the search's last level gathers no rows.
struct ParentRows {
  const bf16_t* prev;       // parent rows: (b*Wp + parent)*(T-1) + t, stride ld_prev
  int64_t ld_prev;
  const int64_t* parents;   // [B, W], clamped to [0, Wp)
  int Wp;
  const bf16_t* cur;        // new rows: b*W + beam, stride ld_cur
  int64_t ld_cur;
};

// LAST (with GATED, last token only): the earlier tokens' q, whose outputs
// nothing reads, enter no product (their k and v still update the state)
template <int T, int NS, bool CONV, bool GATED = false, bool LAST = false, bool PAR = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(T == 1 ? 3 : (T == 4 ? 1 : 2), 8)))
void gdn_replay_lds_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ k,
                           const bf16_t* __restrict__ v, int64_t ld_qk, int64_t ld_v,
                           const void* __restrict__ gdecay, int gate_dtype,
                           const void* __restrict__ beta, int beta_dtype, int64_t ld_gate,
                           const void* __restrict__ state, int state_dtype,
                           bf16_t* __restrict__ out, int64_t ld_out, int W, int H, int HV,
                           float scale, int beams_per_block, int nbb, ConvArgs cv,
                           GateOutArgs go, ParentRows pr) {
  constexpr int KD = 128, VD = 128;
  constexpr int KSTEPS = KD / 32;
  constexpr int VROWS = VD / 4;
  constexpr int MT = VROWS / 16;
  constexpr int ROWS = 16 * T;               // (beam, token) rows of a group
  constexpr int BLK = ROWS * 256;            // bytes of one q, k or v block
  constexpr int STAGE = 3 * BLK + 512;      // + the gates: 64 fp32 decays, 64 beta words
  static_assert(!CONV || T <= 2, "the fused conv takes one- and two-token suffixes");
  static_assert(!GATED || CONV, "the gated output comes with the fused conv");
  static_assert(!LAST || GATED, "the last-token form is a gated form");
  static_assert(!PAR || (LAST && T >= 2), "the parent-row form is a last-token form");
  constexpr int TQ = LAST ? T - 1 : 0;   // the first token whose q is used
  constexpr int TAB = CONV ? ConvTab<T>::bytes : 0;
  // [normed token][beam][piece] row-sum pieces (one token in the last-token form)
  constexpr int PSUM = GATED ? (LAST ? 1 : T) * 16 * 16 * 4 : 0;
  constexpr int PARB = PAR ? 256 * 4 : 0;   // the block's parent indices
  __shared__ __attribute__((aligned(16))) uint8_t stage_buf[NS * STAGE + TAB + PSUM + PARB];
  uint8_t* const tab = stage_buf + NS * STAGE;
  float* const psum = (float*)(stage_buf + NS * STAGE + TAB);
  int* const par_lds = (int*)(stage_buf + NS * STAGE + TAB + PSUM);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lid = xcd_logical_id(blockIdx.x, gridDim.x);
  const int bb = lid % nbb;
  const int rh = lid / nbb;
  const int hv = rh % HV;
  const int b = rh / HV;
  const int h = hv / (HV / H);
  const int v0 = wave * VROWS;
  const int col = lane & 15;   // beam within the 16-beam group (MFMA N index)
  const int quad = lane >> 4;  // 0..3

  const int n_begin = bb * beams_per_block;
  const int n_end = min(W, n_begin + beams_per_block);
  const int ngroups = (n_end - n_begin) / 16;

  // DMA of group gi into stage s: wave w moves 1 KB pieces w*T .. w*T+T-1 of
  // each block; lane L of piece I fills row 4I + L/16, swizzled chunk L%16
  auto dma_group = [&](int gi, int s) {
    const int64_t row0 = ((int64_t)b * W + n_begin + gi * 16) * T;
    uint8_t* sb = stage_buf + s * STAGE;
    const int w = __builtin_amdgcn_readfirstlane(wave);
#pragma unroll
    for (int j = 0; j < T; ++j) {
      const int I = w * T + j;
      const int r = 4 * I + (lane >> 4);
      const int c = (lane & 15) ^ ((r / T) & 15);
      const bf16_t *qs, *ks, *vs;
      if constexpr (PAR) {
        // (beam, token) of row r: an earlier token from the parent's cached
        // row, the new token from the compact buffer
        const int beam = gi * 16 + r / T, t = r % T;
        const bf16_t* base =
            t < T - 1 ? pr.prev + ((int64_t)(b * pr.Wp + par_lds[beam]) * (T - 1) + t) * pr.ld_prev
                      : pr.cur + ((int64_t)b * W + n_begin + beam) * pr.ld_cur;
        qs = base + (int64_t)h * KD + c * 8;
        ks = base + (int64_t)(H + h) * KD + c * 8;
        vs = base + (int64_t)2 * H * KD + (int64_t)hv * VD + c * 8;
      } else {
        const int64_t qrow = (row0 + r) * ld_qk + (int64_t)h * KD + c * 8;
        const int64_t vrow = (row0 + r) * ld_v + (int64_t)hv * VD + c * 8;
        qs = q + qrow;
        ks = k + qrow;
        vs = v + vrow;
      }
      __builtin_amdgcn_global_load_lds((replay_global_t*)qs, (replay_lds_t*)(sb + I * 1024), 16,
                                       0, 0);
      __builtin_amdgcn_global_load_lds((replay_global_t*)ks,
                                       (replay_lds_t*)(sb + BLK + I * 1024), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((replay_global_t*)vs,
                                       (replay_lds_t*)(sb + 2 * BLK + I * 1024), 16, 0, 0);
    }
    // the group's gates, lane r = (beam, token) row: wave 0 the fp32 log
    // decays, wave 1 the 4-byte words holding the bf16 betas (rows have an
    // even stride, so a beta's half of its word is hv % 2)
    if (w < 2 && lane < ROWS) {
      const int64_t gix = (row0 + lane) * ld_gate + hv;
      const void* src = w == 0 ? (const void*)((const float*)gdecay + gix)
                               : (const void*)((const uint32_t*)beta + (gix >> 1));
      __builtin_amdgcn_global_load_lds((replay_global_t*)src,
                                       (replay_lds_t*)(sb + 3 * BLK + w * 256), 4, 0, 0);
    }
  };
  // the conv table of this head's 384 channels (q, k, v), one channel per
  // thread and round: its inputs are loaded here, ahead of the groups' DMA and
  // the state, and the table is formed once the state is in registers
  constexpr int kTabRounds = CONV ? (ConvTab<T>::chunks * 8 + 255) / 256 : 0;
  uint2 tab_w[kTabRounds > 0 ? kTabRounds : 1];
  float tab_tap[kTabRounds > 0 ? kTabRounds : 1][3];
  auto tab_channel = [&](int ci) {
    const int chunk = ci >> 3, e = ci & 7, blk = chunk >> 4, c8 = (chunk & 15) * 8 + e;
    return blk == 0 ? h * KD + c8 : (blk == 1 ? (H + h) * KD + c8 : 2 * H * KD + hv * VD + c8);
  };
  if constexpr (CONV) {
#pragma unroll
    for (int j = 0; j < kTabRounds; ++j) {
      const int ci = threadIdx.x + 256 * j;
      if (ci < ConvTab<T>::chunks * 8) {
        const int gc = tab_channel(ci);
        tab_w[j] = *(const uint2*)(cv.w + (int64_t)gc * 4);
        const bf16_t* sp = cv.state + (int64_t)b * cv.ss_b + (int64_t)gc * cv.ss_c;
#pragma unroll
        for (int i = 0; i < 3; ++i) tab_tap[j][i] = bf2f(sp[(int64_t)(cv.hist - 3 + i) * cv.ss_t]);
      }
    }
  }
  if constexpr (PAR) {
    // the block's parent indices, clamped (their loads precede every DMA)
    for (int i = threadIdx.x; i < n_end - n_begin; i += 256) {
      const int64_t p0 = pr.parents[(int64_t)b * W + n_begin + i];
      par_lds[i] = (int)(p0 < 0 ? 0 : (p0 >= pr.Wp ? pr.Wp - 1 : p0));
    }
    __syncthreads();
  }
  // the first NS - 1 groups' loads go out before the state's, so they land
  // meanwhile
#pragma unroll
  for (int d = 0; d < NS - 1; ++d)
    if (d < ngroups) dma_group(d, d);

  // ---- S0^T fragments, hi/lo bf16, held in registers for the whole kernel
  bf16x8 a_hi[MT][KSTEPS], a_lo[MT][KSTEPS];
  {
    const int64_t sbase = ((int64_t)b * HV + hv) * KD * VD;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
      for (int ks = 0; ks < KSTEPS; ++ks) {
        const int vrow = v0 + mt * 16 + col;
        const int kc = ks * 32 + quad * 8;
        float x[8];
        if (state_dtype == KAD_DTYPE_F32) {
#pragma unroll
          for (int i = 0; i < 8; ++i)
            x[i] = ((const float*)state)[sbase + (int64_t)(kc + i) * VD + vrow];
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i)
            x[i] = load_as_float(state, sbase + (int64_t)(kc + i) * VD + vrow, state_dtype);
        }
        split8(x, a_hi[mt][ks], a_lo[mt][ks]);
      }
    }
  }

  if constexpr (CONV) {
#pragma unroll
    for (int j = 0; j < kTabRounds; ++j) {
      const int ci = threadIdx.x + 256 * j;
      if (ci < ConvTab<T>::chunks * 8) {
        const int chunk = ci >> 3, e = ci & 7;
        const uint2 wr = tab_w[j];
        const float w4[4] = {__uint_as_float(wr.x << 16), __uint_as_float(wr.x & 0xffff0000u),
                             __uint_as_float(wr.y << 16), __uint_as_float(wr.y & 0xffff0000u)};
        uint8_t* tc = tab + chunk * ConvTab<T>::chunk_bytes;
#pragma unroll
        for (int t = 0; t < T; ++t) {
          // c_t: the window's tap terms i < 3 - t, in the conv kernel's order
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < 3 - t; ++i) acc += w4[i] * tab_tap[j][t + i];
          ((float*)(tc + ConvTab<T>::w_bytes + t * 32))[e] = acc;
          // w_3 for token 0's slot, w_2 for token 1's
          ((bf16_t*)(tc + t * 16))[e] = t == 0 ? (bf16_t)(wr.y >> 16) : (bf16_t)(wr.y & 0xffffu);
        }
      }
    }
    // the table's stores complete before the first group's barrier
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
  // the norm weights of this lane's 8 value rows (v0 + mt*16 + quad*4 .. +3)
  u32x2 gw[GATED ? MT : 1];
  if constexpr (GATED) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) gw[mt] = *(const u32x2*)(go.w + v0 + mt * 16 + quad * 4);
  }

  // One group.  At its start, group gi's loads (all DMA into LDS, issued
  // NS - 1 groups earlier) must have landed.  The only loads issued after
  // them are the groups' in between: with NS = 3, group gi + 1's (at least 3T
  // per lane), which may stay outstanding; with NS = 2, none.  Loads complete
  // in issue order, so at most 3T outstanding operations leaves every older
  // load complete, whatever the output stores in between have done.
  auto group = [&](int gi) {
    if (NS == 3 && gi + 1 < ngroups)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * T) : "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // every wave's part of the stage is in, and every wave is done with the
    // stage the next DMA refills; a plain s_barrier, which (unlike
    // __syncthreads) leaves the prefetches in flight
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const int s = gi % NS;
    // the gate rows of the normed tokens, issued before the next DMA so that
    // waiting for them does not wait for it
    u32x2 zg[GATED ? T : 1][GATED ? MT : 1];
    if constexpr (GATED) {
      const int64_t nz = (int64_t)b * W + n_begin + gi * 16 + col;
#pragma unroll
      for (int t = 0; t < T; ++t)
        if (t >= go.t_first) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            zg[t][mt] = *(const u32x2*)(go.z + (PAR ? nz : nz * T + t) * go.ldz +
                                        (int64_t)hv * VD + v0 + mt * 16 + quad * 4);
        }
    }
    if (gi + NS - 1 < ngroups) dma_group(gi + NS - 1, (gi + NS - 1) % NS);

    if constexpr (CONV) {
      // conv + SiLU of the stage's q, k and v rows in place: 16 beams x 48
      // chunks, three (beam, chunk) items per thread, each over the T tokens
      uint8_t* st = stage_buf + s * STAGE;
#pragma unroll
      for (int u = 0; u < 3; ++u) {
        const int item = threadIdx.x + 256 * u;
        const int beam = item / ConvTab<T>::chunks, chunk = item % ConvTab<T>::chunks;
        uint8_t* rp = st + (chunk >> 4) * BLK + beam * T * 256 + (((chunk & 15) ^ beam) * 16);
        const uint8_t* tc = tab + chunk * ConvTab<T>::chunk_bytes;
        u32x4 x[T];
#pragma unroll
        for (int t = 0; t < T; ++t) x[t] = *(const u32x4*)(rp + t * 256);
        const u32x4 w3r = *(const u32x4*)tc;
        u32x4 w2r = u32x4{0u, 0u, 0u, 0u};
        if constexpr (T == 2) w2r = *(const u32x4*)(tc + 16);
        const float* ct = (const float*)(tc + ConvTab<T>::w_bytes);
        u32x4 y[T];   // token 1 reads token 0's inputs: stores after every token
#pragma unroll
        for (int t = 0; t < T; ++t) {
#pragma unroll
          for (int pr = 0; pr < 4; ++pr) {
            float a[2];
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
              const int e = 2 * pr + hh;
              auto lo16 = [&](uint32_t wv) { return __uint_as_float(hh ? (wv & 0xffff0000u) : (wv << 16)); };
              float acc = ct[t * 8 + e];
              if (t == 1) acc += lo16(w2r[pr]) * lo16(x[0][pr]);
              acc += lo16(w3r[pr]) * lo16(x[t][pr]);
              a[hh] = acc;
            }
            const uint32_t pk = pack_bf16x2(a[0], a[1]);
            y[t][pr] = pack_bf16x2(silu_fast(__uint_as_float(pk << 16)),
                                   silu_fast(__uint_as_float(pk & 0xffff0000u)));
          }
        }
#pragma unroll
        for (int t = 0; t < T; ++t) *(u32x4*)(rp + t * 256) = y[t];
      }
      // every wave's conv outputs in place before any fragment read
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
    }

    const uint8_t* sq = stage_buf + s * STAGE;
    const uint8_t* sk = sq + BLK;
    const uint8_t* sv = sq + 2 * BLK;
    const int g0 = n_begin + gi * 16;
    const int64_t n = (int64_t)b * W + g0 + col;

    f32x4 acc_q[T][MT], acc_k[T][MT];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc_q[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        acc_k[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    float qq[T], kk[T], kkx[T][T], kqx[T][T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      qq[t] = 0.f;
      kk[t] = 0.f;
#pragma unroll
      for (int j = 0; j < T; ++j) {
        kkx[j][t] = 0.f;
        kqx[j][t] = 0.f;
      }
    }
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      bf16x8 fq[T], fk[T];
#pragma unroll
      for (int t = 0; t < T; ++t) {
        const int r = col * T + t;
        const int off = r * 256 + (((ks * 4 + quad) ^ (col & 15)) * 16);
        if (t >= TQ) fq[t] = *(const bf16x8*)(sq + off);
        fk[t] = *(const bf16x8*)(sk + off);
      }
#pragma unroll
      for (int t = 0; t < T; ++t) {
        if (t >= TQ) qq[t] = dot8_bf16(fq[t], fq[t], qq[t]);
        kk[t] = dot8_bf16(fk[t], fk[t], kk[t]);
#pragma unroll
        for (int j = 0; j <= t; ++j) {
          if (t >= TQ) kqx[j][t] = dot8_bf16(fk[j], fq[t], kqx[j][t]);
          if (j < t) kkx[j][t] = dot8_bf16(fk[j], fk[t], kkx[j][t]);
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          acc_k[t][mt] = mfma16x16x32(a_hi[mt][ks], fk[t], acc_k[t][mt]);
          acc_k[t][mt] = mfma16x16x32(a_lo[mt][ks], fk[t], acc_k[t][mt]);
          if (t >= TQ) {
            acc_q[t][mt] = mfma16x16x32(a_hi[mt][ks], fq[t], acc_q[t][mt]);
            acc_q[t][mt] = mfma16x16x32(a_lo[mt][ks], fq[t], acc_q[t][mt]);
          }
        }
      }
    }
#pragma unroll
    for (int t = 0; t < T; ++t) {
      if (t >= TQ) qq[t] = add_xor32(add_xor16(qq[t]));
      kk[t] = add_xor32(add_xor16(kk[t]));
#pragma unroll
      for (int j = 0; j <= t; ++j) {
        if (t >= TQ) kqx[j][t] = add_xor32(add_xor16(kqx[j][t]));
        if (j < t) kkx[j][t] = add_xor32(add_xor16(kkx[j][t]));
      }
    }

    float rk[T], rq[T], et[T], btf[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
      rk[t] = 1.0f / sqrtf(kk[t] + 1e-6f);
      rq[t] = t >= TQ ? scale / sqrtf(qq[t] + 1e-6f) : 0.f;
      const uint8_t* sg = stage_buf + s * STAGE + 3 * BLK;
      et[t] = expf(((const float*)sg)[col * T + t]);
      const uint32_t bw = ((const uint32_t*)(sg + 256))[col * T + t];
      btf[t] = __uint_as_float((hv & 1) ? (bw & 0xffff0000u) : (bw << 16));
    }

    float og[MT][4];   // a token's outputs, for the gated form
    // gated RMSNorm of token t's rows and their store (see GateOutArgs)
    auto gated_out = [&](int t, const float (&o)[MT][4], const u32x2 (&zt)[MT], int64_t nrow) {
      float f[MT][4];
      // one buffer per normed token: no barrier between tokens
      float* ps = psum + (LAST ? 0 : t * 256);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        // o rounded to bf16 as the unfused path stores it; this lane's four
        // squares continue the chain of piece wave*4 + mt*2 + quad/2 that
        // the lane 16 down began (odd quads), or begin it (even quads)
#pragma unroll
        for (int i = 0; i < 4; ++i) f[mt][i] = round_bf(o[mt][i]);
        float h = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) h += f[mt][i] * f[mt][i];
        float pc = __shfl_up(h, 16, 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) pc += f[mt][i] * f[mt][i];
        if (quad & 1) ps[col * 16 + wave * 4 + mt * 2 + (quad >> 1)] = pc;
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      // the 16 pieces in rmsnorm_gated_kernel's butterfly order (partners
      // xor 8, then 4, 2, 1)
      float p[16];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 v4 = *(const f32x4*)(ps + col * 16 + j * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) p[j * 4 + i] = v4[i];
      }
      float s1[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) s1[i] = p[i] + p[i + 8];
      float s2[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) s2[i] = s1[i] + s1[i + 4];
      const float s3a = s2[0] + s2[2], s3b = s2[1] + s2[3];
      const float ss = s3a + s3b;
      const float r = 1.0f / sqrtf(ss / (float)VD + go.eps);
      const int64_t orow = nrow * (T - go.t_first) + (t - go.t_first);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t wb = gw[mt][i >> 1], zb = zt[mt][i >> 1];
          const float wv = __uint_as_float((i & 1) ? (wb & 0xffff0000u) : (wb << 16));
          const float zv = __uint_as_float((i & 1) ? (zb & 0xffff0000u) : (zb << 16));
          const float nrm = round_bf(f[mt][i] * r);
          const float wn = round_bf(wv * nrm);
          y[i] = wn * silu_fast(zv);
        }
        const u32x2 yv = {pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
        *(u32x2*)(out + orow * ld_out + (int64_t)hv * VD + v0 + mt * 16 + quad * 4) = yv;
      }
    };
    float u[T][MT][4];
    float c[T];
    float gam = 1.f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
      gam *= et[t];
#pragma unroll
      for (int j = 0; j < t; ++j) c[j] *= et[t];
      const int r = col * T + t;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int e = v0 + mt * 16 + quad * 4;
        const u32x2 raw =
            *(const u32x2*)(sv + r * 256 + (((e >> 3) ^ (col & 15)) * 16) + (e & 7) * 2);
        float vt[4], ov[4];
        vt[0] = __uint_as_float(raw[0] << 16);
        vt[1] = __uint_as_float(raw[0] & 0xffff0000u);
        vt[2] = __uint_as_float(raw[1] << 16);
        vt[3] = __uint_as_float(raw[1] & 0xffff0000u);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float recall = gam * (acc_k[t][mt][i] * rk[t]);
#pragma unroll
          for (int j = 0; j < t; ++j) recall += c[j] * (kkx[j][t] * rk[j] * rk[t]) * u[j][mt][i];
          const float ut = btf[t] * (vt[i] - recall);
          u[t][mt][i] = ut;
          if (t < TQ) continue;   // an output nothing reads
          float o = gam * (acc_q[t][mt][i] * rq[t]);
#pragma unroll
          for (int j = 0; j < t; ++j) o += c[j] * (kqx[j][t] * rk[j] * rq[t]) * u[j][mt][i];
          o += (kqx[t][t] * rk[t] * rq[t]) * ut;
          ov[i] = o;
        }
        if (t < TQ) continue;
        if constexpr (GATED) {
#pragma unroll
          for (int i = 0; i < 4; ++i) og[mt][i] = ov[i];
        } else {
          store4<bf16_t>(out + (n * T + t) * ld_out + (int64_t)hv * VD + e, ov);
        }
      }
      if constexpr (GATED) {
        if (t >= go.t_first) gated_out(t, og, zg[t], n);
      }
      c[t] = 1.f;
    }
  };
  for (int gi = 0; gi < ngroups; ++gi) group(gi);
}

template <int KD, int VD, typename TIN>
int launch_replay(const void* q, const void* k, const void* v, int64_t ld_qk, int64_t ld_v,
                  const void* g, int gdt, const void* beta, int bdt, int64_t ld_gate,
                  const void* state, int sdt, void* out, int64_t ld_out, int B, int W,
                  int T, int H, int HV, float scale, hipStream_t stream) {
  int bpb = W >= 256 ? 128 : ((W + 15) / 16) * 16;
  if (bpb > 128) bpb = 128;
  // the staged kernel takes a request's beams in one workgroup up to 256, so
  // the state prologue is paid once per (request, head): two-token suffixes
  // at 256 beams 7% faster than two workgroups of 128
  if (KD == 128 && VD == 128 && sizeof(TIN) == 2 && T <= 4 && W % 16 == 0 && W <= 256) bpb = W;
  const int nbb = (int)kad_cdiv(W, bpb);
  const int64_t nblocks = (int64_t)B * HV * nbb;
  if (nblocks > 0x7fffffff) {
    kad_set_error("gdn replay grid too large");
    return KAD_ERR_UNSUPPORTED;
  }
  // the LDS-staged kernel for the decode shapes (all groups full, 16-byte rows)
  if constexpr (KD == 128 && VD == 128 && sizeof(TIN) == 2) {
    const bool staged = T <= 4 && W % 16 == 0 && bpb % 16 == 0 && gdt == KAD_DTYPE_F32 &&
                        bdt == KAD_DTYPE_BF16 && ld_gate % 2 == 0 &&
                        ((uintptr_t)beta % 4) == 0 && ((uintptr_t)g % 4) == 0 && ld_qk % 8 == 0 &&
                        ld_v % 8 == 0 && ((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) % 16 == 0;
    if (staged) {
#define KAD_REPLAY_LDS(TT, NS)                                                                \
  if (T == TT) {                                                                              \
    hipLaunchKernelGGL((gdn_replay_lds_kernel<TT, NS, false>), dim3((unsigned)nblocks),       \
                       dim3(256), 0, stream, (const bf16_t*)q, (const bf16_t*)k,              \
                       (const bf16_t*)v, ld_qk, ld_v, g, gdt, beta, bdt, ld_gate, state, sdt, \
                       (bf16_t*)out, ld_out, W, H, HV, scale, bpb, nbb, ConvArgs{},           \
                       GateOutArgs{}, ParentRows{});                                          \
    return kad_launch_status("gdn_replay_lds_kernel");                                        \
  }
      KAD_REPLAY_LDS(1, 3)
      KAD_REPLAY_LDS(2, 3)
      KAD_REPLAY_LDS(3, 2)
      KAD_REPLAY_LDS(4, 2)
#undef KAD_REPLAY_LDS
    }
  }
  // one instantiation per suffix length: the per-token arrays then hold only
  // T entries, which keeps the register count (and so the occupancy) down
#define KAD_REPLAY_T(TT)                                                                      \
  if (T == TT) {                                                                              \
    hipLaunchKernelGGL((gdn_replay_kernel<KD, VD, TIN, TT>), dim3((unsigned)nblocks),          \
                       dim3(256), 0, stream, (const TIN*)q, (const TIN*)k, (const TIN*)v,     \
                       ld_qk, ld_v, g, gdt, beta, bdt, ld_gate, state, sdt, (TIN*)out, ld_out, \
                       W, T, H, HV, scale, bpb, nbb);                                         \
    return kad_launch_status("gdn_replay_kernel");                                            \
  }
  KAD_REPLAY_T(1)
  KAD_REPLAY_T(2)
  KAD_REPLAY_T(3)
  KAD_REPLAY_T(4)
  KAD_REPLAY_T(5)
  KAD_REPLAY_T(6)
  KAD_REPLAY_T(7)
  KAD_REPLAY_T(8)
#undef KAD_REPLAY_T
  kad_set_error("gdn replay supports suffixes of 1..%d tokens, got %d", kTLimit, T);
  return KAD_ERR_UNSUPPORTED;
}

template <typename TIN>
int dispatch_dims(int K, int V, const void* q, const void* k, const void* v, int64_t ld_qk,
                  int64_t ld_v, const void* g, int gdt, const void* beta, int bdt,
                  int64_t ld_gate, const void* state, int sdt, void* out, int64_t ld_out,
                  int B, int W, int T, int H, int HV, float scale, hipStream_t s) {
#define KAD_REPLAY(KK, VV)                                                                  \
  if (K == KK && V == VV)                                                                   \
    return launch_replay<KK, VV, TIN>(q, k, v, ld_qk, ld_v, g, gdt, beta, bdt, ld_gate,     \
                                      state, sdt, out, ld_out, B, W, T, H, HV, scale, s);
  KAD_REPLAY(128, 128)
  KAD_REPLAY(64, 64)
  KAD_REPLAY(128, 64)
  KAD_REPLAY(64, 128)
#undef KAD_REPLAY
  KAD_UNSUPPORTED("gdn replay supports K, V in {64, 128}; got K=%d V=%d", K, V);
}

int launch_replay_conv(const bf16_t* proj, int64_t ld, const ConvArgs& cv, const void* g,
                       const void* beta, int64_t ld_gate, const void* state, int sdt, void* out,
                       int64_t ld_out, int B, int W, int T, int H, int HV, float scale,
                       const GateOutArgs* go, const ParentRows* par, hipStream_t stream) {
  const int bpb = W <= 256 ? W : 128;
  const int nbb = (int)kad_cdiv(W, bpb);
  const int64_t nblocks = (int64_t)B * HV * nbb;
  KAD_REQUIRE(nblocks <= 0x7fffffff, "gdn replay grid too large");
  const bf16_t* q = proj;
  const bf16_t* k = proj + (int64_t)H * 128;
  const bf16_t* v = proj + (int64_t)2 * H * 128;
  const bool last = go != nullptr && go->t_first == T - 1 && T > 1;
  const bool pv = par != nullptr;
#define KAD_REPLAY_CONV(TT, GV, LV, PV)                                                        \
  if (T == TT && (go != nullptr) == GV && last == LV && pv == PV) {                            \
    hipLaunchKernelGGL((gdn_replay_lds_kernel<TT, 3, true, GV, LV, PV>),                       \
                       dim3((unsigned)nblocks), dim3(256), 0, stream, q, k, v, ld, ld, g,      \
                       KAD_DTYPE_F32, beta, KAD_DTYPE_BF16, ld_gate, state, sdt, (bf16_t*)out, \
                       ld_out, W, H, HV, scale, bpb, nbb, cv, go ? *go : GateOutArgs{},        \
                       par ? *par : ParentRows{});                                             \
    return kad_launch_status("gdn_replay_lds_kernel");                                         \
  }
  KAD_REPLAY_CONV(1, false, false, false)
  KAD_REPLAY_CONV(2, false, false, false)
  KAD_REPLAY_CONV(1, true, false, false)
  KAD_REPLAY_CONV(2, true, false, false)
  KAD_REPLAY_CONV(2, true, true, false)
  KAD_REPLAY_CONV(2, true, true, true)
#undef KAD_REPLAY_CONV
  KAD_UNSUPPORTED("the fused conv replay takes 1 or 2 suffix tokens, got %d", T);
}

}  // namespace

namespace {
int replay_conv_common(
    const void* proj, int64_t ld_proj, const void* conv_state, int64_t ss_b, int64_t ss_c,
    int64_t ss_t, int history, const void* conv_weight, const void* log_decay, int gate_dtype,
    const void* beta, int beta_dtype, int64_t ld_gate, const void* state, int state_dtype,
    void* out, int64_t ld_out, int B, int W, int T, int H, int HV, int K, int V, float scale,
    const GateOutArgs* go, kad_stream_t stream, const ParentRows* par = nullptr) {
  KAD_REQUIRE(proj && conv_state && conv_weight && log_decay && beta && state && out,
              "null pointer argument");
  KAD_REQUIRE(B > 0 && W > 0 && T > 0 && H > 0 && HV > 0 && K > 0 && V > 0,
              "dimensions must be positive");
  KAD_REQUIRE(HV % H == 0, "HV must be divisible by H");
  KAD_REQUIRE(history >= 3, "the conv state needs at least 3 taps, got %d", history);
  KAD_REQUIRE(ld_proj >= (int64_t)2 * H * K + (int64_t)HV * V && ld_out >= (int64_t)HV * V &&
                  ld_gate >= HV,
              "row strides smaller than a row");
  KAD_REQUIRE(ld_out % 4 == 0 && ((uintptr_t)out % 8) == 0,
              "out rows must be 8-byte aligned (ld_out a multiple of 4)");
  for (int dt : {gate_dtype, beta_dtype, state_dtype})
    KAD_REQUIRE(dt == KAD_DTYPE_BF16 || dt == KAD_DTYPE_F16 || dt == KAD_DTYPE_F32,
                "unknown dtype code %d", dt);
  if (!(K == 128 && V == 128 && (T == 1 || T == 2) && W % 16 == 0))
    KAD_UNSUPPORTED("the fused conv replay takes K = V = 128, 1 or 2 suffix tokens and beam "
                    "counts that are multiples of 16 (got K=%d V=%d T=%d W=%d)", K, V, T, W);
  if (!(gate_dtype == KAD_DTYPE_F32 && beta_dtype == KAD_DTYPE_BF16 && ld_gate % 2 == 0 &&
        ((uintptr_t)beta % 4) == 0 && ((uintptr_t)log_decay % 4) == 0))
    KAD_UNSUPPORTED("the fused conv replay takes fp32 log decays and bf16 betas with an even "
                    "row stride");
  if (!(ld_proj % 8 == 0 && ((uintptr_t)proj % 16) == 0 && ((uintptr_t)conv_weight % 8) == 0))
    KAD_UNSUPPORTED("the fused conv replay takes 16-byte aligned projection rows and an 8-byte "
                    "aligned [C, 4] weight");
  const ConvArgs cv{(const bf16_t*)conv_state, ss_b, ss_c, ss_t, history,
                    (const bf16_t*)conv_weight};
  return launch_replay_conv((const bf16_t*)proj, ld_proj, cv, log_decay, beta, ld_gate, state,
                            state_dtype, out, ld_out, B, W, T, H, HV, scale, go, par,
                            (hipStream_t)stream);
}
}  // namespace

extern "C" int kad_gdn_suffix_replay_conv(
    const void* proj, int64_t ld_proj, const void* conv_state, int64_t ss_b, int64_t ss_c,
    int64_t ss_t, int history, const void* conv_weight, const void* log_decay, int gate_dtype,
    const void* beta, int beta_dtype, int64_t ld_gate, const void* state, int state_dtype,
    void* out, int64_t ld_out, int B, int W, int T, int H, int HV, int K, int V, float scale,
    kad_stream_t stream) {
  return replay_conv_common(proj, ld_proj, conv_state, ss_b, ss_c, ss_t, history, conv_weight,
                            log_decay, gate_dtype, beta, beta_dtype, ld_gate, state, state_dtype,
                            out, ld_out, B, W, T, H, HV, K, V, scale, nullptr, stream);
}

extern "C" int kad_gdn_suffix_replay_conv_gated(
    const void* proj, int64_t ld_proj, const void* conv_state, int64_t ss_b, int64_t ss_c,
    int64_t ss_t, int history, const void* conv_weight, const void* log_decay, int gate_dtype,
    const void* beta, int beta_dtype, int64_t ld_gate, const void* state, int state_dtype,
    const void* z, int64_t ldz, const void* norm_w, float eps, int last_token_only, void* out,
    int64_t ld_out, int B, int W, int T, int H, int HV, int K, int V, float scale,
    kad_stream_t stream) {
  KAD_REQUIRE(z && norm_w, "null pointer argument");
  KAD_REQUIRE(ldz % 4 == 0 && ((uintptr_t)z % 8) == 0 && ((uintptr_t)norm_w % 8) == 0,
              "z rows and the norm weight must be 8-byte aligned (ldz a multiple of 4)");
  KAD_REQUIRE(ldz >= (int64_t)HV * V, "ldz smaller than a row");
  const GateOutArgs go{(const bf16_t*)z, ldz, (const bf16_t*)norm_w, eps,
                       last_token_only ? T - 1 : 0};
  return replay_conv_common(proj, ld_proj, conv_state, ss_b, ss_c, ss_t, history, conv_weight,
                            log_decay, gate_dtype, beta, beta_dtype, ld_gate, state, state_dtype,
                            out, ld_out, B, W, T, H, HV, K, V, scale, &go, stream);
}

extern "C" int kad_gdn_suffix_replay_conv_gated_parents(
    const void* prev, int64_t ld_prev, const int64_t* parents, int Wp, const void* cur,
    int64_t ld_cur, const void* conv_state, int64_t ss_b, int64_t ss_c, int64_t ss_t,
    int history, const void* conv_weight, const void* log_decay, int gate_dtype,
    const void* beta, int beta_dtype, int64_t ld_gate, const void* state, int state_dtype,
    const void* z, int64_t ldz, const void* norm_w, float eps, void* out, int64_t ld_out, int B,
    int W, int T, int H, int HV, int K, int V, float scale, kad_stream_t stream) {
  KAD_REQUIRE(prev && parents && cur && z && norm_w, "null pointer argument");
  KAD_REQUIRE(Wp > 0, "Wp must be positive");
  KAD_REQUIRE(ldz % 4 == 0 && ((uintptr_t)z % 8) == 0 && ((uintptr_t)norm_w % 8) == 0,
              "z rows and the norm weight must be 8-byte aligned (ldz a multiple of 4)");
  KAD_REQUIRE(ldz >= (int64_t)HV * V, "ldz smaller than a row");
  KAD_REQUIRE(ld_prev >= (int64_t)2 * H * K + (int64_t)HV * V, "ld_prev smaller than a row");
  if (T != 2) KAD_UNSUPPORTED("the parent-row conv replay takes two-token suffixes, got %d", T);
  if (!(ld_prev % 8 == 0 && ((uintptr_t)prev % 16) == 0))
    KAD_UNSUPPORTED("the parent-row conv replay takes 16-byte aligned parent rows");
  const GateOutArgs go{(const bf16_t*)z, ldz, (const bf16_t*)norm_w, eps, T - 1};
  const ParentRows pr{(const bf16_t*)prev, ld_prev, parents, Wp, (const bf16_t*)cur, ld_cur};
  return replay_conv_common(cur, ld_cur, conv_state, ss_b, ss_c, ss_t, history, conv_weight,
                            log_decay, gate_dtype, beta, beta_dtype, ld_gate, state, state_dtype,
                            out, ld_out, B, W, T, H, HV, K, V, scale, &go, stream, &pr);
}

extern "C" int kad_gdn_suffix_replay(const void* q, const void* k, const void* v,
                                     int64_t ld_qk, int64_t ld_v, int qkv_dtype,
                                     const void* log_decay, int gate_dtype, const void* beta,
                                     int beta_dtype, int64_t ld_gate, const void* state,
                                     int state_dtype, void* out, int64_t ld_out, int B, int W,
                                     int T, int H, int HV, int K, int V, float scale,
                                     kad_stream_t stream) {
  KAD_REQUIRE(q && k && v && log_decay && beta && state && out, "null pointer argument");
  KAD_REQUIRE(B > 0 && W > 0 && T > 0 && H > 0 && HV > 0 && K > 0 && V > 0,
              "dimensions must be positive");
  KAD_REQUIRE(HV % H == 0, "HV must be divisible by H");
  KAD_REQUIRE(ld_qk >= (int64_t)H * K && ld_v >= (int64_t)HV * V && ld_out >= (int64_t)HV * V &&
                  ld_gate >= HV,
              "row strides smaller than a row");
  KAD_REQUIRE(ld_qk % 8 == 0 && ld_v % 4 == 0 && ld_out % 4 == 0,
              "q/k row stride must be a multiple of 8 and v/out of 4 elements");
  KAD_REQUIRE(((uintptr_t)q | (uintptr_t)k) % 16 == 0 && ((uintptr_t)v | (uintptr_t)out) % 8 == 0,
              "q/k must be 16-byte and v/out 8-byte aligned");
  if (T > kTLimit) KAD_UNSUPPORTED("gdn replay supports T <= %d suffix tokens, got %d", kTLimit, T);
  for (int dt : {gate_dtype, beta_dtype, state_dtype})
    KAD_REQUIRE(dt == KAD_DTYPE_BF16 || dt == KAD_DTYPE_F16 || dt == KAD_DTYPE_F32,
                "unknown dtype code %d", dt);
  hipStream_t s = (hipStream_t)stream;
  if (qkv_dtype == KAD_DTYPE_BF16)
    return dispatch_dims<bf16_t>(K, V, q, k, v, ld_qk, ld_v, log_decay, gate_dtype, beta,
                                 beta_dtype, ld_gate, state, state_dtype, out, ld_out, B, W, T,
                                 H, HV, scale, s);
  if (qkv_dtype == KAD_DTYPE_F32) {
    KAD_REQUIRE(((uintptr_t)v | (uintptr_t)out) % 16 == 0, "fp32 v/out must be 16-byte aligned");
    return dispatch_dims<float>(K, V, q, k, v, ld_qk, ld_v, log_decay, gate_dtype, beta,
                                beta_dtype, ld_gate, state, state_dtype, out, ld_out, B, W, T, H,
                                HV, scale, s);
  }
  KAD_UNSUPPORTED("gdn replay supports bf16 and fp32 q/k/v, got dtype %d", qkv_dtype);
}
