// Chunked gated delta rule (gfx950): prefill state building and long suffixes.
//
// Replaces, for the prefill, transformers' torch_chunk_gated_delta_rule
// (modeling_qwen3_5.py:249-327) that the reference prefill runs through the
// native model forward (src/kadllm/adapters/qwen3_5.py:111), and, for the
// operator, src/kadllm/ops.py:139-163 when a suffix is longer than the replay
// kernel handles or a final state is requested (ops.py:119-122).
//
// Per chunk of 64 tokens, with G the within-chunk cumulative log decay,
// D_ij = exp(G_i - G_j) and hats the normalised q (incl. scale) and k:
//   A_ij  = -beta_i (k^_i . k^_j) D_ij (j < i); T' = the routine's forward
//           substitution of A (rows 1..63); T = T' + I
//   Z_j   = beta_j (v_j - e^{G_j} k^_j S)           (v_new = T Z equals the
//           routine's U - W S with U = T beta v, W = T beta k^ e^G)
//   o_i   = e^{G_i} q^_i S + sum_{j<=i} In_ij v_new_j,  In_ij = (q^_i . k^_j) D_ij
//   S    <- e^{G_last} S + sum_i e^{G_last - G_i} k^_i v_new_i^T
//
// Two kernels.  gdn_chunk_prep runs every (sequence, head, chunk) in
// parallel: normalisation, the two Gram matrices on bf16 MFMA, the decay
// masks and the triangular solve; it writes the chunk's bf16 q/k rows, T' and
// In as bf16 hi/lo planes (x = hi + lo to 2^-16) and per-token scalars to a
// workspace.  gdn_chunk_scan walks the chunks of one (sequence, head) in
// order with 4 waves, wave w owning value columns [32w, 32w+32) of the fp32
// state S [K, V].  S lives in MFMA accumulator registers (rows k, columns v)
// and the same registers, split hi/lo, are the B operand of k S and q S: the
// accumulator layout gives each lane the k-rows {0-3, 8-11} (+4 in the upper
// half-wave) of every 16-row block of its column, and the A operands are read
// from LDS in that same order.  All products run on v_mfma_f32_32x32x16_bf16
// with fp32 accumulation; fp32 operands take 2-3 hi/lo passes.

#include "kad_common.h"

namespace {

constexpr int kC = 64;
constexpr int kPrepThreads = 256;

// workspace record of one (sequence, head, chunk), in bytes
template <int K>
struct ChunkRec {
  static constexpr size_t kn = 0;                              // bf16 [64][K]
  static constexpr size_t qn = kn + kC * K * 2;                // bf16 [64][K]
  static constexpr size_t thi = qn + kC * K * 2;               // bf16 [64][64]
  static constexpr size_t tlo = thi + kC * kC * 2;
  static constexpr size_t ihi = tlo + kC * kC * 2;
  static constexpr size_t ilo = ihi + kC * kC * 2;
  static constexpr size_t scal = ilo + kC * kC * 2;            // fp32 [5][64]
  static constexpr size_t bytes = scal + 5 * kC * 4;
};
enum { S_EG = 0, S_BT = 1, S_KM = 2, S_QM = 3, S_WU = 4 };

// ---------------------------------------------------------------------------
template <int K>
__global__ __launch_bounds__(kPrepThreads) void gdn_chunk_prep(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, int64_t ld_qk,
    const void* __restrict__ g, int gdt, const void* __restrict__ beta, int bdt,
    int64_t ld_gate, uint8_t* __restrict__ ws, int T, int H, int HV, int nchunks, float scale,
    int hf_norm) {
  constexpr int LD = K + 8;
  constexpr int CPR = K / 8;       // 16-byte chunks per q/k row
  constexpr int RPI = 64 / CPR;    // rows per wave instruction
  // the bf16 q/k rows (Gram phase) and, later, A in residue-major order plus
  // the T' staging tile share one LDS region
  constexpr size_t kRows = 2 * kC * LD * sizeof(bf16_t);
  constexpr size_t kMats = (kC * kC + kC * (kC + 1)) * sizeof(float);
  __shared__ __attribute__((aligned(16))) unsigned char region[kRows > kMats ? kRows : kMats];
  bf16_t* kb = (bf16_t*)region;
  bf16_t* qb = kb + kC * LD;
  float* Ar = (float*)region;                         // Ar[i*64 + (j%4)*16 + j/4] = A[i][j]
  float(*Tm)[kC + 1] = (float(*)[kC + 1])(Ar + kC * kC);
  __shared__ float Gs[kC], bt[kC], kmul[kC], qmul[kC];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = blockIdx.x % nchunks;
  const int nh = blockIdx.x / nchunks;
  const int n = nh / HV, hv = nh % HV;
  const int h = hv / (HV / H);
  const int t0 = c * kC;
  const int nt = min(kC, T - t0);
  uint8_t* rec = ws + (size_t)blockIdx.x * ChunkRec<K>::bytes;

  // ---- rows: wave w normalises rows 16w..16w+15, RPI rows per instruction
  // (lane -> row lane / CPR, 16-byte chunk lane % CPR)
  {
    const int rsub = lane / CPR, ch = lane % CPR;
#pragma unroll
    for (int it = 0; it < 16 / RPI; ++it) {
      const int i = wave * 16 + it * RPI + rsub;
      const bool live = i < nt;
      const int64_t off = ((int64_t)n * T + t0 + (live ? i : 0)) * ld_qk + (int64_t)h * K + ch * 8;
      u32x4 kr = live ? *(const u32x4*)(k + off) : u32x4{0, 0, 0, 0};
      u32x4 qr = live ? *(const u32x4*)(q + off) : u32x4{0, 0, 0, 0};
      float kv[8], qv[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kv[2 * e] = __uint_as_float(kr[e] << 16);
        kv[2 * e + 1] = __uint_as_float(kr[e] & 0xffff0000u);
        qv[2 * e] = __uint_as_float(qr[e] << 16);
        qv[2 * e + 1] = __uint_as_float(qr[e] & 0xffff0000u);
      }
      float kss = 0.f, qss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        kss += hf_norm ? round_bf(kv[e] * kv[e]) : kv[e] * kv[e];
        qss += hf_norm ? round_bf(qv[e] * qv[e]) : qv[e] * qv[e];
      }
#pragma unroll
      for (int o = CPR / 2; o > 0; o >>= 1) {
        kss += __shfl_xor(kss, o, 64);
        qss += __shfl_xor(qss, o, 64);
      }
      float km, qm;
      if (hf_norm) {
        // transformers l2norm in bf16: x * rsqrt(sum(x*x) + eps), each op rounded
        const float krs = round_bf(1.0f / sqrtf(round_bf(round_bf(kss) + 1e-6f)));
        const float qrs = round_bf(1.0f / sqrtf(round_bf(round_bf(qss) + 1e-6f)));
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          kv[e] = round_bf(kv[e] * krs);
          qv[e] = round_bf(qv[e] * qrs);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          kr[e] = (uint32_t)f2bf(kv[2 * e]) | ((uint32_t)f2bf(kv[2 * e + 1]) << 16);
          qr[e] = (uint32_t)f2bf(qv[2 * e]) | ((uint32_t)f2bf(qv[2 * e + 1]) << 16);
        }
        km = 1.f;
        qm = scale;
      } else {
        km = 1.0f / sqrtf(kss + 1e-6f);
        qm = scale / sqrtf(qss + 1e-6f);
      }
      *(u32x4*)(kb + i * LD + ch * 8) = kr;
      *(u32x4*)(qb + i * LD + ch * 8) = qr;
      *(u32x4*)((bf16_t*)(rec + ChunkRec<K>::kn) + i * K + ch * 8) = kr;
      *(u32x4*)((bf16_t*)(rec + ChunkRec<K>::qn) + i * K + ch * 8) = qr;
      if (ch == 0) {
        kmul[i] = km;
        qmul[i] = qm;
      }
    }
  }
  if (tid < kC) {
    const bool live = tid < nt;
    const int64_t gi = ((int64_t)n * T + t0 + (live ? tid : 0)) * ld_gate + hv;
    Gs[tid] = live ? load_as_float(g, gi, gdt) : 0.f;
    bt[tid] = live ? load_as_float(beta, gi, bdt) : 0.f;
  }
  __syncthreads();
  if (tid == 0) {
    float acc = 0.f;
    for (int i = 0; i < kC; ++i) {  // sequential cumulative sum, as torch.cumsum
      acc += Gs[i];
      Gs[i] = acc;
    }
  }
  __syncthreads();
  if (tid < kC) {
    float* sc = (float*)(rec + ChunkRec<K>::scal);
    sc[S_EG * kC + tid] = expf(Gs[tid]);
    sc[S_BT * kC + tid] = bt[tid];
    sc[S_KM * kC + tid] = kmul[tid];
    sc[S_QM * kC + tid] = qmul[tid];
    sc[S_WU * kC + tid] = kmul[tid] * expf(Gs[kC - 1] - Gs[tid]);
  }

  // ---- Gram matrices: 8 tiles of 32x32 (4 for k k^T, 4 for q k^T), 2 per wave.
  // q k^T tiles go straight to the workspace as In hi/lo; k k^T tiles become A
  // once every wave is done reading the rows.
  bf16_t* ihi = (bf16_t*)(rec + ChunkRec<K>::ihi);
  bf16_t* ilo = (bf16_t*)(rec + ChunkRec<K>::ilo);
  f32x16 gram[2];
  {
    const int fr = lane & 31, fk = (lane >> 5) * 8;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      const int tile = wave * 2 + tt;
      const int which = tile >> 2, ti = (tile >> 1) & 1, tj = tile & 1;
      const bf16_t* rowsrc = which == 0 ? kb : qb;
      f32x16 acc = f32x16{};
#pragma unroll
      for (int s = 0; s < K / 16; ++s) {
        const bf16x8 a = as_bf16x8(*(const u32x4*)(rowsrc + (ti * 32 + fr) * LD + s * 16 + fk));
        const bf16x8 b = as_bf16x8(*(const u32x4*)(kb + (tj * 32 + fr) * LD + s * 16 + fk));
        acc = mfma32x32x16(a, b, acc);
      }
      gram[tt] = acc;
      if (which == 1) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int i = ti * 32 + (e / 4) * 8 + (lane >> 5) * 4 + (e % 4);
          const int j = tj * 32 + fr;
          const float iv = j <= i ? (acc[e] * qmul[i] * kmul[j]) * expf(Gs[i] - Gs[j]) : 0.f;
          const bf16_t ih = f2bf(iv);
          ihi[i * kC + j] = ih;
          ilo[i * kC + j] = f2bf(iv - bf2f(ih));
        }
      }
    }
  }
  __syncthreads();  // rows no longer needed: the region becomes A / T'
#pragma unroll
  for (int tt = 0; tt < 2; ++tt) {
    const int tile = wave * 2 + tt;
    const int which = tile >> 2, ti = (tile >> 1) & 1, tj = tile & 1;
    if (which == 0) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int i = ti * 32 + (e / 4) * 8 + (lane >> 5) * 4 + (e % 4);
        const int j = tj * 32 + (lane & 31);
        Ar[i * kC + (j & 3) * 16 + (j >> 2)] =
            j < i ? -bt[i] * (gram[tt][e] * kmul[i] * kmul[j]) * expf(Gs[i] - Gs[j]) : 0.f;
      }
    }
  }
  __syncthreads();

  // ---- forward substitution T'[i][j] = A[i][j] + sum_{m<i} A[i][m] T'[m][j]
  // (A strictly lower).  Columns are independent: wave w owns columns
  // 16w..16w+15 with 4 lanes per column; lane r of column j keeps rows
  // m = 4q + r (q < 16) of the column in registers.  Rows not yet computed are
  // zero, so each row needs no masking; no barriers are involved.
  {
    const int col = wave * 16 + (lane >> 2), r = lane & 3;
    float treg[16];
#pragma unroll
    for (int qq = 0; qq < 16; ++qq) treg[qq] = 0.f;
#pragma unroll
    for (int i = 1; i < kC; ++i) {
      constexpr int kMaxQ = 16;
      const int nq = (i + 3) / 4;  // q < nq covers every m < i of residue r
      const float* arow = Ar + i * kC + r * 16;
      float part = 0.f;
#pragma unroll
      for (int q4 = 0; q4 < kMaxQ / 4; ++q4) {
        if (q4 * 4 >= nq) break;
        const float4 av = *(const float4*)(arow + q4 * 4);
        part += av.x * treg[q4 * 4];
        if (q4 * 4 + 1 < nq) part += av.y * treg[q4 * 4 + 1];
        if (q4 * 4 + 2 < nq) part += av.z * treg[q4 * 4 + 2];
        if (q4 * 4 + 3 < nq) part += av.w * treg[q4 * 4 + 3];
      }
      part += __shfl_xor(part, 1, 64);
      part += __shfl_xor(part, 2, 64);
      const float val = Ar[i * kC + (col & 3) * 16 + (col >> 2)] + part;
      if (r == (i & 3)) treg[i >> 2] = val;
    }
#pragma unroll
    for (int qq = 0; qq < 16; ++qq) Tm[qq * 4 + r][col] = treg[qq];
  }
  __syncthreads();

  // ---- T' as bf16 hi/lo planes, 16 elements (32 bytes per plane) per thread
  {
    bf16_t* thi = (bf16_t*)(rec + ChunkRec<K>::thi);
    bf16_t* tlo = (bf16_t*)(rec + ChunkRec<K>::tlo);
    const int i = tid >> 2, j0 = (tid & 3) * 16;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      u32x4 hv4, lv4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t hw = 0, lw = 0;
#pragma unroll
        for (int b2 = 0; b2 < 2; ++b2) {
          const float tv = Tm[i][j0 + half * 8 + e * 2 + b2];
          const bf16_t th = f2bf(tv);
          hw |= (uint32_t)th << (16 * b2);
          lw |= (uint32_t)f2bf(tv - bf2f(th)) << (16 * b2);
        }
        hv4[e] = hw;
        lv4[e] = lw;
      }
      *(u32x4*)(thi + i * kC + j0 + half * 8) = hv4;
      *(u32x4*)(tlo + i * kC + j0 + half * 8) = lv4;
    }
  }
}

// ---------------------------------------------------------------------------
// A fragment whose K slots follow the accumulator order: slot i of lane half
// `hi` is column base + (i / 4) * 8 + hi * 4 + i % 4 of row `row`.
__device__ __forceinline__ bf16x8 perm_frag(const bf16_t* rowp, int base, int hi) {
  const u32x2 a = *(const u32x2*)(rowp + base + hi * 4);
  const u32x2 b = *(const u32x2*)(rowp + base + 8 + hi * 4);
  const u32x4 v = {a[0], a[1], b[0], b[1]};
  return as_bf16x8(v);
}

// B fragments (hi, lo) of an fp32 accumulator tile for K step s: the 8
// accumulator entries (s%2)*8 .. +7 of 32-row tile s/2
__device__ __forceinline__ void acc_frags(const f32x16& t, int half, bf16x8& hi, bf16x8& lo) {
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = t[half * 8 + i];
  split8(x, hi, lo);
}

template <int K, int V>
__global__ __launch_bounds__(V * 2) void gdn_chunk_scan(
    const bf16_t* __restrict__ v, int64_t ld_v, const uint8_t* __restrict__ ws,
    const void* __restrict__ state0, int sdt, int beams_per_state, bf16_t* __restrict__ out,
    int64_t ld_out, float* __restrict__ final_state, int T, int HV, int nchunks) {
  constexpr int KT = K / 32;      // 32-row k tiles of S
  constexpr int KS = K / 16;      // k16 steps over K
  constexpr int LDK = K + 8;      // bf16 [64][K] rows (16-byte padding)
  constexpr int LD64 = kC + 4;    // bf16 [*][64] rows (8-byte padding)
  constexpr int NTH = V * 2;      // V/32 waves
  __shared__ __attribute__((aligned(16))) bf16_t kb[kC * LDK];
  __shared__ __attribute__((aligned(16))) bf16_t qb[kC * LDK];
  __shared__ __attribute__((aligned(16))) bf16_t kbT[K * LD64];
  __shared__ __attribute__((aligned(16))) bf16_t Th[kC * LD64], Tl[kC * LD64];
  __shared__ __attribute__((aligned(16))) bf16_t Ih[kC * LD64], Il[kC * LD64];
  __shared__ __attribute__((aligned(16))) bf16_t vb[kC * (V + 8)];
  __shared__ float sc[5][kC];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hi = lane >> 5, col = lane & 31;
  const int n = blockIdx.x / HV, hv = blockIdx.x % HV;
  const int vcol = wave * 32 + col;  // this lane's value column

  // S[k][vcol] in accumulator layout: tile kt, entry e -> k = kt*32 + (e/4)*8 + hi*4 + e%4
  f32x16 S[KT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int kk = kt * 32 + (e / 4) * 8 + hi * 4 + (e % 4);
      S[kt][e] = state0 ? load_as_float(state0,
                                        ((int64_t)(n / beams_per_state) * HV + hv) * K * V +
                                            (int64_t)kk * V + vcol,
                                        sdt)
                        : 0.f;
    }
  }

  for (int c = 0; c < nchunks; ++c) {
    const int t0 = c * kC;
    const int nt = min(kC, T - t0);
    const uint8_t* rec = ws + ((size_t)blockIdx.x * nchunks + c) * ChunkRec<K>::bytes;
    __syncthreads();  // previous chunk done with LDS
    {
      // every global load of the chunk is issued before any LDS store, so the
      // load latency is paid once per chunk
      constexpr int kRowV = kC * K / 8 / NTH;       // q/k 16-byte chunks per thread
      constexpr int kPlaneV = kC * kC / 8 / NTH;    // T'/In plane chunks per thread
      constexpr int kVV = kC * V / 8 / NTH;         // v chunks per thread
      static_assert(kRowV * NTH * 8 == kC * K && kPlaneV * NTH * 8 == kC * kC &&
                        kVV * NTH * 8 == kC * V, "chunk tiles must split evenly");
      const bf16_t* kn = (const bf16_t*)(rec + ChunkRec<K>::kn);
      const bf16_t* qn = (const bf16_t*)(rec + ChunkRec<K>::qn);
      const bf16_t* planes[4] = {(const bf16_t*)(rec + ChunkRec<K>::thi),
                                 (const bf16_t*)(rec + ChunkRec<K>::tlo),
                                 (const bf16_t*)(rec + ChunkRec<K>::ihi),
                                 (const bf16_t*)(rec + ChunkRec<K>::ilo)};
      u32x4 rk[kRowV], rq[kRowV], rp[4][kPlaneV], rv[kVV];
#pragma unroll
      for (int u = 0; u < kRowV; ++u) {
        const int e = tid + u * NTH;
        rk[u] = *(const u32x4*)(kn + e * 8);
        rq[u] = *(const u32x4*)(qn + e * 8);
      }
#pragma unroll
      for (int p = 0; p < 4; ++p)
#pragma unroll
        for (int u = 0; u < kPlaneV; ++u) rp[p][u] = *(const u32x4*)(planes[p] + (tid + u * NTH) * 8);
#pragma unroll
      for (int u = 0; u < kVV; ++u) {
        const int e = tid + u * NTH;
        const int i = e / (V / 8), v8 = (e % (V / 8)) * 8;
        rv[u] = i < nt ? *(const u32x4*)(v + ((int64_t)n * T + t0 + i) * ld_v + (int64_t)hv * V + v8)
                       : u32x4{0u, 0u, 0u, 0u};
      }
      const float* scg = (const float*)(rec + ChunkRec<K>::scal);
      float rs[(5 * kC + NTH - 1) / NTH];
#pragma unroll
      for (int u = 0; u < (5 * kC + NTH - 1) / NTH; ++u) {
        const int e = tid + u * NTH;
        rs[u] = e < 5 * kC ? scg[e] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < kRowV; ++u) {
        const int e = tid + u * NTH;
        const int i = e / (K / 8), k8 = (e % (K / 8)) * 8;
        *(u32x4*)(kb + i * LDK + k8) = rk[u];
        *(u32x4*)(qb + i * LDK + k8) = rq[u];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          kbT[(k8 + 2 * w) * LD64 + i] = (bf16_t)(rk[u][w] & 0xffffu);
          kbT[(k8 + 2 * w + 1) * LD64 + i] = (bf16_t)(rk[u][w] >> 16);
        }
      }
      bf16_t* dsts[4] = {Th, Tl, Ih, Il};
#pragma unroll
      for (int p = 0; p < 4; ++p)
#pragma unroll
        for (int u = 0; u < kPlaneV; ++u) {
          const int e = tid + u * NTH;
          const int i = e / (kC / 8), j8 = (e % (kC / 8)) * 8;
          *(u32x2*)(dsts[p] + i * LD64 + j8) = u32x2{rp[p][u][0], rp[p][u][1]};
          *(u32x2*)(dsts[p] + i * LD64 + j8 + 4) = u32x2{rp[p][u][2], rp[p][u][3]};
        }
#pragma unroll
      for (int u = 0; u < kVV; ++u) {
        const int e = tid + u * NTH;
        const int i = e / (V / 8), v8 = (e % (V / 8)) * 8;
        *(u32x4*)(vb + i * (V + 8) + v8) = rv[u];
      }
#pragma unroll
      for (int u = 0; u < (5 * kC + NTH - 1) / NTH; ++u) {
        const int e = tid + u * NTH;
        if (e < 5 * kC) sc[e / kC][e % kC] = rs[u];
      }
    }
    __syncthreads();

    // S as B fragments (hi/lo) for every k16 step
    bf16x8 sh[KS], sl[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) acc_frags(S[s / 2], s % 2, sh[s], sl[s]);

    // ---- Z_j = beta_j (v_j - e^{G_j} kmul_j (k S)_j), tokens j in two 32-row tiles
    f32x16 Z[2];
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) {
      f32x16 acc = f32x16{};
      const bf16_t* rowp = kb + (jt * 32 + col) * LDK;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const bf16x8 a = perm_frag(rowp, s * 16, hi);
        acc = mfma32x32x16(a, sh[s], acc);
        acc = mfma32x32x16(a, sl[s], acc);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int j = jt * 32 + (e / 4) * 8 + hi * 4 + (e % 4);
        const float vj = bf2f(vb[j * (V + 8) + vcol]);
        Z[jt][e] = sc[S_BT][j] * (vj - sc[S_EG][j] * (sc[S_KM][j] * acc[e]));
      }
    }
    // ---- v_new = Z + T' Z (K dim = tokens, accumulator order on both sides)
    bf16x8 zh[4], zl[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) acc_frags(Z[s / 2], s % 2, zh[s], zl[s]);
    f32x16 VN[2];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      f32x16 acc = Z[it];
      const bf16_t* th = Th + (it * 32 + col) * LD64;
      const bf16_t* tl = Tl + (it * 32 + col) * LD64;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 ah = perm_frag(th, s * 16, hi), al = perm_frag(tl, s * 16, hi);
        acc = mfma32x32x16(ah, zh[s], acc);
        acc = mfma32x32x16(ah, zl[s], acc);
        acc = mfma32x32x16(al, zh[s], acc);
      }
      VN[it] = acc;
    }
    // ---- o_i = e^{G_i} qmul_i (q S)_i + In v_new
    bf16x8 vh[4], vl[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) acc_frags(VN[s / 2], s % 2, vh[s], vl[s]);
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      f32x16 qs = f32x16{};
      const bf16_t* rowp = qb + (it * 32 + col) * LDK;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const bf16x8 a = perm_frag(rowp, s * 16, hi);
        qs = mfma32x32x16(a, sh[s], qs);
        qs = mfma32x32x16(a, sl[s], qs);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int i = it * 32 + (e / 4) * 8 + hi * 4 + (e % 4);
        qs[e] *= sc[S_EG][i] * sc[S_QM][i];
      }
      const bf16_t* ih = Ih + (it * 32 + col) * LD64;
      const bf16_t* il = Il + (it * 32 + col) * LD64;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 ah = perm_frag(ih, s * 16, hi), al = perm_frag(il, s * 16, hi);
        qs = mfma32x32x16(ah, vh[s], qs);
        qs = mfma32x32x16(ah, vl[s], qs);
        qs = mfma32x32x16(al, vh[s], qs);
      }
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int i = it * 32 + (e / 4) * 8 + hi * 4 + (e % 4);
        if (i < nt) out[((int64_t)n * T + t0 + i) * ld_out + (int64_t)hv * V + vcol] = f2bf(qs[e]);
      }
    }
    // ---- S <- e^{G_last} S + sum_i (kmul_i e^{G_last-G_i}) k_i v_new_i^T
    bf16x8 wh[4], wl[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float x[8];
#pragma unroll
      for (int i8 = 0; i8 < 8; ++i8) {
        const int e = (s % 2) * 8 + i8;
        const int i = (s / 2) * 32 + (e / 4) * 8 + hi * 4 + (e % 4);
        x[i8] = VN[s / 2][e] * sc[S_WU][i];
      }
      split8(x, wh[s], wl[s]);
    }
    const float egl = sc[S_EG][kC - 1];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      f32x16 acc = S[kt];
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] *= egl;
      const bf16_t* rowp = kbT + (kt * 32 + col) * LD64;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 a = perm_frag(rowp, s * 16, hi);
        acc = mfma32x32x16(a, wh[s], acc);
        acc = mfma32x32x16(a, wl[s], acc);
      }
      S[kt] = acc;
    }
  }
  if (final_state) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int kk = kt * 32 + (e / 4) * 8 + hi * 4 + (e % 4);
        final_state[((int64_t)n * HV + hv) * K * V + (int64_t)kk * V + vcol] = S[kt][e];
      }
  }
}

template <int K, int V>
int launch_chunk(const void* q, const void* k, const void* v, int64_t ld_qk, int64_t ld_v,
                 const void* g, int gdt, const void* beta, int bdt, int64_t ld_gate,
                 const void* state0, int sdt, int bps, void* out, int64_t ld_out, float* fin,
                 void* ws, int N, int T, int H, int HV, float scale, int hf_norm, hipStream_t s) {
  const int nchunks = (T + kC - 1) / kC;
  const int64_t nrec = (int64_t)N * HV * nchunks;
  hipLaunchKernelGGL((gdn_chunk_prep<K>), dim3((unsigned)nrec), dim3(kPrepThreads), 0, s,
                     (const bf16_t*)q, (const bf16_t*)k, ld_qk, g, gdt, beta, bdt, ld_gate,
                     (uint8_t*)ws, T, H, HV, nchunks, scale, hf_norm);
  int rc = kad_launch_status("gdn_chunk_prep");
  if (rc) return rc;
  hipLaunchKernelGGL((gdn_chunk_scan<K, V>), dim3((unsigned)((int64_t)N * HV)), dim3(V * 2), 0, s,
                     (const bf16_t*)v, ld_v, (const uint8_t*)ws, state0, sdt, bps, (bf16_t*)out,
                     ld_out, fin, T, HV, nchunks);
  return kad_launch_status("gdn_chunk_scan");
}

size_t rec_bytes(int K) { return K == 128 ? ChunkRec<128>::bytes : ChunkRec<64>::bytes; }

}  // namespace

static int64_t chunk_ws_bytes(int N, int T, int HV, int K) {
  return (int64_t)N * HV * ((T + kC - 1) / kC) * (int64_t)rec_bytes(K);
}

extern "C" int kad_gdn_chunk_workspace_bytes(int N, int T, int HV, int K, int64_t* bytes) {
  KAD_REQUIRE(bytes, "null pointer argument");
  KAD_REQUIRE(N > 0 && T > 0 && HV > 0, "bad dimensions");
  if (K != 64 && K != 128) KAD_UNSUPPORTED("chunked gated delta supports K in {64, 128}");
  *bytes = chunk_ws_bytes(N, T, HV, K);
  return KAD_OK;
}

extern "C" int kad_gdn_chunk(const void* q, const void* k, const void* v, int64_t ld_qk,
                             int64_t ld_v, int qkv_dtype, const void* log_decay, int gate_dtype,
                             const void* beta, int beta_dtype, int64_t ld_gate,
                             const void* initial_state, int state_dtype, int beams_per_state,
                             void* out, int64_t ld_out, float* final_state, void* workspace,
                             int64_t workspace_bytes, int N, int T, int H, int HV, int K, int V,
                             float scale, int transformers_l2norm, kad_stream_t stream) {
  KAD_REQUIRE(q && k && v && log_decay && beta && out && workspace, "null pointer argument");
  KAD_REQUIRE(N > 0 && T > 0 && H > 0 && HV > 0 && HV % H == 0, "bad dimensions");
  KAD_REQUIRE(!initial_state || (beams_per_state > 0 && N % beams_per_state == 0),
              "N must be a multiple of beams_per_state");
  KAD_REQUIRE(ld_qk >= (int64_t)H * K && ld_v >= (int64_t)HV * V && ld_out >= (int64_t)HV * V &&
                  ld_gate >= HV,
              "row strides smaller than a row");
  KAD_REQUIRE(ld_v % 8 == 0 && ((uintptr_t)v % 16) == 0, "v rows must be 16-byte aligned");
  KAD_REQUIRE(ld_qk % 8 == 0 && ((uintptr_t)q % 16) == 0 && ((uintptr_t)k % 16) == 0,
              "q and k rows must be 16-byte aligned");
  if (qkv_dtype != KAD_DTYPE_BF16) KAD_UNSUPPORTED("chunked gated delta takes bf16 q/k/v");
  if (!((K == 64 || K == 128) && (V == 64 || V == 128)))
    KAD_UNSUPPORTED("chunked gated delta supports K, V in {64, 128}; got K=%d V=%d", K, V);
  const int64_t need = chunk_ws_bytes(N, T, HV, K);
  KAD_REQUIRE(workspace_bytes >= need, "workspace of %lld bytes is smaller than %lld",
              (long long)workspace_bytes, (long long)need);
  KAD_REQUIRE(((uintptr_t)workspace % 16) == 0, "workspace must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
#define KAD_CHUNK(KK, VV)                                                                      \
  if (K == KK && V == VV)                                                                      \
    return launch_chunk<KK, VV>(q, k, v, ld_qk, ld_v, log_decay, gate_dtype, beta, beta_dtype, \
                                ld_gate, initial_state, state_dtype, beams_per_state, out,     \
                                ld_out, final_state, workspace, N, T, H, HV, scale,            \
                                transformers_l2norm, s);
  KAD_CHUNK(128, 128)
  KAD_CHUNK(64, 64)
  KAD_CHUNK(128, 64)
  KAD_CHUNK(64, 128)
#undef KAD_CHUNK
  KAD_UNSUPPORTED("unreachable");
}
