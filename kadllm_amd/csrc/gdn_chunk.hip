// Chunked gated delta rule (gfx950): prefill state building and long suffixes.
//
// Replaces, for the prefill, transformers' torch_chunk_gated_delta_rule
// (modeling_qwen3_5.py:249-327) that the reference prefill runs through the
// native model forward (src/kadllm/adapters/qwen3_5.py:111), and, for the operator,
// src/kadllm/ops.py:139-163 when a suffix is longer than the replay kernel
// handles or a final state is requested (ops.py:119-122).
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
// parallel and does the part that needs no state: the q and k row scales,
// the k Gram matrix and the q k^T tiles on bf16 MFMA, the decay masks, the
// triangular solve, and In.  It writes T' and In as bf16 hi/lo planes
// (x = hi + lo to 2^-16), already in the scan's MFMA fragment order (the
// In^T tiles come out of the MFMA with tokens j in the accumulator order,
// which is the K order of the In v_new product), and per-token scalars:
// 26 KB per chunk.  gdn_chunk_scan walks the chunks of one (sequence, head)
// in order with 4 waves, wave w owning value columns [32w, 32w+32) of the
// fp32 state S [K, V]; two workgroups share a CU so one's loads overlap the
// other's MFMAs.  It reads q, k and v itself and scales q and k with the
// prep's row scales (k to the prep's bits).  Forming In in the prep instead
// of in every wave of the scan took 42% of the VALU instructions out of the
// scan's serial chain.  S lives in accumulator registers (rows k, columns v)
// and the same registers, split hi/lo, are the B operand of k S and q S; the
// S update reads k^T straight from the row-major k tile with transposing LDS
// reads.  All products run on v_mfma_f32_32x32x16_bf16 with fp32
// accumulation; fp32 operands take 2-3 hi/lo passes.

#include "kad_common.h"

namespace {

constexpr int kC = 64;
constexpr int kPrepThreads = 256;

// per-token scalars of a chunk record
// (EG e^G, BT beta, ZK = beta e^G kmul (kmul the k multiplier), WU the
// state-update weight kmul e^{G_last - G}, KRS / QRS the bf16 l2norm row
// scales of k / q (1 in fp32 mode), EQ = e^G qmul (qmul the q multiplier
// incl. scale))
enum { S_EG = 0, S_BT, S_ZK, S_WU, S_KRS, S_QRS, S_EQ, kScal };
constexpr float kLog2e = 1.4426950408889634f;

// workspace record of one (sequence, head, chunk), in bytes: T' and then In
// (both strictly / non-strictly lower triangular 64 x 64) as hi/lo bf16 A
// fragments of the scan's 32x32x16 MFMAs, then fp32 [kScal][64].  Fragment
// (it, s), s < 2 (it + 1) (the others lie above the diagonal), is stored at
// index frag_index(it, s) as [plane 2][lane 64][8]: lane L holds
// X[it*32 + L%32][s*16 + (t/4)*8 + (L/32)*4 + t%4], t < 8.
struct ChunkRec {
  static constexpr int frags = 6;
  static constexpr int frag_elems = frags * 2 * 64 * 8;
  static constexpr int tf_elems = 2 * frag_elems;   // T' then In
  static constexpr size_t tf = 0;
  static constexpr size_t in = tf + frag_elems * 2;
  static constexpr size_t scal = tf + tf_elems * 2;
  static constexpr size_t bytes = scal + kScal * kC * 4;
};
__device__ __forceinline__ int frag_index(int it, int s) { return it == 0 ? s : 2 + s; }

// B fragments (hi, lo) of an fp32 accumulator tile for K step s: the 8
// accumulator entries (s%2)*8 .. +7 of 32-row tile s/2
__device__ __forceinline__ void acc_frags(const f32x16& t, int half, bf16x8& hi, bf16x8& lo) {
  float x[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = t[half * 8 + i];
  split8(x, hi, lo);
}

// x of the lane the DPP control selects (every lane valid)
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                               0xF, 0xF, true));
}

// sum of squares of a row whose CPR 16-byte slices sit in CPR consecutive
// lanes (aligned groups); hf: the squares rounded to bf16 as transformers'
// bf16 l2norm computes them.  Identical in the prep and the scan, so both
// normalise k to the same bits.
template <int CPR>
__device__ __forceinline__ float row_sumsq(const u32x4& r, bool hf) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float lo = __uint_as_float(r[e] << 16), hi = __uint_as_float(r[e] & 0xffff0000u);
    if (hf) {
      // both squares rounded by one packed conversion
      const uint32_t sq = pack_bf16x2(lo * lo, hi * hi);
      ss += __uint_as_float(sq << 16);
      ss += __uint_as_float(sq & 0xffff0000u);
    } else {
      ss += lo * lo;
      ss += hi * hi;
    }
  }
  // the row's sum on DPP lane permutes within its 16- or 8-lane row (xor 1,
  // xor 2, half-row mirror, row mirror): no LDS round trips
  static_assert(CPR == 8 || CPR == 16, "rows span 8 or 16 lanes");
  ss += dpp_f32<0xB1>(ss);   // quad_perm [1, 0, 3, 2]
  ss += dpp_f32<0x4E>(ss);   // quad_perm [2, 3, 0, 1]
  ss += dpp_f32<0x141>(ss);  // row_half_mirror
  if constexpr (CPR == 16) ss += dpp_f32<0x140>(ss);  // row_mirror
  return ss;
}

// transformers l2norm in bf16: x * rsqrt(sum(x*x) + eps), each op rounded;
// hf_l2_rs gives the row scale, hf_l2_apply the scaled slice
__device__ __forceinline__ float hf_l2_rs(float ss) {
  const float y = round_bf(round_bf(ss) + 1e-6f);
  // torch's rsqrt here is 1 / sqrt(y), each step rounded in fp32, then
  // rounded to bf16.  The hardware reciprocal square root lies within 2 ulp
  // of that, so its bf16 rounding is the same unless it sits within a few
  // ulp of a rounding midpoint (low 16 bits near 0x8000: about 1 row in
  // 4,000), where the two-step form is evaluated instead
  const float r = __builtin_amdgcn_rsqf(y);
  const int mid = (int)(__float_as_uint(r) & 0xffffu) - 0x8000;
  if (mid >= -8 && mid <= 8) return round_bf(1.0f / sqrtf(y));
  return round_bf(r);
}
__device__ __forceinline__ void hf_l2_apply(u32x4& r, float rs) {
#pragma unroll
  for (int e = 0; e < 4; ++e)
    r[e] = pack_bf16x2(__uint_as_float(r[e] << 16) * rs, __uint_as_float(r[e] & 0xffff0000u) * rs);
}

// ---------------------------------------------------------------------------
template <int K, bool HF>
__global__ __launch_bounds__(kPrepThreads) void gdn_chunk_prep(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, int64_t ld_qk,
    const void* __restrict__ g, int gdt, const void* __restrict__ beta, int bdt, int64_t ld_gate,
    uint8_t* __restrict__ ws, int T, int H, int HV, int nchunks, float scale) {
  constexpr int LD = K + 8;
  constexpr int CPR = K / 8;       // 16-byte slices per k row
  constexpr int RPI = 64 / CPR;    // rows per wave instruction
  // the bf16 k and q rows (Gram phase) and, later, A in residue-major order
  // plus the T' tile share one LDS region
  constexpr size_t kRows = 2 * kC * LD * sizeof(bf16_t);
  constexpr size_t kMats = (kC * kC + kC * (kC + 1)) * sizeof(float);
  __shared__ __attribute__((aligned(16))) unsigned char region[kRows > kMats ? kRows : kMats];
  bf16_t* kb = (bf16_t*)region;
  bf16_t* qb = kb + kC * LD;
  float* Ar = (float*)region;                         // Ar[i*64 + (j%4)*16 + j/4] = A[i][j]
  float(*Tm)[kC + 1] = (float(*)[kC + 1])(Ar + kC * kC);
  __shared__ __attribute__((aligned(16))) float Gs[kC];
  __shared__ float bt[kC], kmul[kC], krs[kC], qrs[kC], qmul[kC], g2s[kC];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = blockIdx.x % nchunks;
  const int nh = blockIdx.x / nchunks;
  const int n = nh / HV, hv = nh % HV;
  const int h = hv / (HV / H);
  const int t0 = c * kC;
  const int nt = min(kC, T - t0);
  uint8_t* rec = ws + (size_t)blockIdx.x * ChunkRec::bytes;

  // ---- k rows (normalised into LDS) and the q row scales: wave w handles
  // rows 16w..16w+15, RPI rows per instruction (lane -> row lane / CPR,
  // 16-byte slice lane % CPR).  Every load (rows past the sequence end read
  // its last row and are zeroed) goes out before the first use, so the
  // chunk pays one memory round trip.
  {
    constexpr int NIT = 16 / RPI;
    const int rsub = lane / CPR, ch = lane % CPR;
    u32x4 kr[NIT], qr[NIT];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int i = wave * 16 + it * RPI + rsub;
      const int64_t off = ((int64_t)n * T + t0 + min(i, nt - 1)) * ld_qk + (int64_t)h * K + ch * 8;
      kr[it] = *(const u32x4*)(k + off);
      qr[it] = *(const u32x4*)(q + off);
    }
    // the gate scalars after the rows: their dtype conversion waits on them
    const int gt = min(tid, nt - 1);
    const int64_t gi = ((int64_t)n * T + t0 + gt) * ld_gate + hv;
    float gv = 0.f, bv = 0.f;
    if (tid < kC) {
      gv = load_as_float(g, gi, gdt);
      bv = load_as_float(beta, gi, bdt);
    }
    if (tid < kC) {
      Gs[tid] = tid < nt ? gv : 0.f;
      bt[tid] = tid < nt ? bv : 0.f;
    }
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int i = wave * 16 + it * RPI + rsub;
      if (i >= nt) {
        kr[it] = u32x4{0, 0, 0, 0};
        qr[it] = u32x4{0, 0, 0, 0};
      }
      const float kss = row_sumsq<CPR>(kr[it], HF);
      const float qss = row_sumsq<CPR>(qr[it], HF);
      float km = 1.f, kr_s = 1.f, qr_s = 1.f, qm = scale;
      if constexpr (HF) {
        kr_s = hf_l2_rs(kss);
        qr_s = hf_l2_rs(qss);
        hf_l2_apply(kr[it], kr_s);
        hf_l2_apply(qr[it], qr_s);
      } else {
        km = 1.0f / sqrtf(kss + 1e-6f);
        qm = scale / sqrtf(qss + 1e-6f);
      }
      *(u32x4*)(kb + i * LD + ch * 8) = kr[it];
      *(u32x4*)(qb + i * LD + ch * 8) = qr[it];
      if (ch == 0) {
        kmul[i] = km;
        krs[i] = kr_s;
        qrs[i] = qr_s;
        qmul[i] = qm;
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    // sequential cumulative sum (torch.cumsum's order on the CPU), in registers
    float gv[kC];
#pragma unroll
    for (int i = 0; i < kC; i += 4) *(float4*)(gv + i) = *(const float4*)(Gs + i);
#pragma unroll
    for (int i = 1; i < kC; ++i) gv[i] += gv[i - 1];
#pragma unroll
    for (int i = 0; i < kC; i += 4) *(float4*)(Gs + i) = *(const float4*)(gv + i);
  }
  __syncthreads();
  if (tid < kC) {
    float* sc = (float*)(rec + ChunkRec::scal);
    const float eg = expf(Gs[tid]);
    sc[S_EG * kC + tid] = eg;
    sc[S_BT * kC + tid] = bt[tid];
    sc[S_ZK * kC + tid] = bt[tid] * (eg * kmul[tid]);
    sc[S_WU * kC + tid] = kmul[tid] * expf(Gs[kC - 1] - Gs[tid]);
    sc[S_KRS * kC + tid] = krs[tid];
    sc[S_QRS * kC + tid] = qrs[tid];
    sc[S_EQ * kC + tid] = eg * qmul[tid];
    g2s[tid] = Gs[tid] * kLog2e;
  }

  // ---- k k^T and (q k^T)^T: the three 32x32 tiles on or below the diagonal,
  // waves 0..2 (tile (0,1) lies above it: A and In are zero there).  The
  // In^T tile has the k tokens j as rows: its accumulator order is the K
  // order of the scan's In v_new product.
  const int ti = wave == 0 ? 0 : 1, tj = wave == 2 ? 1 : 0;
  f32x16 gram = f32x16{}, inT = f32x16{};
  if (wave < 3) {
    const int fr = lane & 31, fk = (lane >> 5) * 8;
#pragma unroll
    for (int s = 0; s < K / 16; ++s) {
      const bf16x8 a = as_bf16x8(*(const u32x4*)(kb + (ti * 32 + fr) * LD + s * 16 + fk));
      const bf16x8 b = as_bf16x8(*(const u32x4*)(kb + (tj * 32 + fr) * LD + s * 16 + fk));
      const bf16x8 bq = as_bf16x8(*(const u32x4*)(qb + (ti * 32 + fr) * LD + s * 16 + fk));
      gram = mfma32x32x16(a, b, gram);
      inT = mfma32x32x16(b, bq, inT);
    }
  }
  __syncthreads();  // rows no longer needed: the region becomes A / T'
  // In_ij = (q^_i . k^_j) qmul_i kmul_j e^{G_i - G_j} for j <= i, as hi/lo
  // A fragments (it = ti, s = tj * 2 + half) straight from the accumulators
  if (wave < 3) {
    const int irow = ti * 32 + (lane & 31);
    const float qmi = qmul[irow], gi = g2s[irow];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int j = tj * 32 + (e / 4) * 8 + (lane >> 5) * 4 + (e % 4);
      inT[e] = j <= irow ? (inT[e] * qmi * kmul[j]) * __builtin_amdgcn_exp2f(gi - g2s[j]) : 0.f;
    }
    bf16_t* inf = (bf16_t*)(rec + ChunkRec::in);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      bf16x8 ih, il;
      acc_frags(inT, half, ih, il);
      const int f = frag_index(ti, tj * 2 + half);
      *(bf16x8*)(inf + ((f * 2 + 0) * 64 + lane) * 8) = ih;
      *(bf16x8*)(inf + ((f * 2 + 1) * 64 + lane) * 8) = il;
    }
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    // wave 3 clears tile (0,1)
    const int ri = wave == 3 ? 0 : ti, rj = wave == 3 ? 1 : tj;
    const int i = ri * 32 + (e / 4) * 8 + (lane >> 5) * 4 + (e % 4);
    const int j = rj * 32 + (lane & 31);
    // the decay e^{G_i - G_j} as 2^(G_i log2 e - G_j log2 e) on the hardware
    // exp2, as for In (a few ulp from expf of the difference)
    Ar[i * kC + (j & 3) * 16 + (j >> 2)] =
        wave < 3 && j < i
            ? -bt[i] * (gram[e] * kmul[i] * kmul[j]) * __builtin_amdgcn_exp2f(g2s[i] - g2s[j])
            : 0.f;
  }
  __syncthreads();

  // ---- T' = (I - A)^-1 - I (A strictly lower) by 16 x 16 blocks, T = I + T'.
  // 1. Wave w inverts diagonal block w by forward substitution,
  //    T'[i][j] = A[i][j] + sum_{m<i} A[i][m] T'[m][j] within the block: lane
  //    (column j = 16w + lane/4, residue r = lane%4) keeps rows 16w + 4q + r
  //    in registers; rows not yet computed are zero and A is zero on and above
  //    the diagonal, so no term needs a mask.  It also clears the blocks to the
  //    right of its diagonal block.
  // 2. Wave j then walks block column j downwards on fp32 MFMAs:
  //    (I - A_ii) T_ij = sum_{m<i} A_im T_mj gives T'_ij = T_ij = P + T'_ii P
  //    with P = sum_{m=j}^{i-1} A_im T_mj.  A wave reads only the diagonal
  //    blocks and its own column's blocks, in the order it wrote them, so the
  //    walk needs no barrier.
  {
    const int col = wave * 16 + (lane >> 2), r = lane & 3;
    float treg[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int li = 1; li < 16; ++li) {
      const int i = wave * 16 + li;
      const float4 a4 = *(const float4*)(Ar + i * kC + r * 16 + wave * 4);
      float part = a4.x * treg[0];
      part += a4.y * treg[1];
      part += a4.z * treg[2];
      part += a4.w * treg[3];
      // sum over the 4 lanes of the column: DPP quad permutes (xor 1, xor 2)
      part += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                            0, __builtin_bit_cast(int, part), 0xB1, 0xF, 0xF, true));
      part += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                            0, __builtin_bit_cast(int, part), 0x4E, 0xF, 0xF, true));
      const float val = Ar[i * kC + (col & 3) * 16 + (col >> 2)] + part;
      if (r == (li & 3)) treg[li >> 2] = val;
    }
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) Tm[wave * 16 + qq * 4 + r][col] = treg[qq];
    for (int jb = wave + 1; jb < 4; ++jb)
#pragma unroll
      for (int e = 0; e < 4; ++e) Tm[wave * 16 + (lane >> 4) * 4 + e][jb * 16 + (lane & 15)] = 0.f;
  }
  __syncthreads();
  if (wave < 3) {
    // v_mfma_f32_16x16x4_f32: lane l holds A[l%16][l/16] and B[l/16][l%16];
    // accumulator element e of lane l is C[(l/16)*4 + e][l%16]
    const int jb = wave, rr = lane & 15, kq = lane >> 4;
    for (int ib = jb + 1; ib < 4; ++ib) {
      f32x4 P = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int mb = jb; mb < ib; ++mb) {
#pragma unroll
        for (int st = 0; st < 4; ++st) {
          const int kk = st * 4 + kq;
          const float av = Ar[(ib * 16 + rr) * kC + (kk & 3) * 16 + mb * 4 + (kk >> 2)];
          const float bv = Tm[mb * 16 + kk][jb * 16 + rr] + (mb == jb && kk == rr ? 1.f : 0.f);
          P = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, P, 0, 0, 0);
        }
      }
      // P goes through block (ib, jb) of Tm to become the B operand
#pragma unroll
      for (int e = 0; e < 4; ++e) Tm[ib * 16 + kq * 4 + e][jb * 16 + rr] = P[e];
      f32x4 acc = P;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        const int kk = st * 4 + kq;
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(Tm[ib * 16 + rr][ib * 16 + kk],
                                                   Tm[ib * 16 + kk][jb * 16 + rr], acc, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) Tm[ib * 16 + kq * 4 + e][jb * 16 + rr] = acc[e];
    }
  }
  __syncthreads();

  // ---- T' hi/lo in fragment order: 384 (fragment, lane) pairs
  {
    bf16_t* tf = (bf16_t*)(rec + ChunkRec::tf);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int fl_ = tid + u * kPrepThreads;
      if (fl_ >= ChunkRec::frags * 64) break;
      const int f = fl_ >> 6, L = fl_ & 63;
      const int it = f < 2 ? 0 : 1, s = f < 2 ? f : f - 2;
      const int i = it * 32 + (L & 31), jb = s * 16 + (L >> 5) * 4;
      float x[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) x[t] = Tm[i][jb + (t / 4) * 8 + t % 4];
      bf16x8 fh, fl;
      split8(x, fh, fl);
      *(bf16x8*)(tf + ((f * 2 + 0) * 64 + L) * 8) = fh;
      *(bf16x8*)(tf + ((f * 2 + 1) * 64 + L) * 8) = fl;
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

typedef short tr_v4s_t __attribute__((ext_vector_type(4)));

// A fragment of k^T for the state update: lane L gets feature kt*32 + L%32 of
// the tokens s*16 + (t/4)*8 + (L/32)*4 + t%4 (t < 8), read transposed from the
// row-major [token][feature] tile.  ds_read_b64_tr_b16: within each 16-lane
// group lane i receives element i%4 of the 8-byte pieces addressed by lanes
// 4e + i/4 (e < 4), so lane 16g + 4e + m addresses token
// s*16 + r*8 + (g/2)*4 + e, features kt*32 + (g%2)*16 + 4m .. +3.
template <int LDK>
__device__ __forceinline__ bf16x8 kt_frag(const bf16_t* kb, int kt, int s, int lane) {
  const int g = lane >> 4, e = (lane >> 2) & 3, m = lane & 3;
  tr_v4s_t part[2];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const bf16_t* p = kb + (s * 16 + r * 8 + (g >> 1) * 4 + e) * LDK + kt * 32 + (g & 1) * 16 + 4 * m;
    part[r] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) tr_v4s_t*)p);
  }
  const u32x2 lo = __builtin_bit_cast(u32x2, part[0]);
  const u32x2 up = __builtin_bit_cast(u32x2, part[1]);
  return as_bf16x8(u32x4{lo[0], lo[1], up[0], up[1]});
}

// Gated output (GATED): each output row of a value head passes through the
// model's gated RMSNorm on its way out, with the arithmetic of
// rmsnorm_gated_kernel: the row's 8-element pieces sit in CPV consecutive
// lanes as there, the same per-lane sum and butterfly over the lanes, so the
// result equals the chunk rule followed by kad_rmsnorm_gated bit for bit.
struct GateArgs {
  const bf16_t* z;     // [N*T rows, HV*V], row stride ldz
  int64_t ldz;
  const bf16_t* w;     // [V]
  float eps;
};

// sum over the `lanes` consecutive lanes (a power of two) that share a row,
// in the butterfly order of the row-wise kernels (partners lane ^ lanes/2,
// then ^ lanes/4, ...).  For 16-lane rows the partners come by DPP row
// rotations: a rotation by 8 is the xor-8 partner, and after each step the
// lanes a rotation by 4, 2 or 1 reaches hold the xor partner's value, so the
// sums are the same bits without LDS round trips.
template <int LANES>
__device__ __forceinline__ float lane_group_sum(float v) {
  if constexpr (LANES == 16) {
    v += dpp_f32<0x128>(v);   // row_ror:8
    v += dpp_f32<0x124>(v);   // row_ror:4
    v += dpp_f32<0x122>(v);   // row_ror:2
    v += dpp_f32<0x121>(v);   // row_ror:1
  } else {
#pragma unroll
    for (int o = LANES / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  }
  return v;
}

template <int K, int V, bool HF, bool GATED>
__global__ __launch_bounds__(V * 2, V == 128 ? 2 : 1) void gdn_chunk_scan(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ k, int64_t ld_qk,
    const bf16_t* __restrict__ v, int64_t ld_v, const uint8_t* __restrict__ ws,
    const void* __restrict__ state0, int sdt, int beams_per_state, bf16_t* __restrict__ out,
    int64_t ld_out, float* __restrict__ final_state, int T, int H, int HV, int nchunks,
    GateArgs gate) {
  constexpr int KT = K / 32;      // 32-row k tiles of S
  constexpr int KS = K / 16;      // k16 steps over K
  constexpr int LDK = K + 8;      // bf16 [64][K] rows (16-byte padding)
  constexpr int LDV = V + 8;
  constexpr int NTH = V * 2;
  constexpr int CPR = K / 8;      // 16-byte slices per q/k row
  __shared__ __attribute__((aligned(16))) bf16_t kb[kC * LDK];
  __shared__ __attribute__((aligned(16))) bf16_t qb[kC * LDK];
  __shared__ __attribute__((aligned(16))) bf16_t vb[kC * LDV];
  __shared__ __attribute__((aligned(16))) bf16_t tf[ChunkRec::tf_elems];
  __shared__ float sc[kScal][kC];

  const int tid0 = threadIdx.x, wave = tid0 >> 6;
  const int n = blockIdx.x / HV, hv = blockIdx.x % HV;
  const int h = hv / (HV / H);

  // S[k][vcol] in accumulator layout: tile kt, entry e -> k = kt*32 + (e/4)*8 + hi*4 + e%4
  f32x16 S[KT];
  {
    const int lane = tid0 & 63, hi = lane >> 5, vcol = wave * 32 + (lane & 31);
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
  }

  // the chunk's global data pass through registers into LDS; all loads are
  // issued before the barrier, so their latency is paid once per chunk (and
  // the second workgroup on the CU computes meanwhile).  Prefetching the next
  // chunk instead needs the registers of a second workgroup (issuing its
  // loads before the output stage spills 32-128 registers).
  constexpr int kRowU = kC * CPR / NTH;               // q/k slices per thread
  constexpr int kVU = kC * V / 8 / NTH;               // v slices per thread
  constexpr int kTU = ChunkRec::tf_elems / 8 / NTH;   // T' slices per thread
  constexpr int kSU = (kScal * kC + NTH - 1) / NTH;
  static_assert(kRowU * NTH == kC * CPR && kVU * NTH * 8 == kC * V &&
                    kTU * NTH * 8 == ChunkRec::tf_elems && NTH % CPR == 0,
                "chunk tiles must split evenly");
  u32x4 rk[kRowU], rq[kRowU], rv[kVU], rt[kTU];
  float rs[kSU], krs_u[kRowU], qrs_u[kRowU];
  auto fetch = [&](int c, int tid) {
    const int t0 = c * kC, nt = min(kC, T - t0);
    const int64_t row0 = (int64_t)n * T + t0;
    const uint8_t* rec = ws + ((size_t)blockIdx.x * nchunks + c) * ChunkRec::bytes;
    const float* scg = (const float*)(rec + ChunkRec::scal);
#pragma unroll
    for (int u = 0; u < kRowU; ++u) {
      const int e = tid + u * NTH;
      const int i = e / CPR, ch = e % CPR;
      const bool live = i < nt;
      const int64_t off = (row0 + (live ? i : 0)) * ld_qk + (int64_t)h * K + ch * 8;
      rk[u] = live ? *(const u32x4*)(k + off) : u32x4{0u, 0u, 0u, 0u};
      rq[u] = live ? *(const u32x4*)(q + off) : u32x4{0u, 0u, 0u, 0u};
      krs_u[u] = scg[S_KRS * kC + i];
      qrs_u[u] = scg[S_QRS * kC + i];
    }
#pragma unroll
    for (int u = 0; u < kVU; ++u) {
      const int e = tid + u * NTH;
      const int i = e / (V / 8), v8 = (e % (V / 8)) * 8;
      rv[u] = i < nt ? *(const u32x4*)(v + (row0 + i) * ld_v + (int64_t)hv * V + v8)
                     : u32x4{0u, 0u, 0u, 0u};
    }
    const bf16_t* tfg = (const bf16_t*)(rec + ChunkRec::tf);
#pragma unroll
    for (int u = 0; u < kTU; ++u) rt[u] = *(const u32x4*)(tfg + (tid + u * NTH) * 8);
#pragma unroll
    for (int u = 0; u < kSU; ++u) {
      const int e = tid + u * NTH;
      rs[u] = e < kScal * kC ? scg[e] : 0.f;
    }
  };
  // q and k rows normalised with the prep's row scales (bit-identical to the
  // prep's own k rows)
  auto stash = [&](int tid) {
#pragma unroll
    for (int u = 0; u < kRowU; ++u) {
      const int e = tid + u * NTH;
      const int i = e / CPR, ch = e % CPR;
      if constexpr (HF) {
        hf_l2_apply(rk[u], krs_u[u]);
        hf_l2_apply(rq[u], qrs_u[u]);
      }
      *(u32x4*)(kb + i * LDK + ch * 8) = rk[u];
      *(u32x4*)(qb + i * LDK + ch * 8) = rq[u];
    }
#pragma unroll
    for (int u = 0; u < kVU; ++u) {
      const int e = tid + u * NTH;
      const int i = e / (V / 8), v8 = (e % (V / 8)) * 8;
      *(u32x4*)(vb + i * LDV + v8) = rv[u];
    }
#pragma unroll
    for (int u = 0; u < kTU; ++u) *(u32x4*)(tf + (tid + u * NTH) * 8) = rt[u];
#pragma unroll
    for (int u = 0; u < kSU; ++u) {
      const int e = tid + u * NTH;
      if (e < kScal * kC) sc[e / kC][e % kC] = rs[u];
    }
  };

  constexpr int kOUG = kC * (V / 8) / NTH;   // output pieces per thread
  for (int c = 0; c < nchunks; ++c) {
    // lane-derived indices are recomputed from an opaque copy of the thread
    // id every chunk, so the compiler does not keep dozens of precomputed
    // addresses live across the loop
    int tid = tid0;
    asm volatile("" : "+v"(tid));
    const int lane = tid & 63, hi = lane >> 5, col = lane & 31;
    const int vcol = wave * 32 + col;  // this lane's value column
    const int t0 = c * kC;
    const int nt = min(kC, T - t0);
    const int64_t row0 = (int64_t)n * T + t0;
    fetch(c, tid);
    // the gate rows of this thread's output pieces, loaded with the chunk's
    // inputs (their latency is not on the store path)
    u32x4 zr[GATED ? kOUG : 1], wr = u32x4{0u, 0u, 0u, 0u};
    if constexpr (GATED) {
#pragma unroll
      for (int u = 0; u < kOUG; ++u) {
        const int i = min((tid + u * NTH) / (V / 8), nt - 1);
        zr[u] = *(const u32x4*)(gate.z + (row0 + i) * gate.ldz + (int64_t)hv * V + (tid % (V / 8)) * 8);
      }
      wr = *(const u32x4*)(gate.w + (tid % (V / 8)) * 8);
    }
    __syncthreads();  // previous chunk done with LDS
    stash(tid);
    __syncthreads();

    // ---- k S and q S for both 32-token tiles, S split hi/lo per k16 step
    f32x16 KSa[2], QSa[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
      KSa[tt] = f32x16{};
      QSa[tt] = f32x16{};
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      bf16x8 shf, slf;
      acc_frags(S[s / 2], s % 2, shf, slf);
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        const bf16x8 ak = perm_frag(kb + (tt * 32 + col) * LDK, s * 16, hi);
        const bf16x8 aq = perm_frag(qb + (tt * 32 + col) * LDK, s * 16, hi);
        KSa[tt] = mfma32x32x16(ak, shf, KSa[tt]);
        KSa[tt] = mfma32x32x16(ak, slf, KSa[tt]);
        QSa[tt] = mfma32x32x16(aq, shf, QSa[tt]);
        QSa[tt] = mfma32x32x16(aq, slf, QSa[tt]);
      }
      // one step of fragments in flight at a time keeps the register count
      // within the two-workgroups-per-CU budget
      __builtin_amdgcn_sched_barrier(0);
    }
    // ---- Z_j = beta_j (v_j - e^{G_j} kmul_j (k S)_j) = beta_j v_j - ZK_j (k S)_j
    f32x16 Z[2];
#pragma unroll
    for (int jt = 0; jt < 2; ++jt) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int j = jt * 32 + (e / 4) * 8 + hi * 4 + (e % 4);
        const float vj = bf2f(vb[j * LDV + vcol]);
        Z[jt][e] = fmaf(-sc[S_ZK][j], KSa[jt][e], sc[S_BT][j] * vj);
      }
    }
    // ---- v_new = Z + T' Z (T' strictly lower: rows 0..31 see tokens 0..31)
    bf16x8 zh[4], zl[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) acc_frags(Z[s / 2], s % 2, zh[s], zl[s]);
    f32x16 VN[2];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      f32x16 acc = Z[it];
#pragma unroll
      for (int s = 0; s < 2 * (it + 1); ++s) {
        const int f = frag_index(it, s);
        const bf16x8 ah = *(const bf16x8*)(tf + ((f * 2 + 0) * 64 + lane) * 8);
        const bf16x8 al = *(const bf16x8*)(tf + ((f * 2 + 1) * 64 + lane) * 8);
        acc = mfma32x32x16(ah, zh[s], acc);
        acc = mfma32x32x16(ah, zl[s], acc);
        acc = mfma32x32x16(al, zh[s], acc);
      }
      VN[it] = acc;
    }
    // v_new as B fragments (hi + lo carries it to 2^-16 relative; the state
    // update takes its weights from them, which keeps the register count
    // within budget)
    bf16x8 vh[4], vl[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) acc_frags(VN[s / 2], s % 2, vh[s], vl[s]);
    // ---- o_i = e^{G_i} qmul_i (q S)_i + sum_{j<=i} In_ij v_new_j, In from
    // the prep's fragments
    const bf16_t* inb = tf + ChunkRec::frag_elems;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      f32x16& o = QSa[it];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int i = it * 32 + (e / 4) * 8 + hi * 4 + (e % 4);
        o[e] *= sc[S_EQ][i];
      }
#pragma unroll
      for (int s = 0; s < 2 * (it + 1); ++s) {
        const int f = frag_index(it, s);
        const bf16x8 ih = *(const bf16x8*)(inb + ((f * 2 + 0) * 64 + lane) * 8);
        const bf16x8 il = *(const bf16x8*)(inb + ((f * 2 + 1) * 64 + lane) * 8);
        o = mfma32x32x16(ih, vh[s], o);
        o = mfma32x32x16(ih, vl[s], o);
        o = mfma32x32x16(il, vh[s], o);
      }
    }
    // ---- output: o goes through LDS (the v tile, which every wave has
    // finished reading after the barrier) and leaves as 16-byte row slices;
    // the state update runs between the two barriers
    constexpr int CPV = V / 8;                // 16-byte slices per output row
    constexpr int kOU = kC * CPV / NTH;       // slices per thread
    static_assert(kOU * NTH == kC * CPV && NTH % CPV == 0, "output tile must split evenly");
    const int och = tid % CPV;
    __syncthreads();
#pragma unroll
    for (int it = 0; it < 2; ++it)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int i = it * 32 + (e / 4) * 8 + hi * 4 + (e % 4);
        vb[i * LDV + vcol] = f2bf(QSa[it][e]);
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
        x[i8] = ((float)vh[s][i8] + (float)vl[s][i8]) * sc[S_WU][i];
      }
      split8(x, wh[s], wl[s]);
    }
    const float egl = sc[S_EG][kC - 1];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      f32x16 acc = S[kt];
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] *= egl;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 a = kt_frag<LDK>(kb, kt, s, lane);
        acc = mfma32x32x16(a, wh[s], acc);
        acc = mfma32x32x16(a, wl[s], acc);
      }
      S[kt] = acc;
    }
    __syncthreads();
    if constexpr (GATED) {
#pragma unroll
      for (int u = 0; u < kOU; ++u) {
        const int i = (tid + u * NTH) / CPV;
        const u32x4 ov = *(const u32x4*)(vb + i * LDV + och * 8);
        float f[8], wv[8], zv[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          f[2 * e] = __uint_as_float(ov[e] << 16);
          f[2 * e + 1] = __uint_as_float(ov[e] & 0xffff0000u);
          wv[2 * e] = __uint_as_float(wr[e] << 16);
          wv[2 * e + 1] = __uint_as_float(wr[e] & 0xffff0000u);
          zv[2 * e] = __uint_as_float(zr[u][e] << 16);
          zv[2 * e + 1] = __uint_as_float(zr[u][e] & 0xffff0000u);
        }
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
        ss = lane_group_sum<CPV>(ss);
        const float r = 1.0f / sqrtf(ss / (float)V + gate.eps);
        // each bf16 rounding of a pair as one packed conversion (the same
        // bits as rounding the elements one by one)
        u32x4 y;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t nb = pack_bf16x2(f[2 * e] * r, f[2 * e + 1] * r);
          const uint32_t wb = pack_bf16x2(wv[2 * e] * __uint_as_float(nb << 16),
                                          wv[2 * e + 1] * __uint_as_float(nb & 0xffff0000u));
          y[e] = pack_bf16x2(__uint_as_float(wb << 16) * silu_fast(zv[2 * e]),
                             __uint_as_float(wb & 0xffff0000u) * silu_fast(zv[2 * e + 1]));
        }
        if (i < nt) *(u32x4*)(out + (row0 + i) * ld_out + (int64_t)hv * V + och * 8) = y;
      }
    } else {
#pragma unroll
      for (int u = 0; u < kOU; ++u) {
        const int i = (tid + u * NTH) / CPV;
        const u32x4 ov = *(const u32x4*)(vb + i * LDV + och * 8);
        if (i < nt) *(u32x4*)(out + (row0 + i) * ld_out + (int64_t)hv * V + och * 8) = ov;
      }
    }
  }
  if (final_state) {
    const int lane = tid0 & 63, hi = lane >> 5, vcol = wave * 32 + (lane & 31);
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
                 void* ws, int N, int T, int H, int HV, float scale, int hf_norm,
                 const GateArgs* gate, hipStream_t s) {
  const int nchunks = (T + kC - 1) / kC;
  const int64_t nrec = (int64_t)N * HV * nchunks;
  const GateArgs ga = gate ? *gate : GateArgs{nullptr, 0, nullptr, 0.f};
  // transformers' bf16 l2norm rounding (hf_norm) or the operator's fp32
  // scales: an instantiation each, so the VALU-bound loops carry no test
#define KAD_CHUNK(HFV, GV)                                                                     \
  hipLaunchKernelGGL((gdn_chunk_prep<K, HFV>), dim3((unsigned)nrec), dim3(kPrepThreads), 0, s, \
                     (const bf16_t*)q, (const bf16_t*)k, ld_qk, g, gdt, beta, bdt, ld_gate,    \
                     (uint8_t*)ws, T, H, HV, nchunks, scale);                                  \
  if (const int rc = kad_launch_status("gdn_chunk_prep")) return rc;                           \
  hipLaunchKernelGGL((gdn_chunk_scan<K, V, HFV, GV>), dim3((unsigned)((int64_t)N * HV)),      \
                     dim3(V * 2), 0, s, (const bf16_t*)q, (const bf16_t*)k, ld_qk,             \
                     (const bf16_t*)v, ld_v, (const uint8_t*)ws, state0, sdt, bps,             \
                     (bf16_t*)out, ld_out, fin, T, H, HV, nchunks, ga);                        \
  return kad_launch_status("gdn_chunk_scan")
  // the gated output only with the transformers normalisation (the model
  // prefill, whose layer applies the norm)
  if (gate) {
    KAD_CHUNK(true, true);
  }
  if (hf_norm) {
    KAD_CHUNK(true, false);
  }
  KAD_CHUNK(false, false);
#undef KAD_CHUNK
}

int64_t chunk_ws_bytes(int N, int T, int HV) {
  return (int64_t)N * HV * ((T + kC - 1) / kC) * (int64_t)ChunkRec::bytes;
}

int chunk_common(const void* q, const void* k, const void* v, int64_t ld_qk, int64_t ld_v,
                 int qkv_dtype, const void* log_decay, int gate_dtype, const void* beta,
                 int beta_dtype, int64_t ld_gate, const void* initial_state, int state_dtype,
                 int beams_per_state, void* out, int64_t ld_out,
                 float* final_state, void* workspace, int64_t workspace_bytes, int N, int T,
                 int H, int HV, int K, int V, float scale, int transformers_l2norm,
                 const GateArgs* gate, hipStream_t s) {
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
  KAD_REQUIRE(ld_out % 8 == 0 && ((uintptr_t)out % 16) == 0, "out rows must be 16-byte aligned");
  if (qkv_dtype != KAD_DTYPE_BF16) KAD_UNSUPPORTED("chunked gated delta takes bf16 q/k/v");
  if (!((K == 64 || K == 128) && (V == 64 || V == 128)))
    KAD_UNSUPPORTED("chunked gated delta supports K, V in {64, 128}; got K=%d V=%d", K, V);
  const int64_t need = chunk_ws_bytes(N, T, HV);
  KAD_REQUIRE(workspace_bytes >= need, "workspace of %lld bytes is smaller than %lld",
              (long long)workspace_bytes, (long long)need);
  KAD_REQUIRE(((uintptr_t)workspace % 16) == 0, "workspace must be 16-byte aligned");
  if (gate) {
    KAD_REQUIRE(gate->z && gate->w, "null pointer argument");
    KAD_REQUIRE(transformers_l2norm, "the gated output takes the transformers l2norm");
    KAD_REQUIRE(gate->ldz >= (int64_t)HV * V && gate->ldz % 8 == 0 &&
                    ((uintptr_t)gate->z % 16) == 0 && ((uintptr_t)gate->w % 16) == 0,
                "z rows and the norm weight must be 16-byte aligned, ldz >= HV*V");
  }
#define KAD_CHUNK(KK, VV)                                                                      \
  if (K == KK && V == VV)                                                                      \
    return launch_chunk<KK, VV>(q, k, v, ld_qk, ld_v, log_decay, gate_dtype, beta, beta_dtype, \
                                ld_gate, initial_state, state_dtype, beams_per_state, out,     \
                                ld_out, final_state, workspace, N, T, H, HV, scale,            \
                                transformers_l2norm, gate, s);
  KAD_CHUNK(128, 128)
  KAD_CHUNK(64, 64)
  KAD_CHUNK(128, 64)
  KAD_CHUNK(64, 128)
#undef KAD_CHUNK
  KAD_UNSUPPORTED("unreachable");
}

}  // namespace

extern "C" int kad_gdn_chunk_workspace_bytes(int N, int T, int HV, int K, int64_t* bytes) {
  KAD_REQUIRE(bytes, "null pointer argument");
  KAD_REQUIRE(N > 0 && T > 0 && HV > 0, "bad dimensions");
  if (K != 64 && K != 128) KAD_UNSUPPORTED("chunked gated delta supports K in {64, 128}");
  *bytes = chunk_ws_bytes(N, T, HV);
  return KAD_OK;
}

extern "C" int kad_gdn_chunk(const void* q, const void* k, const void* v, int64_t ld_qk,
                             int64_t ld_v, int qkv_dtype, const void* log_decay, int gate_dtype,
                             const void* beta, int beta_dtype, int64_t ld_gate,
                             const void* initial_state, int state_dtype, int beams_per_state,
                             void* out, int64_t ld_out, float* final_state, void* workspace,
                             int64_t workspace_bytes, int N, int T, int H, int HV, int K, int V,
                             float scale, int transformers_l2norm, kad_stream_t stream) {
  return chunk_common(q, k, v, ld_qk, ld_v, qkv_dtype, log_decay, gate_dtype, beta, beta_dtype,
                      ld_gate, initial_state, state_dtype, beams_per_state, out, ld_out,
                      final_state, workspace, workspace_bytes, N, T, H, HV, K, V, scale,
                      transformers_l2norm, nullptr, (hipStream_t)stream);
}

extern "C" int kad_gdn_chunk_gated(const void* q, const void* k, const void* v, int64_t ld_qk,
                                   int64_t ld_v, int qkv_dtype, const void* log_decay,
                                   int gate_dtype, const void* beta, int beta_dtype,
                                   int64_t ld_gate, const void* initial_state, int state_dtype,
                                   int beams_per_state, void* out, int64_t ld_out,
                                   float* final_state, void* workspace, int64_t workspace_bytes,
                                   int N, int T, int H, int HV, int K, int V, float scale,
                                   const void* z, int64_t ldz, const void* norm_w, float eps,
                                   kad_stream_t stream) {
  const GateArgs ga{(const bf16_t*)z, ldz, (const bf16_t*)norm_w, eps};
  return chunk_common(q, k, v, ld_qk, ld_v, qkv_dtype, log_decay, gate_dtype, beta, beta_dtype,
                      ld_gate, initial_state, state_dtype, beams_per_state, out, ld_out,
                      final_state, workspace, workspace_bytes, N, T, H, HV, K, V, scale, 1, &ga,
                      (hipStream_t)stream);
}
