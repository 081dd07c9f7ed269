// Full-vocabulary log-softmax + beam top-k + history update (gfx950).
//
// Replaces the per-request selection loop of src/kadllm/grbeam.py:89-104:
//   logp = logits[r].float().log_softmax(-1); logp[~mask] = -inf;
//   logp += scores[r, :, None]; top-W of logp.reshape(-1) (sorted);
//   parents = idx // V; tokens = idx % V; history = cat(history[parents], tokens)
// without materialising any [W, V] fp32 temporary.
//
// Stage 1, kad_beam_row_select (one workgroup per beam row): a first pass
// takes the row max and a 4096-bin histogram of the top 12 bits of the bf16
// order key of every allowed logit; a second pass sums exp(x - max) for the
// row's log-sum-exp and resolves the low 4 bits inside the bin that holds the
// row's K-th largest logit, giving its exact value; a third pass emits exactly
// the row's K best entries (ties taken in column order).  Within a row the score
// order is the logit order, so the request's top W is among these rows'
// top min(W, V) entries.  Keys are ((x - max) - log(sum exp)) + parent in fp32.
//
// Stage 2, kad_beam_merge_select (one workgroup per request): an 8-bit radix
// select over the request's Wp*K candidate keys finds the W-th key, a second
// radix select over flat indices resolves ties (lower flat index first), and
// the W winners are bitonic-sorted by (key desc, index asc) in LDS, for W up
// to 16384.  kad_beam_merge_select_wide serves wider levels (the reference's
// topk has no width cap): the same radix rounds, histogrammed by many
// workgroups per request, and the winners sorted in caller workspace.
//
// Stage 3, kad_beam_history: new_history[b, w] = [history[b, parent], token].

#include "kad_common.h"

#include <algorithm>
#include <mutex>

// Scratch of kad_beam_select_noalloc (32 MiB per GPU; see scratch_address).
static __device__ __align__(256) uint8_t scratch[32ll << 20];

namespace {

constexpr int kRowThreads = 256;
constexpr int kBins = 4096;

__device__ __forceinline__ uint32_t order16(uint16_t bits) {
  return (bits & 0x8000u) ? (uint32_t)(~bits & 0xffffu) : (uint32_t)(bits | 0x8000u);
}
__device__ __forceinline__ uint32_t order32(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// block-wide exclusive scan of one int per thread (blockDim = kRowThreads)
__device__ int block_exclusive_scan(int v, int* scratch, int* total) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) scratch[wave] = x;
  __syncthreads();
  int base = 0, tot = 0;
  for (int w = 0; w < kRowThreads / 64; ++w) {
    if (w < wave) base += scratch[w];
    tot += scratch[w];
  }
  __syncthreads();
  *total = tot;
  return base + x - v;
}

__device__ void row_select_exact(int64_t row,
    const bf16_t* __restrict__ logits, int64_t ld, const uint8_t* __restrict__ mask,
    int64_t ld_mask, const float* __restrict__ parent, int Wp, int V, int K,
    float* __restrict__ cand_key, int* __restrict__ cand_idx, int* hist) {
  __shared__ int scan_tmp[kRowThreads / 64];
  __shared__ float red_m[kRowThreads / 64], red_s[kRowThreads / 64];
  __shared__ int sh_bin, sh_above, sh_low;
  __shared__ int sh_emit;
  const int tid = threadIdx.x;
  const bf16_t* x = logits + row * ld;
  const uint8_t* mk = mask ? mask + row * ld_mask : nullptr;

  for (int i = tid; i < kBins; i += kRowThreads) hist[i] = 0;
  if (tid == 0) sh_emit = 0;
  __syncthreads();

  // pass 1: max over all logits (log_softmax normalises before masking);
  // histogram of the order keys of the allowed logits
  float m = -INFINITY;
  for (int c = tid; c < V; c += kRowThreads) {
    const uint16_t bits = x[c];
    m = fmaxf(m, bf2f(bits));
    const bool ok = mk ? mk[c] != 0 : true;
    atomicAdd(&hist[ok ? (order16(bits) >> 4) : 0], 1);
  }
  m = wave_max(m);
  if ((tid & 63) == 0) red_m[tid >> 6] = m;
  __syncthreads();
  float M = -INFINITY;
  for (int w = 0; w < kRowThreads / 64; ++w) M = fmaxf(M, red_m[w]);

  // find the bin holding the K-th largest allowed key (masked entries count
  // in bin 0 so that rows with fewer than K allowed logits still yield K)
  if (tid == 0) {
    int acc = 0, b = kBins - 1;
    for (; b > 0; --b) {
      if (acc + hist[b] >= K) break;
      acc += hist[b];
    }
    sh_bin = b;
    sh_above = acc;  // entries in bins above b
  }
  __syncthreads();
  const int bin = sh_bin;
  for (int i = tid; i < 16; i += kRowThreads) hist[i] = 0;
  __syncthreads();

  // pass 2: exact sum exp(x - M); low-4-bit histogram inside `bin`
  float se = 0.f;
  for (int c = tid; c < V; c += kRowThreads) {
    const uint16_t bits = x[c];
    se += expf(bf2f(bits) - M);
    const bool ok = mk ? mk[c] != 0 : true;
    const uint32_t u = ok ? order16(bits) : 0u;
    if ((int)(u >> 4) == bin) atomicAdd(&hist[u & 15], 1);
  }
  se = wave_sum(se);
  if ((tid & 63) == 0) red_s[tid >> 6] = se;
  __syncthreads();
  if (tid == 0) {
    int acc = sh_above, lo = 15;
    for (; lo > 0; --lo) {
      if (acc + hist[lo] >= K) break;
      acc += hist[lo];
    }
    sh_low = lo;
    sh_above = acc;  // entries strictly above the threshold key
  }
  __syncthreads();
  float SE = 0.f;
  for (int w = 0; w < kRowThreads / 64; ++w) SE += red_s[w];
  const float lse = logf(SE);
  const uint32_t thr = ((uint32_t)bin << 4) | (uint32_t)sh_low;
  const int need_ties = K - sh_above;
  const float p = parent[row];
  const int r_local = (int)(row % Wp);
  float* ck = cand_key + row * K;
  int* ci = cand_idx + row * K;

  // pass 3: emit entries above the threshold, and the first `need_ties`
  // threshold entries in column order (tiles of kRowThreads consecutive columns)
  int ties_taken = 0;
  for (int c0 = 0; c0 < V; c0 += kRowThreads) {
    const int c = c0 + tid;
    uint32_t u = 0;
    float v = -INFINITY;
    bool ok = false;
    if (c < V) {
      const uint16_t bits = x[c];
      ok = mk ? mk[c] != 0 : true;
      u = ok ? order16(bits) : 0u;
      v = bf2f(bits);
    }
    const bool above = c < V && u > thr;
    const bool tie = c < V && u == thr;
    int tot = 0;
    const int rank = block_exclusive_scan(tie ? 1 : 0, scan_tmp, &tot);
    const bool take_tie = tie && (ties_taken + rank < need_ties);
    if (above || take_tie) {
      const int slot = atomicAdd(&sh_emit, 1);
      const float key = ok ? ((v - M) - lse) + p : -INFINITY;
      if (slot < K) {  // exactly K entries qualify; the bound only guards memory
        ck[slot] = key;
        ci[slot] = r_local * V + c;
      }
    }
    ties_taken += tot;
  }
}


// LDS candidate capacity: 2048 (16 KB) while about 2K + 256 <= 1024
// candidates are expected, which leaves room for two workgroups more per CU
// than 4096 (32 KB); the samples (bf16 keys) and the exact path's 4096-bin
// histogram alias the same buffer
constexpr int kCandCapSmall = 2048, kCandCapLarge = 4096;
constexpr int kLine = 64;                      // logits per 128-byte line
constexpr int kTargetLines = 128;              // sampled lines per row (~8k samples)

// r-th largest of the keys histogrammed in hist[256] (bin 0 excluded), run by
// one full wave: lane l owns bins 4l..4l+3.  Returns the bin and, through
// *above, how many keys lie in higher bins; bin -1 if fewer than r keys.
__device__ int wave_rank_bin(const int* hist, int r, int* above) {
  const int lane = threadIdx.x & 63;
  int b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = (lane == 0 && i == 0) ? 0 : hist[lane * 4 + i];
  const int t = b[0] + b[1] + b[2] + b[3];
  int suf = t;  // keys in lanes >= lane
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_down(suf, o, 64);
    if (lane + o < 64) suf += y;
  }
  const uint64_t reach = __ballot(suf >= r);
  const int L = __popcll(reach) - 1;  // suffix sums fall with the lane: reach is a prefix
  int bin = -1, acc = 0;
  if (L >= 0 && lane == L) {
    acc = suf - t;
    for (int i = 3; i >= 0; --i) {
      if (acc + b[i] >= r) {
        bin = lane * 4 + i;
        break;
      }
      acc += b[i];
    }
  }
  if (L < 0) return -1;
  *above = __shfl(acc, L, 64);
  return __shfl(bin, L, 64);
}

// Fast path, one workgroup per beam row:
//  1. sample every line_stride-th 128-byte line of the row and take the
//     rank-th largest sampled key (exact, two 8-bit radix rounds); about
//     rank * line_stride >= 2K + 256 entries are expected at or above it;
//  2. one vectorised pass over the row computes the max and the sum of exp
//     (online rescaling) and gathers every allowed entry at or above the
//     threshold into LDS;
//  3. a radix select over the candidates' keys (ties at the K-th key ranked by
//     column) emits the row's top K, unordered: the merge stage orders them.
// If fewer than K or more than CAP entries qualify, the exact histogram path
// runs instead, so the result never depends on the sample.
template <int CAP, bool MASKED>
__global__ __launch_bounds__(kRowThreads) void row_select_kernel(
    const bf16_t* __restrict__ logits, int64_t ld, const uint8_t* __restrict__ mask,
    int64_t ld_mask, const float* __restrict__ parent, int Wp, int V, int K,
    float* __restrict__ cand_key, int* __restrict__ cand_idx, int line_stride, int rank) {
  constexpr int kSampleCap = CAP * 4;   // bf16 sample keys aliasing the candidates
  static_assert(CAP * 8 >= 4096 * 4, "the exact path's histogram must fit the buffer");
  __shared__ __attribute__((aligned(16))) uint64_t cand[CAP];
  __shared__ int hist[256];
  __shared__ float red_m[kRowThreads / 64], red_s[kRowThreads / 64], red_smax[kRowThreads / 64];
  __shared__ int sh_count, sh_hi, sh_above, sh_thr;
  uint16_t* samples = (uint16_t*)cand;
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;
  const bf16_t* x = logits + row * ld;
  // a separate instantiation for unmasked rows drops the mask tests from the
  // per-logit loop, which is VALU-bound
  const uint8_t* mk = MASKED ? mask + row * ld_mask : nullptr;
  const bool vec = (ld % 8) == 0 && (((uintptr_t)logits) % 16) == 0 &&
                   (!mask || ((ld_mask % 8) == 0 && (((uintptr_t)mask) % 8) == 0));
  auto key_of = [&](uint16_t bits, int c) -> uint32_t {
    return (mk && mk[c] == 0) ? 0u : order16(bits);
  };

  // ---- 1. sample and threshold
  const int nlines = (V + kLine - 1) / kLine;
  const int ns = min(kSampleCap, ((nlines + line_stride - 1) / line_stride) * kLine);
  hist[tid] = 0;
  if (tid == 0) sh_count = 0;
  __syncthreads();
  float smax = -INFINITY;  // max sampled logit (masked or not): the sum's start
  for (int s = tid; s < ns; s += kRowThreads) {
    const int c = (s / kLine) * line_stride * kLine + (s % kLine);
    uint32_t k = 0u;
    if (c < V) {
      const uint16_t bits = x[c];
      k = key_of(bits, c);
      smax = fmaxf(smax, bf2f(bits));
    }
    samples[s] = (uint16_t)k;
    atomicAdd(&hist[k >> 8], 1);
  }
  smax = wave_max(smax);
  if ((tid & 63) == 0) red_smax[tid >> 6] = smax;
  __syncthreads();
  if (tid < 64) {
    int above = 0;
    const int hi = wave_rank_bin(hist, rank, &above);
    if (tid == 0) {
      sh_hi = hi;
      sh_above = above;
    }
  }
  __syncthreads();
  const int hi = sh_hi;
  if (hi > 0) {
    hist[tid] = 0;
    __syncthreads();
    for (int s = tid; s < ns; s += kRowThreads) {
      const uint32_t k = samples[s];
      if ((int)(k >> 8) == hi) atomicAdd(&hist[k & 255], 1);
    }
    __syncthreads();
    if (tid < 64) {
      // bin 0 of this round is a real key (hi > 0): count it
      const int lane = tid;
      int b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) b[i] = hist[lane * 4 + i];
      const int t = b[0] + b[1] + b[2] + b[3];
      int suf = t;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_down(suf, o, 64);
        if (lane + o < 64) suf += y;
      }
      const int need = rank - sh_above;
      const uint64_t reach = __ballot(suf >= need);
      const int L = __popcll(reach) - 1;  // need <= keys in bin hi, so L >= 0
      if (lane == L) {
        int acc = suf - t, lo = 0;
        for (int i = 3; i >= 0; --i) {
          if (acc + b[i] >= need) {
            lo = lane * 4 + i;
            break;
          }
          acc += b[i];
        }
        sh_thr = (hi << 8) | lo;
      }
    }
  } else if (tid == 0) {
    sh_thr = 0;
  }
  __syncthreads();
  const uint32_t thr = (uint32_t)sh_thr;

  // ---- 2. max, sum exp, and candidates >= thr in one pass.  The sum is taken
  // against a fixed reference, the sample max (each term one fma and the
  // hardware exp2: exp(v - m) = 2^(v log2 e - m log2 e)); a row whose true max
  // exceeds it by more than 60 sums again against the true max.  Candidates
  // are screened with a float compare against the threshold's value and
  // confirmed on the order key.
  constexpr float kLog2e = 1.4426950408889634f;
  float mref = -INFINITY;
  for (int w = 0; w < kRowThreads / 64; ++w) mref = fmaxf(mref, red_smax[w]);
  if (mref == -INFINITY) mref = 0.f;
  float m = -INFINITY, se = 0.f;
  float nb = -mref * kLog2e;
  const uint32_t tb = thr & 0x8000u ? (thr & 0x7fffu) : (~thr & 0xffffu);
  const float tf = thr > 0 ? bf2f((uint16_t)tb) : INFINITY;
  auto visit = [&](uint16_t bits, int c, bool ok) {
    const float v = bf2f(bits);
    m = fmaxf(m, v);
    se += __builtin_amdgcn_exp2f(fmaf(v, kLog2e, nb));
    if (v >= tf && ok) {
      const uint32_t u = order16(bits);
      if (u >= thr) {
        const int slot = atomicAdd(&sh_count, 1);
        if (slot < CAP) cand[slot] = ((uint64_t)u << 32) | (uint64_t)(0xffffffffu - (uint32_t)c);
      }
    }
  };
  const int V8 = vec ? V / 8 : 0;
  constexpr int kUnroll = 4;
  int c8 = tid;
  for (; c8 + (kUnroll - 1) * kRowThreads < V8; c8 += kUnroll * kRowThreads) {
    u32x4 r[kUnroll];
    u32x2 mr[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      r[u] = *(const u32x4*)(x + (c8 + u * kRowThreads) * 8);
      if (mk) mr[u] = *(const u32x2*)(mk + (c8 + u * kRowThreads) * 8);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int c = (c8 + u * kRowThreads) * 8;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool ok0 = mk ? ((mr[u][e / 2] >> (16 * (e % 2))) & 0xffu) != 0 : true;
        const bool ok1 = mk ? ((mr[u][e / 2] >> (16 * (e % 2) + 8)) & 0xffu) != 0 : true;
        visit((uint16_t)(r[u][e] & 0xffffu), c + 2 * e, ok0);
        visit((uint16_t)(r[u][e] >> 16), c + 2 * e + 1, ok1);
      }
    }
  }
  for (; c8 < V8; c8 += kRowThreads) {
    const u32x4 r = *(const u32x4*)(x + c8 * 8);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      visit((uint16_t)(r[e] & 0xffffu), c8 * 8 + 2 * e, mk ? mk[c8 * 8 + 2 * e] != 0 : true);
      visit((uint16_t)(r[e] >> 16), c8 * 8 + 2 * e + 1, mk ? mk[c8 * 8 + 2 * e + 1] != 0 : true);
    }
  }
  for (int c = V8 * 8 + tid; c < V; c += kRowThreads) visit(x[c], c, mk ? mk[c] != 0 : true);
  {
    const float mm = wave_max(m), ss = wave_sum(se);
    if ((tid & 63) == 0) {
      red_m[tid >> 6] = mm;
      red_s[tid >> 6] = ss;
    }
  }
  __syncthreads();
  float M = -INFINITY;
  for (int w = 0; w < kRowThreads / 64; ++w) M = fmaxf(M, red_m[w]);
  float SE = 0.f;
  for (int w = 0; w < kRowThreads / 64; ++w) SE += red_s[w];
  if (M > mref + 60.f) {
    // the sample missed the top by far: sum again against the true max
    __syncthreads();
    mref = M;
    nb = -mref * kLog2e;
    float s2 = 0.f;
    for (int c = tid; c < V; c += kRowThreads) s2 += __builtin_amdgcn_exp2f(fmaf(bf2f(x[c]), kLog2e, nb));
    s2 = wave_sum(s2);
    if ((tid & 63) == 0) red_s[tid >> 6] = s2;
    __syncthreads();
    SE = 0.f;
    for (int w = 0; w < kRowThreads / 64; ++w) SE += red_s[w];
  }
  // log sum exp(v - M) = log(sum exp(v - mref)) + (mref - M)
  const float lse = logf(SE) + (mref - M);
  const int count = sh_count;
  if (thr == 0 || count < K || count > CAP) {
    // exact fallback: reuses the candidate buffer as the 4096-bin histogram
    __syncthreads();
    row_select_exact(row, logits, ld, mask, ld_mask, parent, Wp, V, K, cand_key, cand_idx,
                     (int*)cand);
    return;
  }
  // ---- 3. exact top K of the candidates (the merge stage orders them; the
  // row's output order is free).  Candidate = (order key u << 32) | ~column,
  // unique per column: a radix select over u (two 8-bit rounds) finds the
  // K-th largest key u*; the ties at u* are ranked by column.
  const float p = parent[row];
  const int r_local = (int)(row % Wp);
  int* bins = hist;  // 256 ints
  auto select_bin = [&](int need_in, int* above_out) -> int {
    // one wave: the bin holding the need_in-th largest entry of bins[]
    if (tid < 64) {
      int above = 0;
      int b = -1;
      {
        const int lane = tid;
        int v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = bins[lane * 4 + i];
        const int t = v[0] + v[1] + v[2] + v[3];
        int suf = t;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int y = __shfl_down(suf, o, 64);
          if (lane + o < 64) suf += y;
        }
        const uint64_t reach = __ballot(suf >= need_in);
        const int L = __popcll(reach) - 1;
        int acc = 0;
        if (lane == L) {
          acc = suf - t;
          for (int i = 3; i >= 0; --i) {
            if (acc + v[i] >= need_in) {
              b = lane * 4 + i;
              break;
            }
            acc += v[i];
          }
        }
        above = __shfl(acc, L, 64);
        b = __shfl(b, L, 64);
      }
      if (tid == 0) {
        sh_hi = b;
        sh_above = above;
      }
    }
    __syncthreads();
    *above_out = sh_above;
    return sh_hi;
  };
  // round 1: high byte of u
  bins[tid] = 0;
  __syncthreads();
  for (int i = tid; i < count; i += kRowThreads) atomicAdd(&bins[(uint32_t)(cand[i] >> 40) & 255], 1);
  __syncthreads();
  int above1;
  const int b1 = select_bin(K, &above1);
  __syncthreads();
  // round 2: low byte of u inside bin b1
  bins[tid] = 0;
  __syncthreads();
  for (int i = tid; i < count; i += kRowThreads) {
    const uint32_t u = (uint32_t)(cand[i] >> 32);
    if ((int)(u >> 8) == b1) atomicAdd(&bins[u & 255], 1);
  }
  __syncthreads();
  int above2;
  const int b2 = select_bin(K - above1, &above2);
  const uint32_t ustar = ((uint32_t)b1 << 8) | (uint32_t)b2;
  const int need = K - above1 - above2;  // ties at u* to take, lowest columns first
  auto emit = [&](uint64_t e) {
    const int slot = atomicAdd(&sh_count, 1);
    const int c = (int)(0xffffffffu - (uint32_t)e);
    const float v = bf2f(x[c]);
    if (slot < K) {  // exactly K qualify; the bound only guards memory
      cand_key[row * K + slot] = ((v - M) - lse) + p;
      cand_idx[row * K + slot] = r_local * V + c;
    }
  };
  // keys above u* are taken; the ties at u* (their ~column words) are gathered
  uint32_t* ties = (uint32_t*)bins;
  if (tid == 0) {
    sh_count = 0;
    sh_thr = 0;  // number of ties
  }
  __syncthreads();
  for (int i = tid; i < count; i += kRowThreads) {
    const uint64_t e = cand[i];
    const uint32_t u = (uint32_t)(e >> 32);
    if (u > ustar) {
      emit(e);
    } else if (u == ustar) {
      const int t = atomicAdd(&sh_thr, 1);
      if (t < 256) ties[t] = (uint32_t)e;
    }
  }
  __syncthreads();
  const int nties = sh_thr;
  if (nties <= 256) {
    // rank of each tie = ties with a lower column (a larger ~column word)
    for (int t = tid; t < nties; t += kRowThreads) {
      const uint32_t me = ties[t];
      int rank_t = 0;
      for (int j = 0; j < nties; ++j) rank_t += ties[j] > me ? 1 : 0;
      if (rank_t < need) emit(((uint64_t)ustar << 32) | me);
    }
  } else {
    // many equal keys: rank every tie against the whole candidate list
    for (int i = tid; i < count; i += kRowThreads) {
      const uint64_t e = cand[i];
      if ((uint32_t)(e >> 32) != ustar) continue;
      int rank_t = 0;
      for (int j = 0; j < count; ++j) {
        const uint64_t f = cand[j];
        rank_t += ((uint32_t)(f >> 32) == ustar && (uint32_t)f > (uint32_t)e) ? 1 : 0;
      }
      if (rank_t < need) emit(e);
    }
  }
}

// ---------------------------------------------------------------------------
constexpr int kMergeThreads = 1024;
// widest level: the winners and their sort buffer (the next power of two of
// W entries, 8 bytes each) live in dynamic LDS, 128 KB at W = 16384
constexpr int kMaxW = 16384;

__device__ __forceinline__ bool before(float ka, int ia, float kb, int ib) {
  return ka > kb || (ka == kb && ia < ib);
}

// Every radix round reads the request's candidate keys again (L2-resident);
// each thread loads kMergeBatch of them before using any, so that many loads
// are in flight instead of one.
constexpr int kMergeBatch = 8;

// Run by one full wave: the bin d at which the running count of hist,
// taken from bin 255 down (DESC) or from bin 0 up, first reaches need, and
// the count before it -- as the serial scan that stops at the last bin
// without testing it.  Lane l holds the 4 bins 4l.. in scan order; returns
// true in the one lane that found d.
template <bool DESC>
__device__ __forceinline__ bool pick_bin(const int* hist, int need, int lane, int& d_out,
                                         int& acc_out) {
  int b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) b[i] = hist[DESC ? 255 - 4 * lane - i : 4 * lane + i];
  const int s = b[0] + b[1] + b[2] + b[3];
  int incl = s;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o, 64);
    if (lane >= o) incl += t;
  }
  const unsigned long long hit = __ballot(incl >= need);
  const int L = hit ? __ffsll((long long)hit) - 1 : 63;
  if (lane == L) {
    int acc = incl - s, d = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      d = DESC ? 255 - 4 * L - i : 4 * L + i;
      if (d == (DESC ? 0 : 255) || acc + b[i] >= need) break;
      acc += b[i];
    }
    d_out = d;
    acc_out = acc;
  }
  return lane == L;  // the lane that holds the result
}

// Rows of fp32 or fp16 logits (the reference upcasts any float dtype before
// its log-softmax, src/kadllm/grbeam.py:91), one workgroup per row, exact:
// the row max, the sum of exp(x - max), four 8-bit radix rounds over the
// order keys of the row's scores key = ((x - max) - lse) + parent (-inf where
// masked) for the K-th largest, then one pass that emits every key above it
// and the first ties in column order.  Each pass recomputes the keys with the
// same operations, so every pass sees the same values.
__global__ __launch_bounds__(kRowThreads) void row_select_float_kernel(
    const void* __restrict__ logits, int dtype, int64_t ld, const uint8_t* __restrict__ mask,
    int64_t ld_mask, const float* __restrict__ parent, int Wp, int V, int K,
    float* __restrict__ cand_key, int* __restrict__ cand_idx) {
  __shared__ int hist[256];
  __shared__ int scan_tmp[kRowThreads / 64];
  __shared__ float red[kRowThreads / 64];
  __shared__ uint32_t sh_prefix;
  __shared__ int sh_need, sh_emit;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const int64_t xrow = row * ld;
  const uint8_t* mk = mask ? mask + row * ld_mask : nullptr;

  float m = -INFINITY;
  for (int c = tid; c < V; c += kRowThreads) m = fmaxf(m, load_as_float(logits, xrow + c, dtype));
  m = wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  float M = -INFINITY;
  for (int w = 0; w < kRowThreads / 64; ++w) M = fmaxf(M, red[w]);
  __syncthreads();
  float se = 0.f;
  for (int c = tid; c < V; c += kRowThreads) se += expf(load_as_float(logits, xrow + c, dtype) - M);
  se = wave_sum(se);
  if (lane == 0) red[wave] = se;
  if (tid == 0) sh_emit = 0;
  __syncthreads();
  float SE = 0.f;
  for (int w = 0; w < kRowThreads / 64; ++w) SE += red[w];
  const float lse = logf(SE);
  const float p = parent[row];
  auto key_at = [&](int c) -> float {
    const bool ok = mk ? mk[c] != 0 : true;
    return ok ? ((load_as_float(logits, xrow + c, dtype) - M) - lse) + p : -INFINITY;
  };

  uint32_t prefix = 0, pmask = 0;
  int need = K;
  for (int shift = 24; shift >= 0; shift -= 8) {
    hist[tid] = 0;  // kRowThreads == 256 bins
    __syncthreads();
    for (int c = tid; c < V; c += kRowThreads) {
      const uint32_t u = order32(key_at(c));
      if ((u & pmask) == prefix) atomicAdd(&hist[(u >> shift) & 255], 1);
    }
    __syncthreads();
    if (tid < 64) {
      int d = 0, acc = 0;
      if (pick_bin<true>(hist, need, tid, d, acc)) {
        sh_prefix = prefix | ((uint32_t)d << shift);
        sh_need = need - acc;
      }
    }
    __syncthreads();
    prefix = sh_prefix;
    need = sh_need;
    pmask |= 255u << shift;
    __syncthreads();
  }
  const uint32_t kth = prefix;  // the K-th largest key; `need` of its ties are taken
  const int r_local = (int)(row % Wp);
  float* ck = cand_key + row * K;
  int* ci = cand_idx + row * K;
  int ties_taken = 0;
  for (int c0 = 0; c0 < V; c0 += kRowThreads) {
    const int c = c0 + tid;
    float key = -INFINITY;
    uint32_t u = 0;
    if (c < V) {
      key = key_at(c);
      u = order32(key);
    }
    const bool above = c < V && u > kth;
    const bool tie = c < V && u == kth;
    int tot = 0;
    const int rank = block_exclusive_scan(tie ? 1 : 0, scan_tmp, &tot);
    if (above || (tie && ties_taken + rank < need)) {
      const int slot = atomicAdd(&sh_emit, 1);
      if (slot < K) {  // exactly K entries qualify; the bound only guards memory
        ck[slot] = key;
        ci[slot] = r_local * V + c;
      }
    }
    ties_taken += tot;
  }
}

// hist[bin] += 1 for the active lanes.  The merge's keys are cumulative
// log-probabilities of one request, so its first radix rounds put nearly
// every key in one or two bins, where one atomic per lane serialises on a
// single LDS address: the lanes of the (up to) two most common bins of the
// wave instruction add their count with one atomic each, the rest one by one.
__device__ __forceinline__ void hist_add_grouped(int* hist, bool active, int bin) {
  const int lane = threadIdx.x & 63;
  uint64_t pending = __ballot(active);
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    if (pending == 0) break;
    const int leader = __ffsll((unsigned long long)pending) - 1;
    const int lb = __shfl(bin, leader, 64);
    const uint64_t same = __ballot(active && bin == lb) & pending;
    if (lane == leader) atomicAdd(&hist[lb], (int)__popcll(same));
    pending &= ~same;
  }
  if ((pending >> lane) & 1ull) atomicAdd(&hist[bin], 1);
}

__global__ __launch_bounds__(kMergeThreads) void merge_select_kernel(
    const float* __restrict__ cand_key, const int* __restrict__ cand_idx, int ncand, int W,
    int V, float* __restrict__ scores, int64_t* __restrict__ parents,
    int64_t* __restrict__ tokens, uint8_t* __restrict__ valid, int cap) {
  __shared__ int hist[256];
  __shared__ uint32_t sh_prefix;
  __shared__ int sh_need, sh_count, sh_ties;
  // cap = the next power of two >= W keys, then as many indices
  extern __shared__ __attribute__((aligned(16))) float merge_lds[];
  float* sk = merge_lds;
  int* si = (int*)(merge_lds + cap);
  const int tid = threadIdx.x;
  const int b = blockIdx.x;
  const float* keys = cand_key + (int64_t)b * ncand;
  const int* idxs = cand_idx + (int64_t)b * ncand;
  // f(order key, candidate index) over this thread's candidates
  auto for_each = [&](auto&& f) {
    int i0 = tid;
    for (; i0 + (kMergeBatch - 1) * kMergeThreads < ncand; i0 += kMergeBatch * kMergeThreads) {
      float kv[kMergeBatch];
#pragma unroll
      for (int q = 0; q < kMergeBatch; ++q) kv[q] = keys[i0 + q * kMergeThreads];
#pragma unroll
      for (int q = 0; q < kMergeBatch; ++q) f(order32(kv[q]), i0 + q * kMergeThreads);
    }
    for (int i = i0; i < ncand; i += kMergeThreads) f(order32(keys[i]), i);
  };

  // radix select of the W-th largest key (order32 space), 4 x 8 bits
  uint32_t prefix = 0, pmask = 0;
  int need = W;  // rank (1-based) of the target within the current prefix class
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256; i += kMergeThreads) hist[i] = 0;
    __syncthreads();
    for_each([&](uint32_t u, int) {
      hist_add_grouped(hist, (u & pmask) == prefix, (int)((u >> shift) & 255));
    });
    __syncthreads();
    if (tid < 64) {
      int d = 0, acc = 0;
      if (pick_bin<true>(hist, need, tid, d, acc)) {
        sh_prefix = prefix | ((uint32_t)d << shift);
        sh_need = need - acc;
        sh_ties = hist[d];  // after the last round: the candidates equal to the key
      }
    }
    __syncthreads();
    prefix = sh_prefix;
    need = sh_need;
    pmask |= 255u << shift;
    __syncthreads();
  }
  const uint32_t kth = prefix;  // order key of the W-th largest
  // `need` ties at kth are taken, smallest flat index first: radix select on
  // index, unless every tie is taken
  uint32_t iprefix = 0xffffffffu, imask = 0;
  int ineed = need;
  const bool all_ties = need == sh_ties;
  if (!all_ties) iprefix = 0;
  for (int shift = 24; shift >= 0 && !all_ties; shift -= 8) {
    for (int i = tid; i < 256; i += kMergeThreads) hist[i] = 0;
    __syncthreads();
    for_each([&](uint32_t k, int i) {
      if (k != kth) return;
      const uint32_t u = (uint32_t)idxs[i];
      if ((u & imask) == iprefix) atomicAdd(&hist[(u >> shift) & 255], 1);
    });
    __syncthreads();
    if (tid < 64) {
      int d = 0, acc = 0;
      if (pick_bin<false>(hist, ineed, tid, d, acc)) {
        sh_prefix = iprefix | ((uint32_t)d << shift);
        sh_need = ineed - acc;
      }
    }
    __syncthreads();
    iprefix = sh_prefix;
    ineed = sh_need;
    imask |= 255u << shift;
    __syncthreads();
  }
  const uint32_t idx_cut = iprefix;  // largest tied index taken

  // gather the W winners
  if (tid == 0) sh_count = 0;
  __syncthreads();
  for_each([&](uint32_t u, int i) {
    const bool take = u > kth || (u == kth && (uint32_t)idxs[i] <= idx_cut);
    if (take) {
      const int slot = atomicAdd(&sh_count, 1);
      if (slot < cap) {
        sk[slot] = keys[i];
        si[slot] = idxs[i];
      }
    }
  });
  __syncthreads();
  // pad to a power of two and bitonic-sort by (key desc, idx asc)
  int P = 1;
  while (P < W) P <<= 1;
  for (int i = W + tid; i < P; i += kMergeThreads) {
    sk[i] = -INFINITY;
    si[i] = 0x7fffffff;
  }
  __syncthreads();
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = tid; i < P; i += kMergeThreads) {
        const int j = i ^ stride;
        if (j > i) {
          const bool dir = (i & size) == 0;  // ascending in "before" order
          const bool sw = dir ? before(sk[j], si[j], sk[i], si[i])
                              : before(sk[i], si[i], sk[j], si[j]);
          if (sw) {
            const float tk = sk[i];
            sk[i] = sk[j];
            sk[j] = tk;
            const int ti = si[i];
            si[i] = si[j];
            si[j] = ti;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int i = tid; i < W; i += kMergeThreads) {
    const float key = sk[i];
    const int id = si[i];
    scores[(int64_t)b * W + i] = key;
    parents[(int64_t)b * W + i] = id / V;
    tokens[(int64_t)b * W + i] = id % V;
    valid[(int64_t)b * W + i] = (key == key) && (key != INFINITY) && (key != -INFINITY);
  }
}

// ---------------------------------------------------------------------------
// Wide levels (W > kMaxW): the same selection as merge_select_kernel -- the
// W-th largest order key by four 8-bit radix rounds, the ties at it taken
// lowest flat index first by up to four rounds over the indices -- but each
// round's histogram is built by many workgroups per request (global atomics
// into a per-request 256-bin histogram), and the winners are sorted in
// global memory.  Winners are 64-bit words (~order key << 32 | index), so an
// ascending sort orders them by (key desc, index asc); P = the next power of
// two >= W words per request, the tail padded with all-ones words.
//
// Workspace: [B][P] u64 sort words, then [B][256] int histograms, then
// [B][kWideState] int per-request selection state.
constexpr int kWideState = 8;
enum { WS_PREFIX, WS_PMASK, WS_NEED, WS_TIES, WS_IPREFIX, WS_IMASK, WS_INEED, WS_COUNT };
constexpr int kWideThreads = 256;
constexpr int kWideItems = 16;        // candidates per thread per histogram block
constexpr int kSortLocal = 8192;      // sort words per workgroup in LDS (64 KB)
constexpr int kSortThreads = 1024;

__global__ __launch_bounds__(kWideThreads) void wide_init_kernel(uint64_t* __restrict__ words,
                                                                 int* __restrict__ hist,
                                                                 int* __restrict__ state, int B,
                                                                 int W, int P) {
  const int b = blockIdx.y;
  for (int i = W + blockIdx.x * kWideThreads + threadIdx.x; i < P; i += gridDim.x * kWideThreads)
    words[(int64_t)b * P + i] = ~0ull;
  if (blockIdx.x == 0) {
    hist[b * 256 + threadIdx.x] = 0;
    if (threadIdx.x < kWideState) {
      int v = 0;
      if (threadIdx.x == WS_NEED || threadIdx.x == WS_INEED) v = W;
      state[b * kWideState + threadIdx.x] = v;
    }
  }
}

// one histogram round over a block of kWideThreads * kWideItems candidates of
// request blockIdx.y: IDX false: bins of (key >> shift) among the keys
// matching the prefix so far; IDX true: bins of (index >> shift) among the
// keys equal to the W-th key whose indices match the index prefix so far.
template <bool IDX>
__global__ __launch_bounds__(kWideThreads) void wide_hist_kernel(
    const float* __restrict__ cand_key, const int* __restrict__ cand_idx, int ncand,
    int* __restrict__ hist, const int* __restrict__ state, int shift) {
  __shared__ int h[256];
  const int b = blockIdx.y;
  const int* st = state + b * kWideState;
  const uint32_t prefix = (uint32_t)st[WS_PREFIX], pmask = (uint32_t)st[WS_PMASK];
  if (IDX && st[WS_NEED] == st[WS_TIES]) return;  // every tie is taken: no index rounds
  const uint32_t iprefix = (uint32_t)st[WS_IPREFIX], imask = (uint32_t)st[WS_IMASK];
  h[threadIdx.x] = 0;
  __syncthreads();
  const float* keys = cand_key + (int64_t)b * ncand;
  const int* idxs = cand_idx + (int64_t)b * ncand;
  const int64_t i0 = (int64_t)blockIdx.x * kWideThreads * kWideItems + threadIdx.x;
  float kv[kWideItems];
#pragma unroll
  for (int q = 0; q < kWideItems; ++q) {
    const int64_t i = i0 + q * kWideThreads;
    kv[q] = i < ncand ? keys[i] : 0.f;
  }
#pragma unroll
  for (int q = 0; q < kWideItems; ++q) {
    const int64_t i = i0 + q * kWideThreads;
    const uint32_t u = order32(kv[q]);
    if (!IDX) {
      hist_add_grouped(h, i < ncand && (u & pmask) == prefix, (int)((u >> shift) & 255));
    } else if (i < ncand && u == prefix) {
      const uint32_t x = (uint32_t)idxs[i];
      if ((x & imask) == iprefix) atomicAdd(&h[(x >> shift) & 255], 1);
    }
  }
  __syncthreads();
  const int c = h[threadIdx.x];
  if (c) atomicAdd(&hist[b * 256 + threadIdx.x], c);
}

// one wave per request: the bin of this round (as in merge_select_kernel),
// the state update, and the histogram cleared for the next round
template <bool IDX>
__global__ __launch_bounds__(64) void wide_pick_kernel(int* __restrict__ hist,
                                                       int* __restrict__ state, int shift) {
  const int b = blockIdx.x, lane = threadIdx.x;
  int* st = state + b * kWideState;
  int* hb = hist + b * 256;
  if (IDX && st[WS_NEED] == st[WS_TIES]) return;
  int d = 0, acc = 0;
  const int need = IDX ? st[WS_INEED] : st[WS_NEED];
  const bool found = IDX ? pick_bin<false>(hb, need, lane, d, acc)
                         : pick_bin<true>(hb, need, lane, d, acc);
  const int ties = found ? hb[d] : 0;
  __syncthreads();  // every lane has read the histogram
#pragma unroll
  for (int i = 0; i < 4; ++i) hb[lane * 4 + i] = 0;
  if (found) {
    if (!IDX) {
      st[WS_PREFIX] = (int)((uint32_t)st[WS_PREFIX] | ((uint32_t)d << shift));
      st[WS_PMASK] = (int)((uint32_t)st[WS_PMASK] | (255u << shift));
      st[WS_NEED] = need - acc;
      st[WS_TIES] = ties;  // after the last round: the candidates equal to the key
      st[WS_INEED] = need - acc;  // the index rounds start from the ties still needed
    } else {
      st[WS_IPREFIX] = (int)((uint32_t)st[WS_IPREFIX] | ((uint32_t)d << shift));
      st[WS_IMASK] = (int)((uint32_t)st[WS_IMASK] | (255u << shift));
      st[WS_INEED] = need - acc;
    }
  }
}

// the W winners of each request as sort words, one slot each (wave-aggregated
// slot counter); words [W, P) were padded by wide_init_kernel
__global__ __launch_bounds__(kWideThreads) void wide_gather_kernel(
    const float* __restrict__ cand_key, const int* __restrict__ cand_idx, int ncand,
    int* __restrict__ state, uint64_t* __restrict__ words, int W, int P) {
  const int b = blockIdx.y;
  int* st = state + b * kWideState;
  const uint32_t kth = (uint32_t)st[WS_PREFIX];
  const bool all_ties = st[WS_NEED] == st[WS_TIES];
  const uint32_t idx_cut = all_ties ? 0xffffffffu : (uint32_t)st[WS_IPREFIX];
  const float* keys = cand_key + (int64_t)b * ncand;
  const int* idxs = cand_idx + (int64_t)b * ncand;
  const int lane = threadIdx.x & 63;
  const int64_t i0 = (int64_t)blockIdx.x * kWideThreads * kWideItems + threadIdx.x;
#pragma unroll 4
  for (int q = 0; q < kWideItems; ++q) {
    const int64_t i = i0 + q * kWideThreads;
    uint32_t u = 0, x = 0;
    bool take = false;
    if (i < ncand) {
      u = order32(keys[i]);
      if (u >= kth) {
        x = (uint32_t)idxs[i];
        take = u > kth || x <= idx_cut;
      }
    }
    const uint64_t m = __ballot(take);
    if (!m) continue;
    const int leader = __ffsll((unsigned long long)m) - 1;
    int base = 0;
    if (lane == leader) base = atomicAdd(&st[WS_COUNT], (int)__popcll(m));
    base = __shfl(base, leader, 64);
    if (take) {
      const int slot = base + (int)__popcll(m & ((1ull << lane) - 1));
      if (slot < W) words[(int64_t)b * P + slot] = ((uint64_t)(~u) << 32) | x;
    }
  }
}

// bitonic stages on LDS chunks of `chunk` words: sizes size_lo..size_hi, for
// each the strides below min(size, chunk); a pair's direction follows its
// position inside the request's P words (ascending where (pos & size) == 0)
__global__ __launch_bounds__(kSortThreads) void bitonic_local_kernel(uint64_t* __restrict__ words,
                                                                     int P, int chunk,
                                                                     int size_lo, int size_hi) {
  __shared__ uint64_t t[kSortLocal];
  const int64_t base = (int64_t)blockIdx.x * chunk;
  const int pos0 = (int)(base & (P - 1));
  for (int i = threadIdx.x; i < chunk; i += kSortThreads) t[i] = words[base + i];
  __syncthreads();
  for (int size = size_lo; size <= size_hi; size <<= 1) {
    for (int stride = min(size, chunk) >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < chunk / 2; i += kSortThreads) {
        const int lo = ((i & ~(stride - 1)) << 1) | (i & (stride - 1));
        const int hi = lo | stride;
        const bool asc = ((pos0 + lo) & size) == 0;
        const uint64_t a = t[lo], c = t[hi];
        if ((a > c) == asc) {
          t[lo] = c;
          t[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < chunk; i += kSortThreads) words[base + i] = t[i];
}

// one bitonic stage (size, stride >= the LDS chunk) over all requests' words
__global__ __launch_bounds__(256) void bitonic_global_kernel(uint64_t* __restrict__ words, int P,
                                                             int size, int stride,
                                                             int64_t npairs) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= npairs) return;
  const int64_t lo = ((i & ~(int64_t)(stride - 1)) << 1) | (i & (stride - 1));
  const int64_t hi = lo | stride;
  const bool asc = ((lo & (P - 1)) & size) == 0;
  const uint64_t a = words[lo], c = words[hi];
  if ((a > c) == asc) {
    words[lo] = c;
    words[hi] = a;
  }
}

__global__ __launch_bounds__(256) void wide_emit_kernel(const uint64_t* __restrict__ words, int P,
                                                        int B, int W, int V,
                                                        float* __restrict__ scores,
                                                        int64_t* __restrict__ parents,
                                                        int64_t* __restrict__ tokens,
                                                        uint8_t* __restrict__ valid) {
  const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (n >= (int64_t)B * W) return;
  const int64_t b = n / W, j = n % W;
  const uint64_t w = words[b * P + j];
  const uint32_t u = ~(uint32_t)(w >> 32);
  // inverse of order32
  const float key = __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
  const int id = (int)(uint32_t)w;
  scores[n] = key;
  parents[n] = id / V;
  tokens[n] = id % V;
  valid[n] = (key == key) && (key != INFINITY) && (key != -INFINITY);
}

__global__ __launch_bounds__(256) void history_kernel(const int64_t* __restrict__ hist, int Wp,
                                                      int step, const int64_t* __restrict__ parents,
                                                      const int64_t* __restrict__ tokens,
                                                      int64_t* __restrict__ out, int B, int W) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)B * W * (step + 1)) return;
  const int j = (int)(i % (step + 1));
  const int64_t bw = i / (step + 1);
  const int b = (int)(bw / W);
  if (j == step) {
    out[i] = tokens[bw];
  } else {
    int64_t p = parents[bw];
    p = p < 0 ? 0 : (p >= Wp ? Wp - 1 : p);
    out[i] = hist[((int64_t)b * Wp + p) * step + j];
  }
}

// dst rows (n, t), t < rows_copy, of beam n = b * W + w  <-  src rows
// (b * Wp + parents[n], t): a beam's cached per-token rows follow its parent.
// 16 bytes per thread; rows are row_bytes long (a multiple of 16).
// IDX: the index type of the flat chunk count (32-bit divisions whenever
// it fits, the 64-bit ones costing several times the copy's own work)
template <typename IDX>
__global__ __launch_bounds__(256) void gather_beam_rows_kernel(
    const uint8_t* __restrict__ src, int64_t ld_src, int src_rows_per_beam,
    uint8_t* __restrict__ dst, int64_t ld_dst, int dst_rows_per_beam, int rows_copy,
    const int64_t* __restrict__ parents, int W, int Wp, int64_t nbeams, int chunks_per_row) {
  const IDX idx = (IDX)blockIdx.x * 256 + threadIdx.x;
  const IDX per_beam = (IDX)rows_copy * chunks_per_row;
  if (idx >= (IDX)nbeams * per_beam) return;
  const IDX n = idx / per_beam;
  const int rest = (int)(idx - n * per_beam);
  const int t = rest / chunks_per_row, c = rest - t * chunks_per_row;
  const int64_t b = n / (IDX)W;
  const int64_t pn = parents[n];
  const int64_t sn = b * Wp + (pn < 0 ? 0 : (pn >= Wp ? Wp - 1 : pn));  // stay in bounds
  const u32x4 v = *(const u32x4*)(src + (sn * src_rows_per_beam + t) * ld_src + c * 16);
  // row offsets in 64 bits: only the flat chunk count is bounded by IDX
  *(u32x4*)(dst + ((int64_t)n * dst_rows_per_beam + t) * ld_dst + c * 16) = v;
}

int launch_row_select(const void* logits, int logits_dtype, int64_t ld, const void* mask,
                      int64_t ld_mask, const float* parent_scores, int rows, int Wp, int V,
                      int K, float* cand_key, int* cand_idx, hipStream_t s) {
  if (logits_dtype != KAD_DTYPE_BF16) {
    hipLaunchKernelGGL(row_select_float_kernel, dim3(rows), dim3(kRowThreads), 0, s, logits,
                       logits_dtype, ld, (const uint8_t*)mask, ld_mask, parent_scores, Wp, V, K,
                       cand_key, cand_idx);
    return kad_launch_status("row_select_float_kernel");
  }
  // sample ~kTargetLines lines; rank chosen so that rank * line_stride >= 2K + 256
  const int nlines = (V + kLine - 1) / kLine;
  const int line_stride = nlines > kTargetLines ? nlines / kTargetLines : 1;
  const int rank = (int)kad_cdiv(2 * (int64_t)K + 256, line_stride);
#define KAD_ROW_SELECT(CAP, MASKED)                                                        \
  hipLaunchKernelGGL((row_select_kernel<CAP, MASKED>), dim3(rows), dim3(kRowThreads), 0, s,  \
                     (const bf16_t*)logits, ld, (const uint8_t*)mask, ld_mask, parent_scores,  \
                     Wp, V, K, cand_key, cand_idx, line_stride, rank)
  const bool small = 2 * (int64_t)K + 256 <= kCandCapSmall / 2;
  if (mask) {
    if (small) KAD_ROW_SELECT(kCandCapSmall, true);
    else KAD_ROW_SELECT(kCandCapLarge, true);
  } else {
    if (small) KAD_ROW_SELECT(kCandCapSmall, false);
    else KAD_ROW_SELECT(kCandCapLarge, false);
  }
#undef KAD_ROW_SELECT
  return kad_launch_status("row_select_kernel");
}

int launch_merge(const float* cand_key, const int* cand_idx, int B, int ncand, int W, int V,
                 float* scores, int64_t* parents, int64_t* tokens, void* valid, hipStream_t s) {
  int cap = 1;
  while (cap < W) cap <<= 1;
  const size_t lds = (size_t)cap * 8;
  if (lds > 64 * 1024) {
    // beyond the default 64 KB of dynamic LDS per workgroup (the CU has 160 KB)
    const hipError_t e = hipFuncSetAttribute((const void*)merge_select_kernel,
                                             hipFuncAttributeMaxDynamicSharedMemorySize,
                                             (int)lds);
    if (e != hipSuccess) {
      kad_set_error("merge_select_kernel: cannot raise its LDS limit to %zu bytes: %s", lds,
                    hipGetErrorString(e));
      return KAD_ERR_HIP;
    }
  }
  hipLaunchKernelGGL(merge_select_kernel, dim3(B), dim3(kMergeThreads), lds, s, cand_key, cand_idx,
                     ncand, W, V, scores, parents, tokens, (uint8_t*)valid, cap);
  return kad_launch_status("merge_select_kernel");
}

int64_t wide_words(int W) {
  int64_t P = 1;
  while (P < W) P <<= 1;
  return P;
}

int64_t wide_ws_bytes(int B, int W) {
  return (int64_t)B * wide_words(W) * 8 + (int64_t)B * 256 * 4 + (int64_t)B * kWideState * 4;
}

int launch_merge_wide(const float* cand_key, const int* cand_idx, int B, int ncand, int W, int V,
                      float* scores, int64_t* parents, int64_t* tokens, void* valid, void* ws,
                      hipStream_t s) {
  const int64_t P = wide_words(W);
  uint64_t* words = (uint64_t*)ws;
  int* hist = (int*)(words + (int64_t)B * P);
  int* state = hist + (int64_t)B * 256;
  const int64_t init_blocks = std::min<int64_t>(std::max<int64_t>((P - W + kWideThreads - 1) /
                                                                      kWideThreads, 1), 4096);
  hipLaunchKernelGGL(wide_init_kernel, dim3((unsigned)init_blocks, (unsigned)B), dim3(kWideThreads),
                     0, s, words, hist, state, B, W, (int)P);
  if (const int rc = kad_launch_status("wide_init_kernel")) return rc;
  const int64_t per_block = (int64_t)kWideThreads * kWideItems;
  const dim3 grid((unsigned)((ncand + per_block - 1) / per_block), (unsigned)B);
  for (int shift = 24; shift >= 0; shift -= 8) {
    hipLaunchKernelGGL((wide_hist_kernel<false>), grid, dim3(kWideThreads), 0, s, cand_key,
                       cand_idx, ncand, hist, state, shift);
    hipLaunchKernelGGL((wide_pick_kernel<false>), dim3(B), dim3(64), 0, s, hist, state, shift);
  }
  for (int shift = 24; shift >= 0; shift -= 8) {
    hipLaunchKernelGGL((wide_hist_kernel<true>), grid, dim3(kWideThreads), 0, s, cand_key,
                       cand_idx, ncand, hist, state, shift);
    hipLaunchKernelGGL((wide_pick_kernel<true>), dim3(B), dim3(64), 0, s, hist, state, shift);
  }
  if (const int rc = kad_launch_status("wide_hist_kernel")) return rc;
  hipLaunchKernelGGL(wide_gather_kernel, grid, dim3(kWideThreads), 0, s, cand_key, cand_idx,
                     ncand, state, words, W, (int)P);
  if (const int rc = kad_launch_status("wide_gather_kernel")) return rc;
  const int chunk = (int)std::min<int64_t>(P, kSortLocal);
  const int64_t total = (int64_t)B * P;
  hipLaunchKernelGGL(bitonic_local_kernel, dim3((unsigned)(total / chunk)), dim3(kSortThreads), 0,
                     s, words, (int)P, chunk, 2, chunk);
  for (int64_t size = 2 * (int64_t)chunk; size <= P; size <<= 1) {
    for (int64_t stride = size / 2; stride >= chunk; stride >>= 1)
      hipLaunchKernelGGL(bitonic_global_kernel, dim3((unsigned)((total / 2 + 255) / 256)),
                         dim3(256), 0, s, words, (int)P, (int)size, (int)stride, total / 2);
    hipLaunchKernelGGL(bitonic_local_kernel, dim3((unsigned)(total / chunk)), dim3(kSortThreads),
                       0, s, words, (int)P, chunk, (int)size, (int)size);
  }
  if (const int rc = kad_launch_status("bitonic_kernels")) return rc;
  hipLaunchKernelGGL(wide_emit_kernel, dim3((unsigned)(((int64_t)B * W + 255) / 256)), dim3(256),
                     0, s, words, (int)P, B, W, V, scores, parents, tokens, (uint8_t*)valid);
  return kad_launch_status("wide_emit_kernel");
}

int check_logits_dtype(int dtype) {
  KAD_REQUIRE(dtype == KAD_DTYPE_BF16 || dtype == KAD_DTYPE_F16 || dtype == KAD_DTYPE_F32,
              "unknown logits dtype code %d", dtype);
  return KAD_OK;
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free selection (kad_beam_select_noalloc): the
// per-row candidates (keys, then flat indices) live in this file-scope device
// array, one copy per GPU for the life of the process.  Host code never uses
// the array's name as an address: scratch_address() asks the runtime for the
// current device's copy once and keeps it.
constexpr int64_t kSelectScratchBytes = 32ll << 20;

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

static_assert(sizeof(scratch) == kSelectScratchBytes, "scratch size");

int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    kad_set_error("hipGetDevice failed: %s", hipGetErrorString(e));
    return KAD_ERR_HIP;
  }
  if (dev < 0 || dev >= kMaxDevices) KAD_UNSUPPORTED("device ordinal %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      kad_set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                    hipGetErrorString(e));
      return KAD_ERR_HIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KAD_OK;
}

}  // namespace

extern "C" int kad_beam_row_select(const void* logits, int logits_dtype, int64_t ld,
                                   const void* mask, int64_t ld_mask, const float* parent_scores,
                                   int rows, int Wp, int V, int K, float* cand_key, int* cand_idx,
                                   kad_stream_t stream) {
  KAD_REQUIRE(logits && parent_scores && cand_key && cand_idx, "null pointer argument");
  KAD_REQUIRE(rows > 0 && Wp > 0 && rows % Wp == 0 && V > 0 && ld >= V, "bad dimensions");
  KAD_REQUIRE(K >= 1 && K <= V, "K must be in [1, V]");
  KAD_REQUIRE((int64_t)Wp * V < 0x7fffffff, "Wp * V must fit in int32 flat indices");
  if (const int rc = check_logits_dtype(logits_dtype)) return rc;
  return launch_row_select(logits, logits_dtype, ld, mask, ld_mask, parent_scores, rows, Wp, V, K,
                           cand_key, cand_idx, (hipStream_t)stream);
}

extern "C" int kad_beam_merge_select(const float* cand_key, const int* cand_idx, int B, int ncand,
                                     int W, int V, float* scores, int64_t* parents,
                                     int64_t* tokens, void* valid, kad_stream_t stream) {
  KAD_REQUIRE(cand_key && cand_idx && scores && parents && tokens && valid, "null pointer argument");
  KAD_REQUIRE(B > 0 && W > 0 && ncand >= W && V > 0, "bad dimensions (need ncand >= W)");
  if (W > kMaxW)
    KAD_UNSUPPORTED("beam width %d exceeds %d; kad_beam_merge_select_wide sorts wider levels", W,
                    kMaxW);
  return launch_merge(cand_key, cand_idx, B, ncand, W, V, scores, parents, tokens, valid,
                      (hipStream_t)stream);
}

extern "C" int kad_beam_merge_select_wide_workspace_bytes(int B, int W, int64_t* bytes) {
  KAD_REQUIRE(bytes, "null pointer argument");
  KAD_REQUIRE(B > 0 && W > 0, "bad dimensions");
  *bytes = wide_ws_bytes(B, W);
  return KAD_OK;
}

extern "C" int kad_beam_merge_select_wide(const float* cand_key, const int* cand_idx, int B,
                                          int ncand, int W, int V, float* scores,
                                          int64_t* parents, int64_t* tokens, void* valid,
                                          void* workspace, int64_t workspace_bytes,
                                          kad_stream_t stream) {
  KAD_REQUIRE(cand_key && cand_idx && scores && parents && tokens && valid && workspace,
              "null pointer argument");
  KAD_REQUIRE(B > 0 && W > 0 && ncand >= W && V > 0, "bad dimensions (need ncand >= W)");
  KAD_REQUIRE(B <= 65535, "at most 65535 requests per call");
  KAD_REQUIRE(wide_words(W) <= (1ll << 30), "beam width %d too large", W);
  const int64_t need = wide_ws_bytes(B, W);
  KAD_REQUIRE(workspace_bytes >= need, "workspace of %lld bytes is smaller than %lld",
              (long long)workspace_bytes, (long long)need);
  KAD_REQUIRE(((uintptr_t)workspace % 16) == 0, "workspace must be 16-byte aligned");
  return launch_merge_wide(cand_key, cand_idx, B, ncand, W, V, scores, parents, tokens, valid,
                           workspace, (hipStream_t)stream);
}

extern "C" int kad_beam_select_noalloc(const void* logits, int logits_dtype, int64_t ld,
                                       const void* mask, int64_t ld_mask,
                                       const float* parent_scores, int B, int Wp, int V, int W,
                                       float* scores, int64_t* parents, int64_t* tokens,
                                       void* valid, kad_stream_t stream) {
  KAD_REQUIRE(logits && parent_scores && scores && parents && tokens && valid,
              "null pointer argument");
  KAD_REQUIRE(B > 0 && Wp > 0 && V > 0 && W > 0 && ld >= V, "bad dimensions");
  KAD_REQUIRE((int64_t)Wp * V < 0x7fffffff, "Wp * V must fit in int32 flat indices");
  KAD_REQUIRE((int64_t)W <= (int64_t)Wp * V, "beam width exceeds the number of candidate slots");
  if (W > kMaxW) KAD_UNSUPPORTED("beam width %d exceeds %d", W, kMaxW);
  if (const int rc = check_logits_dtype(logits_dtype)) return rc;
  const int K = W < V ? W : V;
  const int64_t rows = (int64_t)B * Wp;
  const int64_t ncand = rows * K;
  const int64_t key_bytes = (ncand * 4 + 255) / 256 * 256;
  if (key_bytes + ncand * 4 > kSelectScratchBytes)
    KAD_UNSUPPORTED("allocation-free selection holds at most %lld candidates "
                    "(B * Wp * min(W, V) = %lld); use kad_beam_row_select + "
                    "kad_beam_merge_select with caller workspace",
                    (long long)(kSelectScratchBytes / 8), (long long)ncand);
  KAD_REQUIRE(rows < 0x7fffffffLL, "too many beam rows");
  void* base = nullptr;
  if (const int rc = scratch_address(&base)) return rc;
  float* cand_key = (float*)base;
  int* cand_idx = (int*)((uint8_t*)base + key_bytes);
  hipStream_t s = (hipStream_t)stream;
  // the row stage writes exactly K candidates per row, so nothing is cleared
  if (const int rc = launch_row_select(logits, logits_dtype, ld, mask, ld_mask, parent_scores,
                                       (int)rows, Wp, V, K, cand_key, cand_idx, s))
    return rc;
  return launch_merge(cand_key, cand_idx, B, Wp * K, W, V, scores, parents, tokens, valid, s);
}

extern "C" int kad_beam_history(const int64_t* history, int Wp, int step, const int64_t* parents,
                                const int64_t* tokens, int64_t* out, int B, int W,
                                kad_stream_t stream) {
  KAD_REQUIRE(parents && tokens && out && (history || step == 0), "null pointer argument");
  KAD_REQUIRE(B > 0 && W > 0 && Wp > 0 && step >= 0, "bad dimensions");
  const int64_t total = (int64_t)B * W * (step + 1);
  hipLaunchKernelGGL(history_kernel, dim3((unsigned)kad_cdiv(total, 256)), dim3(256), 0,
                     (hipStream_t)stream, history, Wp, step, parents, tokens, out, B, W);
  return kad_launch_status("history_kernel");
}

extern "C" int kad_gather_beam_rows(const void* src, int64_t ld_src_bytes, int src_rows_per_beam,
                                    void* dst, int64_t ld_dst_bytes, int dst_rows_per_beam,
                                    int rows_copy, int64_t row_bytes, const int64_t* parents,
                                    int B, int W, int Wp, kad_stream_t stream) {
  KAD_REQUIRE(src && dst && parents, "null pointer argument");
  KAD_REQUIRE(B > 0 && W > 0 && Wp > 0 && rows_copy >= 0 && rows_copy <= src_rows_per_beam &&
                  rows_copy <= dst_rows_per_beam && row_bytes > 0,
              "bad dimensions");
  KAD_REQUIRE(row_bytes % 16 == 0 && ld_src_bytes % 16 == 0 && ld_dst_bytes % 16 == 0 &&
                  ((uintptr_t)src % 16) == 0 && ((uintptr_t)dst % 16) == 0,
              "rows must be 16-byte aligned multiples of 16 bytes");
  KAD_REQUIRE(ld_src_bytes >= row_bytes && ld_dst_bytes >= row_bytes, "row strides too small");
  if (rows_copy == 0) return KAD_OK;
  const int64_t nbeams = (int64_t)B * W;
  const int cpr = (int)(row_bytes / 16);
  const int64_t total = nbeams * rows_copy * cpr;
  if (total + 256 < ((int64_t)1 << 31))
    hipLaunchKernelGGL(gather_beam_rows_kernel<uint32_t>, dim3((unsigned)kad_cdiv(total, 256)),
                       dim3(256), 0, (hipStream_t)stream, (const uint8_t*)src, ld_src_bytes,
                       src_rows_per_beam, (uint8_t*)dst, ld_dst_bytes, dst_rows_per_beam,
                       rows_copy, parents, W, Wp, nbeams, cpr);
  else
    hipLaunchKernelGGL(gather_beam_rows_kernel<int64_t>, dim3((unsigned)kad_cdiv(total, 256)),
                       dim3(256), 0, (hipStream_t)stream, (const uint8_t*)src, ld_src_bytes,
                       src_rows_per_beam, (uint8_t*)dst, ld_dst_bytes, dst_rows_per_beam,
                       rows_copy, parents, W, Wp, nbeams, cpr);
  return kad_launch_status("gather_beam_rows_kernel");
}
