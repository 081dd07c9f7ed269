// Gated GQA attention on gfx950 MFMA: prefix-shared beam decode and causal prefill.
//
// Decode replaces src/kadllm/ops.py:252-341 (prefix_attention, torch path)
// and src/kadllm/kernels/flash_attention.py:11-66 (FlashAttention glue), plus
// the sigmoid output gate of src/kadllm/adapters/qwen3_5.py:199-201.
// Prefill replaces the causal SDPA attention of the transformers forward the
// reference prefill runs (qwen3_5.py:111).
//
// Work unit: one (request b, KV head kh) and a block of query rows (256, or
// 128 for head dim 256), 4 waves of 64 rows.  Decode rows are ordered (beam,
// q-head in the group, suffix token); every row of a request/KV-head shares
// one prefix K/V, so each 32-key K and V tile is staged in LDS once per
// workgroup and consumed by all its rows.
//
// Scores are formed transposed, S^T = K Q^T (v_mfma_f32_32x32x16_bf16, A = K
// tile, B = the wave's query rows held in registers for the whole kernel),
// so each lane owns one query column.  P is rounded to bf16 and
// O^T += V^T P^T accumulates in fp32 registers.  The causal per-beam suffix
// (up to 8 keys: a 4-key fold, and an 8-key one for longer suffixes) is
// folded in first, with fp32 dot products, as the initial softmax state; the
// result equals the reference's LSE merge of the prefix and suffix
// partitions (ops.py:243-249).  A fully masked prefix contributes nothing, as
// in ops.py:229-240.
//
// CAUSAL (prefill) mode: rows are (position, q-head in group) of one
// sequence, keys are the same sequence's K/V and key j is visible to a row at
// position p iff j <= p; no suffix.

#include <type_traits>

#include "kad_common.h"

namespace {

constexpr int kThreads = 256;

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>)
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<N, I + 1>(f);
  }
}
// suffix keys folded per beam row (decode): 4, or 8 for longer suffixes
constexpr int kSuffixFold = 4, kSuffixFoldLong = 8, kSuffixFoldShort = 2;

struct AttnArgs {
  const bf16_t* q; int64_t sq_n, sq_t, sq_h;
  const bf16_t* pk; const bf16_t* pv; int64_t sp_b, sp_l, sp_h;   // prefix K/V (same strides)
  const bf16_t* sk; const bf16_t* sv; int64_t ssk_n, ssk_t, ssk_h, ssv_n, ssv_t, ssv_h;
  const uint8_t* mask;                                             // [B, L] or null
  const bf16_t* gate; int64_t sg_n, sg_t, sg_h;                     // or null
  bf16_t* out; int64_t so_n, so_t, so_h;
  int W, T, H, HK, L;     // T: query tokens per beam
  float scale;
  int nqblk;
  int Tk, qoff;           // suffix keys per beam; query t is suffix position t + qoff
};

// ---------------------------------------------------------------------------
// Attention with 64 query rows per wave (two 32-row MFMA column blocks), so
// every K and V fragment read from LDS feeds two MFMAs.  Work unit: one
// (request, KV head) and 256 query rows; 32-key tiles of K and V move
// HBM -> LDS by global_load_lds_dwordx4 (three stages in flight) in their
// row-major layout, XOR-swizzled per 16-byte chunk so that every fragment
// read is bank-conflict free.  Vᵀ fragments come straight from the row-major
// V tile with ds_read_b64_tr_b16 (within each 16-lane group, lane i receives
// element i % 4 of the 8-byte pieces addressed by lanes 4e + i / 4, e < 4):
// lanes address 4 keys x 4 pieces of d and each receives 4 keys of one d.
// The running max is raised lazily (only when a tile's max exceeds it by
// more than 2^8), which skips the rescale of O in almost every tile; a row's
// result does not depend on the other rows of its wave.
constexpr int kKeys2 = 32;                 // keys per tile
constexpr int kStages2 = 3;

template <int D>
struct Attn2 {
  // head dim 256: two waves share 64 query rows and split the head dim (the
  // full 256 x 64 fp32 O^T plus 64 query rows of Q would not fit one wave's
  // registers): each forms the partial scores over its half of d, the two
  // exchange them through LDS, and each accumulates its half of O.  Smaller
  // heads: one wave per 64 rows.
  static constexpr int DS = D > 128 ? 2 : 1;
  static constexpr int ROWS = 64 * 4 / DS;          // query rows per workgroup
  static constexpr int CPR = D / 8;                 // 16-byte chunks per K/V row
  static constexpr int tile = kKeys2 * D;           // elements per K (or V) tile
  static constexpr int stage = 2 * tile;
  // bytes: the K/V stages, then (head dim 256) the partial-score exchange of
  // the two waves of a query group, 32 floats per lane
  static constexpr int xoff = kStages2 * stage;     // elements
  static constexpr int lds = kStages2 * stage * 2 + (DS == 2 ? 4 * 64 * 32 * 4 : 0);
  static constexpr int LOADS = CPR / 8;             // DMA instructions per wave per K (or V) tile
  // physical chunk of logical chunk c in row r
  __device__ static __forceinline__ int swk(int r) { return D == 64 ? (r >> 1) & 7 : r & 15; }
  __device__ static __forceinline__ int swv(int r) { return D == 64 ? ((r >> 1) & 1) * 4 : (r & 3) * 4; }
};

// barrier without the full memory fence of __syncthreads (which also waits
// for the prefetch loads still in flight); LDS traffic is ordered by the
// caller's waits
__device__ __forceinline__ void tile_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

typedef __attribute__((address_space(3))) void attn_lds_t;
typedef __attribute__((address_space(1))) void attn_global_t;
typedef short v4s_t __attribute__((ext_vector_type(4)));

template <int D, bool CAUSAL, int NSUF>
__global__ __launch_bounds__(kThreads, 1) void attn2_kernel(AttnArgs a) {
  using AT = Attn2<D>;
  constexpr int KS = D / 16;   // k16 steps over the head dim
  constexpr int DS = AT::DS;   // waves sharing one group of 64 query rows
  constexpr int DT = D / 32 / DS;  // 32-row d tiles of O^T per wave
  constexpr int KSW = KS / DS;     // k16 steps of the partial scores per wave
  constexpr int ROWS = AT::ROWS;
  constexpr int CPR = AT::CPR;
  extern __shared__ __attribute__((aligned(1024))) bf16_t smem[];
  __shared__ int redo;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hi = lane >> 5, col = lane & 31;
  const int qgrp = wave / DS;            // query group of 64 rows
  const int dbase = (wave % DS) * DT;    // this wave's first d tile
  const int lid = xcd_logical_id(blockIdx.x, gridDim.x);
  // causal: the blocks of a (request, KV head) go out longest first (the
  // last query rows see the most keys), so that the short ones fill the tail
  const int qb_blk = CAUSAL ? a.nqblk - 1 - lid % a.nqblk : lid % a.nqblk;
  const int bk = lid / a.nqblk;
  const int kh = bk % a.HK, b = bk / a.HK;
  const int G = a.H / a.HK;
  const int64_t rows_total = CAUSAL ? (int64_t)a.L * G : (int64_t)a.W * G * a.T;

  // head dim 256: block 0 of a wave holds the 32 query rows whose softmax it
  // forms, block 1 its partner's (so the odd wave of a pair swaps them)
  const int swap = DS == 2 ? (wave & 1) : 0;
  // this lane's query row of block qb: token n (batch row), suffix position
  // or prompt position t, head h (recomputed where needed to save registers)
  auto row_of_q = [&](int qb, int64_t& n, int& t, int& h) {
    int64_t r = (int64_t)qb_blk * ROWS + qgrp * 64 + (qb ^ swap) * 32 + col;
    if (r >= rows_total) r = 0;
    int g;
    if (CAUSAL) {
      t = (int)(r / G);
      g = (int)(r % G);
      n = b;
    } else {
      t = (int)(r % a.T);
      const int64_t wg = r / a.T;
      g = (int)(wg % G);
      n = (int64_t)b * a.W + wg / G;
    }
    h = kh * G + g;
  };
  bf16x8 qf[2][KSW];  // this wave's half of d (head dim 256) or all of it
  int pos[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    int64_t n;
    int t, h;
    row_of_q(qb, n, t, h);
    pos[qb] = t;
    const bf16_t* qrow = a.q + n * a.sq_n + (int64_t)t * a.sq_t + (int64_t)h * a.sq_h;
#pragma unroll
    for (int s = 0; s < KSW; ++s)
      qf[qb][s] = as_bf16x8(*(const u32x4*)(qrow + (dbase * 2 + s) * 16 + hi * 8));
  }
  // partial suffix scores of the two waves of a query group: v holds n/2
  // values of block 0 then n/2 of block 1; the partner's block 1 is this
  // wave's block 0 and the other way round, so the halves are swapped
  float* xbuf = (float*)(smem + AT::xoff);
  auto exchange = [&](float* v, int n) {  // n <= 32, a multiple of 8
    if constexpr (DS == 2) {
      float* mine = xbuf + wave * 64 * 32;
      const float* other = xbuf + (wave ^ 1) * 64 * 32;
#pragma unroll
      for (int c = 0; c < n / 4; ++c)
        *(f32x4*)(mine + (c * 64 + lane) * 4) = f32x4{v[4 * c], v[4 * c + 1], v[4 * c + 2], v[4 * c + 3]};
      // LDS writes done, then the barrier; the K/V prefetch loads in flight
      // are not waited for (__syncthreads would wait for them too)
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0) only
      tile_barrier();
#pragma unroll
      for (int c = 0; c < n / 4; ++c) {
        const int cp = (c + n / 8) % (n / 4);
        const f32x4 o = *(const f32x4*)(other + (cp * 64 + lane) * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * c + e] += o[e];
      }
    }
  };
  const float sl2 = a.scale * 1.4426950408889634f;  // scores in log2 units

  // this wave's part of the raw suffix dot product j of block qb (decode)
  auto suffix_part = [&](int qb, int j) -> float {
    if (CAUSAL || j >= a.Tk) return 0.f;
    int64_t n;
    int t, h;
    row_of_q(qb, n, t, h);
    const bf16_t* krow = a.sk + n * a.ssk_n + (int64_t)j * a.ssk_t + (int64_t)kh * a.ssk_h;
    float part = 0.f;
#pragma unroll
    for (int s = 0; s < KSW; ++s) {
      const bf16x8 kb = as_bf16x8(*(const u32x4*)(krow + (dbase * 2 + s) * 16 + hi * 8));
#pragma unroll
      for (int i = 0; i < 8; ++i) part += (float)qf[qb][s][i] * (float)kb[i];
    }
    return part + __shfl_xor(part, 32, 64);
  };

  // ---- prefix key range and the DMA plan
  int kend = a.L;
  if (CAUSAL) {
    const int64_t rlast = min((int64_t)(qb_blk + 1) * ROWS, rows_total) - 1;
    kend = (int)(rlast / G) + 1;
  }
  const int ntiles = (kend + kKeys2 - 1) / kKeys2;
  const bf16_t* pkb = a.pk + (int64_t)b * a.sp_b + (int64_t)kh * a.sp_h;
  const bf16_t* pvb = a.pv + (int64_t)b * a.sp_b + (int64_t)kh * a.sp_h;
  // DMA: instruction ii = wave + 4 k of a tile covers tile chunks ii*64 + lane
  // (row = chunk / CPR, physical chunk = chunk % CPR; the lane fetches the
  // logical chunk that belongs there).  Rows of instruction k are
  // (wave + 4k) * (64 / CPR) + lane / CPR.
  const int d_row = lane / CPR, d_pc = lane % CPR;
  auto issue = [&](int tile, int stage) {
    const int k0 = tile * kKeys2;
    bf16_t* kd = smem + stage * AT::stage;
    bf16_t* vd = kd + AT::tile;
#pragma unroll
    for (int k = 0; k < AT::LOADS; ++k) {
      const int r = (wave + 4 * k) * (64 / CPR) + d_row;
      const int64_t key = min(k0 + r, a.L - 1);
      const int ioff = (wave + 4 * k) * 64 * 8;
      __builtin_amdgcn_global_load_lds(
          (attn_global_t*)(pkb + key * a.sp_l + (d_pc ^ AT::swk(r)) * 8),
          (attn_lds_t*)(kd + ioff), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(
          (attn_global_t*)(pvb + key * a.sp_l + (d_pc ^ AT::swv(r)) * 8),
          (attn_lds_t*)(vd + ioff), 16, 0, 0);
    }
  };

  // K fragment (A operand, 32 keys x 16 d): row col, logical chunk 2s + hi.
  // The swizzle only touches the low 4 bits of the chunk, so the offsets of
  // steps s and s + 8 differ by 16 chunks: 8 per-lane offsets cover all steps.
  int k_off[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const int c = 2 * s + hi;
    k_off[s] = col * D + (c < CPR ? (c ^ AT::swk(col)) * 8 : 0);
  }
  // V^T fragment pieces: lane i of group g (h = g / 2, dg = g % 2) addresses
  // key 16 ks + 8 rd + 4 h + i / 4 at d = dt*32 + dg*16 + (i % 4)*4.  The
  // swizzle depends on key % 4 = (i / 4) % 4 only, and touches the low two
  // bits of the 32-d tile index: 4 per-lane offsets cover every (ks, rd, dt).
  int v_off[4];
  {
    const int grp = lane >> 4, gi = lane & 15;
    const int v_row = 4 * (grp >> 1) + (gi >> 2);
    const int v_dq = (grp & 1) * 16 + (gi & 3) * 4;
    const int v_sw = AT::swv(v_row);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int d = dt * 32 + v_dq;
      v_off[dt] = v_row * D + ((d >> 3) < CPR ? (((d >> 3) ^ v_sw) * 8) + (d & 7) : 0);
    }
  }

  // Softmax with a fixed reference: p = 2^(s - m_ref), where m_ref is the
  // first max a row sees (its suffix, or its first key tile).  O is never
  // rescaled; a row whose later scores exceed m_ref by more than 2^64 is
  // flagged, and then the workgroup runs the whole key loop again with
  // m_ref = the row's true max (which no score exceeds).  The suffix keys'
  // scores are formed first (they set m_ref in decode) and their V rows are
  // added in the epilogue, so that O is only ever touched by MFMAs in the loop.
  float m_ref[2] = {-INFINITY, -INFINITY};
  float sc[2][NSUF];  // suffix scores (decode), key j of the beam
  if (!CAUSAL) {
    float part[2 * NSUF];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int j = 0; j < NSUF; ++j) part[qb * NSUF + j] = suffix_part(qb, j);
    exchange(part, 2 * NSUF);
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      int64_t n;
      int t, h;
      row_of_q(qb, n, t, h);
#pragma unroll
      for (int j = 0; j < NSUF; ++j) {
        sc[qb][j] = j < a.Tk && j <= t + a.qoff ? part[qb * NSUF + j] * sl2 : -INFINITY;
        m_ref[qb] = fmaxf(m_ref[qb], sc[qb][j]);
      }
    }
  } else {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int j = 0; j < NSUF; ++j) sc[qb][j] = -INFINITY;
  }
  float m_true[2] = {m_ref[0], m_ref[1]};
  float l[2];
  f32x16 O[2][DT];
  for (int pass = 0; pass < 2; ++pass) {
    bool overflow = false;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      l[qb] = 0.f;
#pragma unroll
      for (int j = 0; j < NSUF; ++j)
        if (sc[qb][j] != -INFINITY) l[qb] += exp2f(sc[qb][j] - m_ref[qb]);
#pragma unroll
      for (int i = 0; i < DT; ++i) O[qb][i] = f32x16{};
    }

    // ---- prefix keys [0, kend)
    if (ntiles > 0) issue(0, 0);
    if (ntiles > 1) issue(1, 1);
    for (int tile = 0; tile < ntiles; ++tile) {
      const int stage = tile % kStages2;
      // this tile's loads have landed (the newer tile's stay in flight)
      if (tile + 1 < ntiles)
        __builtin_amdgcn_s_waitcnt(0x0070 | ((2 * AT::LOADS) & 0xF) | (((2 * AT::LOADS) >> 4) << 14));
      else
        __builtin_amdgcn_s_waitcnt(0x0070);
      tile_barrier();
      const bf16_t* ks = smem + stage * AT::stage;
      const bf16_t* vs = ks + AT::tile;

      // S^T[key, query] for 32 keys, both query blocks; each K fragment read
      // is issued one step ahead of its two MFMAs
      f32x16 st[2] = {f32x16{}, f32x16{}};
      auto kfrag = [&](int s) {
        const int sg = dbase * 2 + s;  // d step
        return as_bf16x8(*(const u32x4*)(ks + k_off[sg & 7] + (sg >> 3) * 128));
      };
      __builtin_amdgcn_sched_barrier(0);
      bf16x8 kf[2];
      kf[0] = kfrag(0);
#pragma unroll
      for (int s = 0; s < KSW; ++s) {
        // step s: the read of step s + 1, then the two MFMAs of step s
        if (s + 1 < KSW) kf[(s + 1) & 1] = kfrag(s + 1);
        st[0] = mfma32x32x16(kf[s & 1], qf[0][s], st[0]);
        st[1] = mfma32x32x16(kf[s & 1], qf[1][s], st[1]);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      // head dim 256: each wave completes and exponentiates only its own
      // block 0 (the partner does block 1), so no score is exponentiated twice
      constexpr int NQ = DS == 2 ? 1 : 2;
      if constexpr (DS == 2) {
        // send the partial scores of block 1, add the partner's to block 0
        float* mine = xbuf + wave * 64 * 32;
        const float* other = xbuf + (wave ^ 1) * 64 * 32;
#pragma unroll
        for (int c = 0; c < 4; ++c)
          *(f32x4*)(mine + (c * 64 + lane) * 4) =
              f32x4{st[1][4 * c], st[1][4 * c + 1], st[1][4 * c + 2], st[1][4 * c + 3]};
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0) only
        tile_barrier();
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const f32x4 o = *(const f32x4*)(other + (c * 64 + lane) * 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) st[0][4 * c + e] += o[e];
        }
      }

      const int k0 = tile * kKeys2;
      // keys of this tile a lane sees: k0 + hi*4 + kj, kj = (j/4)*8 + j%4 <= 27;
      // tiles wholly visible to every row of the wave skip the masking
      int lim[2];
#pragma unroll
      for (int qb = 0; qb < NQ; ++qb)
        lim[qb] = (CAUSAL ? min(kend - 1, pos[qb]) : kend - 1) - k0 - hi * 4;
      const bool masked =
          __ballot((NQ == 1 ? lim[0] : min(lim[0], lim[1])) < 27) != 0 || (!CAUSAL && a.mask);
      if (masked) {
#pragma unroll
        for (int qb = 0; qb < NQ; ++qb)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int kj = (j / 4) * 8 + (j % 4);
            bool ok = kj <= lim[qb];
            if (!CAUSAL && a.mask)
              ok = ok && a.mask[(int64_t)b * a.L + min(k0 + hi * 4 + kj, a.L - 1)] != 0;
            if (!ok) st[qb][j] = -INFINITY;
          }
      }
      bf16x8 pf[2][2];
#pragma unroll
      for (int qb = 0; qb < NQ; ++qb) {
        // raw scores: the max is taken before scaling (scale > 0)
        float tmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < 16; ++j) tmax = fmaxf(tmax, st[qb][j]);
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64)) * sl2;
        if (m_ref[qb] == -INFINITY) m_ref[qb] = tmax;  // nothing accumulated yet
        m_true[qb] = fmaxf(m_true[qb], tmax);
        overflow |= tmax > m_ref[qb] + 64.0f;
        // p = 2^(s*scale - m_ref): the hardware exp2 gives 0 for -inf
        const float nm = m_ref[qb] == -INFINITY ? 0.f : -m_ref[qb];
        float psum = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float p = __builtin_amdgcn_exp2f(fminf(fmaf(st[qb][j], sl2, nm), 64.0f));
          psum += p;
          pf[qb][j / 8][j % 8] = (__bf16)p;
        }
        psum += __shfl_xor(psum, 32, 64);
        l[qb] += psum;
      }
      if constexpr (DS == 2) {
        // hand P of block 0 to the partner, take the partner's as block 1
        float* mine = xbuf + wave * 64 * 32 + 4 * 64 * 4;
        const float* other = xbuf + (wave ^ 1) * 64 * 32 + 4 * 64 * 4;
#pragma unroll
        for (int c = 0; c < 2; ++c)
          *(u32x4*)(mine + (c * 64 + lane) * 4) = __builtin_bit_cast(u32x4, pf[0][c]);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0) only
        tile_barrier();
#pragma unroll
        for (int c = 0; c < 2; ++c)
          pf[1][c] = as_bf16x8(*(const u32x4*)(other + (c * 64 + lane) * 4));
      }
      // O^T[d, query] += V^T[d, keys] P^T[keys, query]; k-step ks covers keys
      // 16ks + {0-3, 8-11} (+4 for the upper half-wave), the order S^T leaves.
      // Each fragment's two transpose reads are issued one step ahead.
      __builtin_amdgcn_sched_barrier(0);
      // fragment f = ks2 * DT + dt: two transpose reads
      auto vfrag = [&](int f) {
        const int ks2 = f / DT, dg = dbase + f % DT;
        v4s_t part[2];
#pragma unroll
        for (int rd = 0; rd < 2; ++rd) {
          const bf16_t* p = vs + v_off[dg & 3] + (dg >> 2) * 128 + (16 * ks2 + 8 * rd) * D;
          part[rd] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s_t*)p);
        }
        const u32x2 lo = __builtin_bit_cast(u32x2, part[0]);
        const u32x2 up = __builtin_bit_cast(u32x2, part[1]);
        return as_bf16x8(u32x4{lo[0], lo[1], up[0], up[1]});
      };
      bf16x8 vf[2];
      vf[0] = vfrag(0);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int f = 0; f < 2 * DT; ++f) {
        if (f + 1 < 2 * DT) vf[(f + 1) & 1] = vfrag(f + 1);
        const int ks2 = f / DT, dt = f % DT;
        O[0][dt] = mfma32x32x16(vf[f & 1], pf[0][ks2], O[0][dt]);
        O[1][dt] = mfma32x32x16(vf[f & 1], pf[1][ks2], O[1][dt]);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      // tile + 2 goes into the stage of tile - 1, which every wave finished
      // before the barrier above.  Issued after this tile's LDS reads: the
      // compiler makes the transpose reads wait for all outstanding LDS DMA,
      // and this way only tile + 1's (issued an iteration ago) is pending.
      if (tile + 2 < ntiles) issue(tile + 2, (tile + 2) % kStages2);
    }
    // every wave has finished with the LDS stages; decide together.  Head
    // dim 256: block 1's row statistics are the partner's block 0 ones
    if constexpr (DS == 2)
      *(f32x4*)(xbuf + wave * 64 * 32 + lane * 4) = f32x4{m_ref[0], m_true[0], l[0], 0.f};
    __builtin_amdgcn_s_waitcnt(0);
    if (tid == 0) redo = 0;
    __syncthreads();
    if constexpr (DS == 2) {
      const f32x4 o = *(const f32x4*)(xbuf + (wave ^ 1) * 64 * 32 + lane * 4);
      m_ref[1] = o[0];
      m_true[1] = o[1];
      l[1] = o[2];
    }
    if (__ballot(overflow) != 0 && lane == 0) atomicOr(&redo, 1);
    __syncthreads();
    if (pass == 1 || redo == 0) break;
    m_ref[0] = m_true[0];
    m_ref[1] = m_true[1];
    __syncthreads();
  }

  // suffix keys' V rows (decode), then normalise, gate and store
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    int64_t n;
    int t, h;
    row_of_q(qb, n, t, h);
    if (!CAUSAL) {
#pragma unroll
      for (int j = 0; j < NSUF; ++j) {
        const float sj = sc[qb][j];
        if (sj == -INFINITY) continue;
        const float pj = exp2f(sj - m_ref[qb]);
        const bf16_t* vrow = a.sv + n * a.ssv_n + (int64_t)j * a.ssv_t + (int64_t)kh * a.ssv_h;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            const int d0 = (dbase + dt) * 32 + gq * 8 + hi * 4;
            const u32x2 v2 = *(const u32x2*)(vrow + d0);
            O[qb][dt][gq * 4 + 0] += pj * __uint_as_float(v2[0] << 16);
            O[qb][dt][gq * 4 + 1] += pj * __uint_as_float(v2[0] & 0xffff0000u);
            O[qb][dt][gq * 4 + 2] += pj * __uint_as_float(v2[1] << 16);
            O[qb][dt][gq * 4 + 3] += pj * __uint_as_float(v2[1] & 0xffff0000u);
          }
      }
    }
    const int64_t r = (int64_t)qb_blk * ROWS + qgrp * 64 + (qb ^ swap) * 32 + col;
    if (r >= rows_total) continue;
    const float inv = l[qb] > 0.f ? 1.0f / l[qb] : 0.f;
    bf16_t* orow = a.out + n * a.so_n + (int64_t)t * a.so_t + (int64_t)h * a.so_h;
    const bf16_t* grow =
        a.gate ? a.gate + n * a.sg_n + (int64_t)t * a.sg_t + (int64_t)h * a.sg_h : nullptr;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const int d0 = (dbase + dt) * 32 + gq * 8 + hi * 4;
        float o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = round_bf(O[qb][dt][gq * 4 + i] * inv);
        if (grow) {
          const u32x2 g2 = *(const u32x2*)(grow + d0);
          const float gv[4] = {__uint_as_float(g2[0] << 16), __uint_as_float(g2[0] & 0xffff0000u),
                               __uint_as_float(g2[1] << 16), __uint_as_float(g2[1] & 0xffff0000u)};
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = o[i] * round_bf(sigmoid_f(gv[i]));
        }
        u32x2 packed;
        packed[0] = (uint32_t)f2bf(o[0]) | ((uint32_t)f2bf(o[1]) << 16);
        packed[1] = (uint32_t)f2bf(o[2]) | ((uint32_t)f2bf(o[3]) << 16);
        *(u32x2*)(orow + d0) = packed;
      }
  }
}

template <int D, bool CAUSAL, int NSUF>
int launch_attn2(AttnArgs a, int64_t rows, int64_t bh, hipStream_t s) {
  a.nqblk = (int)kad_cdiv(rows, Attn2<D>::ROWS);
  const int64_t nblocks = bh * a.nqblk;
  KAD_REQUIRE(nblocks < 0x7fffffff, "grid too large");
  const size_t lds = Attn2<D>::lds;
  static bool configured = false;
  if (!configured) {
    if (hipFuncSetAttribute((const void*)attn2_kernel<D, CAUSAL, NSUF>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
      kad_set_error("attention: cannot reserve %zu bytes of LDS", lds);
      return KAD_ERR_HIP;
    }
    configured = true;
  }
  hipLaunchKernelGGL((attn2_kernel<D, CAUSAL, NSUF>), dim3((unsigned)nblocks), dim3(kThreads), lds, s,
                     a);
  return kad_launch_status("attn2_kernel");
}

// ---------------------------------------------------------------------------
// Head dim 256: one wave per 32 query rows over the whole head dim (128 rows
// per workgroup, 4 waves, one per SIMD), software-pipelined over key tiles.
// Iteration t runs the softmax of tile t on the VALU while the MFMAs of tile
// t+1's scores S^T = K Q^T execute (interleaved step by step), then
// O^T += V^T P^T for tile t, with the second half of tile t's exponentials
// and the loads of tile t+3 between its MFMAs.  No wave depends on another's
// scores, so the only barrier per tile is the one that frees an LDS stage.
// K/V tiles move HBM -> LDS by global_load_lds_dwordx4 into a ring of 4
// stages, three tiles ahead (per-lane source offsets computed once); the V^T
// transpose reads are written as inline assembly with their own waits, so
// that they do not wait for those loads (the compiler makes the
// ds_read_b64_tr_b16 builtin wait for every LDS DMA in flight).  The
// epilogue transposes O through LDS, so that the suffix V rows, the gate and
// the output move as whole 512-byte rows.  Per row the arithmetic is fixed:
// the score is one MFMA chain over the 256-d dot product, the suffix dot
// products a sequential fp32 sum, whatever the launch shape.
constexpr int kStages3 = 4;

struct Attn3 {
  static constexpr int D = 256, CPR = D / 8, ROWS = 128;
  static constexpr int tile = kKeys2 * D, stage = 2 * tile;
  static constexpr int LOADS = CPR / 8;               // DMA instructions per wave per K (or V) tile
  static constexpr int EpiLd = D + 4;                 // fp32 row stride of the epilogue transpose
  static constexpr int stage_bytes = kStages3 * stage * 2;
  static constexpr int epi_bytes = ROWS * EpiLd * 4;
  static constexpr int lds = stage_bytes > epi_bytes ? stage_bytes : epi_bytes;  // bytes
};

// p with both halves read from the first active lane: a wave-uniform value
// the compiler can see as one (a buffer resource it cannot prove uniform
// turns every load into a loop over lanes)
__device__ __forceinline__ const bf16_t* uniform_ptr(const bf16_t* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi32 = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const bf16_t*)(uintptr_t)(((uint64_t)hi32 << 32) | lo);
}
// 16 bytes per lane from base + voff into LDS through a buffer resource of
// nbytes bytes (pieces past it read zeros); base and nbytes wave-uniform
__device__ __forceinline__ void dma16_extent(const bf16_t* base, int nbytes, uint32_t voff,
                                             bf16_t* lds) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(base), 0, nbytes, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (attn_lds_t*)lds, 16, voff, 0, 0, 0);
}

// max and sum of a value over lanes l and l ^ 32 (both lanes get the same bits)
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// one ds_read_b64_tr_b16 whose result may be used only after an
// s_waitcnt lgkmcnt(N) issued by the caller through tr_wait
__device__ __forceinline__ u32x2 tr_read(const bf16_t* p) {
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r) : "v"((uint32_t)(uintptr_t)p) : "memory");
  return r;
}
// the same at a constant byte offset from p (the instruction's offset field,
// so that a tile's reads share a few base addresses)
template <int OFF>
__device__ __forceinline__ u32x2 tr_read_at(const bf16_t* p) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field is 16 bits");
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
               : "=v"(r)
               : "v"((uint32_t)(uintptr_t)p), "i"(OFF)
               : "memory");
  return r;
}
// lgkmcnt(N) (vmcnt and expcnt not waited), tied to the fragment registers so
// that their uses stay after it
template <int N>
__device__ __forceinline__ void tr_wait(u32x2& a, u32x2& b) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a), "+v"(b) : "i"(N));
}

// MASKED: a prefix mask is given (decode); an instantiation of its own, so
// that the unmasked key loop carries no mask loads or branches
template <bool CAUSAL, int NSUF, bool MASKED>
__global__ __launch_bounds__(kThreads, 1) void attn3_kernel(AttnArgs a) {
  constexpr int D = 256, KS = D / 16, DT = D / 32, ROWS = Attn3::ROWS, CPR = Attn3::CPR;
  constexpr int LOADS = Attn3::LOADS;
  extern __shared__ __attribute__((aligned(1024))) bf16_t smem[];
  __shared__ int redo;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int hi = lane >> 5, col = lane & 31;
  const int lid = xcd_logical_id(blockIdx.x, gridDim.x);
  // causal: the blocks of a (request, KV head) go out longest first (the
  // last query rows see the most keys), so that the short ones fill the tail
  const int qb_blk = CAUSAL ? a.nqblk - 1 - lid % a.nqblk : lid % a.nqblk;
  const int bk = lid / a.nqblk;
  const int kh = bk % a.HK, b = bk / a.HK;
  const int G = a.H / a.HK;
  const int64_t rows_total = CAUSAL ? (int64_t)a.L * G : (int64_t)a.W * G * a.T;

  // query row r of this (request, KV head): batch row n, suffix (or prompt)
  // position t, head h
  auto row_of = [&](int64_t r, int64_t& n, int& t, int& h) {
    int g;
    if (CAUSAL) {
      t = (int)(r / G);
      g = (int)(r % G);
      n = b;
    } else {
      t = (int)(r % a.T);
      const int64_t wg = r / a.T;
      g = (int)(wg % G);
      n = (int64_t)b * a.W + wg / G;
    }
    h = kh * G + g;
  };
  const int64_t r_lane = (int64_t)qb_blk * ROWS + wave * 32 + col;
  int64_t n;
  int t, h;
  row_of(r_lane < rows_total ? r_lane : 0, n, t, h);
  bf16x8 qf[KS];
  {
    const bf16_t* qrow = a.q + n * a.sq_n + (int64_t)t * a.sq_t + (int64_t)h * a.sq_h;
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = as_bf16x8(*(const u32x4*)(qrow + s * 16 + hi * 8));
  }
  const float sl2 = a.scale * 1.4426950408889634f;  // scores in log2 units

  // ---- prefix key range and the DMA plan: instruction k of a wave covers
  // tile rows (wave + 4k) * 2 + lane / 32, 16-byte chunk lane % 32 of each
  int kend = a.L;
  if (CAUSAL) {
    const int64_t rlast = min((int64_t)(qb_blk + 1) * ROWS, rows_total) - 1;
    kend = (int)(rlast / G) + 1;
  }
  const int ntiles = (kend + kKeys2 - 1) / kKeys2;
  // leading tiles every row of the block sees whole (no prefix mask either)
  int nfull = kend / kKeys2;
  if (CAUSAL) nfull = min(nfull, (int)(((int64_t)qb_blk * ROWS / G + 1) / kKeys2));
  if (MASKED) nfull = 0;
  const bf16_t* pkb = a.pk + (int64_t)b * a.sp_b + (int64_t)kh * a.sp_h;
  const bf16_t* pvb = a.pv + (int64_t)b * a.sp_b + (int64_t)kh * a.sp_h;
  const int d_row = lane / CPR, d_pc = lane % CPR;
  // byte offsets of this lane's 16-byte pieces from the tile's first key
  uint32_t dk_off[LOADS], dv_off[LOADS];
#pragma unroll
  for (int k = 0; k < LOADS; ++k) {
    const int r = (wave + 4 * k) * (64 / CPR) + d_row;
    dk_off[k] = (uint32_t)(r * (int)a.sp_l + (d_pc ^ (r & 15)) * 8) * 2u;
    dv_off[k] = (uint32_t)(r * (int)a.sp_l + (d_pc ^ ((r & 3) * 4)) * 8) * 2u;
  }
  // loads of one tile through buffer resources based at the tile's first key
  // whose extent ends at the prefix end: rows past the prefix (in its last
  // tile) read zeros, which the key mask makes weightless; the wave's
  // destination in the tile's stage
  struct TileLoad {
    const bf16_t* kb;
    const bf16_t* vb;
    int nrec;   // bytes from the tile's first key to the prefix end
    bf16_t* dst;
  };
  auto tile_load = [&](int tile) {
    TileLoad tl;
    const int k0 = tile * kKeys2;
    tl.kb = uniform_ptr(pkb + (int64_t)k0 * a.sp_l);
    tl.vb = uniform_ptr(pvb + (int64_t)k0 * a.sp_l);
    // (the launcher bounds L * sp_l * 2 below 2^31)
    tl.nrec = __builtin_amdgcn_readfirstlane(max(a.L - k0, 0) * (int)a.sp_l * 2);
    tl.dst = smem + (tile % kStages3) * Attn3::stage + wave * 64 * 8;
    return tl;
  };
  auto issue_one = [&](const TileLoad& tl, int k) {
    bf16_t* kd = tl.dst + k * 4 * 64 * 8;
    dma16_extent(tl.kb, tl.nrec, dk_off[k], kd);
    dma16_extent(tl.vb, tl.nrec, dv_off[k], kd + Attn3::tile);
  };
  auto issue = [&](int tile) {
    const TileLoad tl = tile_load(tile);
#pragma unroll
    for (int k = 0; k < LOADS; ++k) issue_one(tl, k);
  };
  // K fragment offsets (A operand, 32 keys x 16 d; row col, logical chunk
  // 2s + hi stored at chunk ^ (row & 15)) and V^T transpose-read offsets, as
  // in attn2_kernel for head dim 256
  int k_off[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) k_off[s] = col * D + ((2 * s + hi) ^ (col & 15)) * 8;
  int v_off[4];
  {
    const int grp = lane >> 4, gi = lane & 15;
    const int v_row = 4 * (grp >> 1) + (gi >> 2);
    const int v_dq = (grp & 1) * 16 + (gi & 3) * 4;
    const int v_sw = (v_row & 3) * 4;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int d = dt * 32 + v_dq;
      v_off[dt] = v_row * D + (((d >> 3) ^ v_sw) * 8) + (d & 7);
    }
  }

  // suffix scores (decode): sequential fp32 dot products over the head dim
  float m_ref = -INFINITY;
  float sc[NSUF];
#pragma unroll
  for (int j = 0; j < NSUF; ++j) sc[j] = -INFINITY;
  if (!CAUSAL) {
#pragma unroll
    for (int j = 0; j < NSUF; ++j) {
      if (j >= a.Tk) continue;
      const bf16_t* krow = a.sk + n * a.ssk_n + (int64_t)j * a.ssk_t + (int64_t)kh * a.ssk_h;
      float part = 0.f;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const bf16x8 kb = as_bf16x8(*(const u32x4*)(krow + s * 16 + hi * 8));
#pragma unroll
        for (int i = 0; i < 8; ++i) part += (float)qf[s][i] * (float)kb[i];
      }
      part += __shfl_xor(part, 32, 64);
      if (j <= t + a.qoff) {
        sc[j] = part * sl2;
        m_ref = fmaxf(m_ref, sc[j]);
      }
    }
  }

  // Softmax with a fixed reference, as attn2_kernel: p = 2^(s - m_ref), m_ref
  // the first max the row sees; a row whose later scores exceed it by more
  // than 2^64 makes the workgroup run the key loop again with its true max
  // (so the first pass needs no clamp: its p can only exceed 2^64 when that
  // pass is discarded).
  float m_true = m_ref;
  float l = 0.f;
  f32x16 O[DT];
  const int pos = t;
  auto kfrag = [&](const bf16_t* ks, int s) {
    return as_bf16x8(*(const u32x4*)(ks + k_off[s & 7] + (s >> 3) * 128));
  };
  for (int pass = 0; pass < 2; ++pass) {
    bool overflow = false;
    l = 0.f;
#pragma unroll
    for (int j = 0; j < NSUF; ++j)
      if (sc[j] != -INFINITY) l += exp2f(sc[j] - m_ref);
#pragma unroll
    for (int i = 0; i < DT; ++i) O[i] = f32x16{};

    if (ntiles > 0) {
      issue(0);
      if (ntiles > 1) issue(1);
      if (ntiles > 2) issue(2);
      // tile 0 landed (the later ones stay in flight)
      if (ntiles > 2)
        __builtin_amdgcn_s_waitcnt(0x0070 | ((4 * LOADS) & 0xF) | (((4 * LOADS) >> 4) << 14));
      else if (ntiles > 1)
        __builtin_amdgcn_s_waitcnt(0x0070 | ((2 * LOADS) & 0xF) | (((2 * LOADS) >> 4) << 14));
      else
        __builtin_amdgcn_s_waitcnt(0x0070);
      tile_barrier();
      f32x16 st0 = f32x16{}, st1 = f32x16{};
      {
        bf16x8 kf[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) kf[s] = kfrag(smem, s);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          st0 = mfma32x32x16(kf[s & 3], qf[s], st0);
          if (s + 4 < KS) kf[s & 3] = kfrag(smem, s + 4);
        }
      }
      // one key tile: st holds its scores; with kNext, the scores of tile + 1
      // go to st_next.  Straight-line code apart from the rare prefix mask
      // and the load issue, so that the accumulators keep their registers.
      // kMaskC: the tile holds keys some row must not see (the prefix end,
      // or a causal row's own position); tiles below nfull need no mask
      auto step = [&](const int tile, f32x16& st, f32x16& st_next, auto next_c, auto mask_c) {
        constexpr bool kNext = decltype(next_c)::value;
        constexpr bool kMaskC = decltype(mask_c)::value;
        // tile + 1 landed (tile + 2 may still be in flight); every wave has
        // finished iteration tile - 1, whose stage the loads of tile + 3 reuse
        if (tile + 2 < ntiles)
          __builtin_amdgcn_s_waitcnt(0x0070 | ((2 * LOADS) & 0xF) | (((2 * LOADS) >> 4) << 14));
        else
          __builtin_amdgcn_s_waitcnt(0x0070);
        tile_barrier();
        const int k0 = tile * kKeys2;
        if constexpr (!CAUSAL && MASKED) {
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int kj = (j / 4) * 8 + (j % 4);
            if (a.mask[(int64_t)b * a.L + min(k0 + hi * 4 + kj, a.L - 1)] == 0) st[j] = -INFINITY;
          }
        }
        // keys of this tile a lane sees: k0 + hi*4 + kj, kj = (j/4)*8 + j%4 <= 27
        const int lim = (CAUSAL ? min(kend - 1, pos) : kend - 1) - k0 - hi * 4;
        bf16x8 pf[2];
        float tmax = -INFINITY, tmax_o = 0.f, nm = 0.f, psum = 0.f;
        // VALU work of score step s: masking and the row max over 4 scores
        // (s < 4), the max across the half-waves (4, 5), then the
        // exponentials of keys 0-7 (6..13); keys 8-15 follow in the PV steps
        auto softmax_step = [&](int s) {
          if (s < 4) {
#pragma unroll
            for (int j = 4 * s; j < 4 * s + 4; ++j) {
              const int kj = (j / 4) * 8 + (j % 4);
              if constexpr (kMaskC) st[j] = kj <= lim ? st[j] : -INFINITY;
              tmax = fmaxf(tmax, st[j]);
            }
          } else if (s == 4) {
            tmax_o = xor32_max(tmax);
          } else if (s == 5) {
            tmax = tmax_o * sl2;
            m_ref = m_ref == -INFINITY ? tmax : m_ref;
            m_true = fmaxf(m_true, tmax);
            overflow |= tmax > m_ref + 64.0f;
            nm = m_ref == -INFINITY ? 0.f : -m_ref;
          } else if (s < 14) {
            const int j = s - 6;
            const float p = __builtin_amdgcn_exp2f(fmaf(st[j], sl2, nm));
            psum += p;
            pf[0][j] = (__bf16)p;
          }
        };
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (kNext) {
          const bf16_t* ks = smem + ((tile + 1) % kStages3) * Attn3::stage;
          bf16x8 kf[4];
#pragma unroll
          for (int s = 0; s < 4; ++s) kf[s] = kfrag(ks, s);
          st_next = f32x16{};
#pragma unroll
          for (int s = 0; s < KS; ++s) {
            st_next = mfma32x32x16(kf[s & 3], qf[s], st_next);
            if (s + 4 < KS) kf[s & 3] = kfrag(ks, s + 4);
            softmax_step(s);
            __builtin_amdgcn_sched_barrier(0);
          }
        } else {
#pragma unroll
          for (int s = 0; s < KS; ++s) softmax_step(s);
        }
        __builtin_amdgcn_sched_barrier(0);
        // the loads of tile + 3 go into the stage of tile - 1 (free since the
        // barrier above), spread over the PV steps below so that the four
        // waves' loads do not queue up at once; the transpose reads do not
        // wait for them
        const bool load3 = tile + 3 < ntiles;
        const TileLoad tl3 = tile_load(tile + 3);

        // ---- O^T[d, query] += V^T[d, keys] P^T[keys, query] for tile; k-step
        // ks2 covers keys 16ks2 + {0-3, 8-11} (+4 for the upper half-wave);
        // each fragment's two transpose reads go out three fragments ahead,
        // and the exponentials of keys 8-15 run under the first 8 MFMAs
        const bf16_t* vs = smem + (tile % kStages3) * Attn3::stage + Attn3::tile;
        // fragment f, read rd: base vb[dg & 3] plus a constant byte offset
        const bf16_t* vb[4] = {vs + v_off[0], vs + v_off[1], vs + v_off[2], vs + v_off[3]};
        constexpr int NF = 2 * DT, AHEAD = 3;
        auto vread = [&](auto f_c, auto rd_c) {
          constexpr int f = decltype(f_c)::value, rd = decltype(rd_c)::value;
          constexpr int ks2 = f / DT, dg = f % DT;
          return tr_read_at<((dg >> 2) * 128 + (16 * ks2 + 8 * rd) * D) * 2>(vb[dg & 3]);
        };
        u32x2 vlo[AHEAD + 1], vup[AHEAD + 1];
        static_for<AHEAD>([&](auto f_c) {
          constexpr int f = decltype(f_c)::value;
          vlo[f] = vread(f_c, std::integral_constant<int, 0>{});
          vup[f] = vread(f_c, std::integral_constant<int, 1>{});
        });
        static_for<NF>([&](auto f_c) {
          constexpr int f = decltype(f_c)::value;
          const int cur = f % (AHEAD + 1);
          if constexpr (f + AHEAD < NF) {
            const int nxt = (f + AHEAD) % (AHEAD + 1);
            vlo[nxt] = vread(std::integral_constant<int, f + AHEAD>{},
                             std::integral_constant<int, 0>{});
            vup[nxt] = vread(std::integral_constant<int, f + AHEAD>{},
                             std::integral_constant<int, 1>{});
            tr_wait<2 * AHEAD>(vlo[cur], vup[cur]);
          } else if constexpr (f + 2 == NF) {
            tr_wait<2>(vlo[cur], vup[cur]);
          } else if constexpr (f + 1 == NF) {
            tr_wait<0>(vlo[cur], vup[cur]);
          } else {
            tr_wait<4>(vlo[cur], vup[cur]);
          }
          const bf16x8 vf = as_bf16x8(u32x4{vlo[cur][0], vlo[cur][1], vup[cur][0], vup[cur][1]});
          O[f % DT] = mfma32x32x16(vf, pf[f / DT], O[f % DT]);
          if constexpr (f < 8) {
            const float p = __builtin_amdgcn_exp2f(fmaf(st[8 + f], sl2, nm));
            psum += p;
            pf[1][f] = (__bf16)p;
          }
          if constexpr (f == 8) l += xor32_sum(psum);
          if constexpr (f % 4 == 2) {
            if (load3) issue_one(tl3, f / 4);
          }
          __builtin_amdgcn_sched_barrier(0);
        });
      };
      using yes = std::integral_constant<bool, true>;
      using no = std::integral_constant<bool, false>;
      int tile = 0;
      for (; tile + 2 < ntiles && tile + 2 <= nfull; tile += 2) {
        step(tile, st0, st1, yes{}, no{});
        step(tile + 1, st1, st0, yes{}, no{});
      }
      for (; tile + 2 < ntiles; tile += 2) {
        step(tile, st0, st1, yes{}, yes{});
        step(tile + 1, st1, st0, yes{}, yes{});
      }
      if (tile + 1 < ntiles) {
        step(tile, st0, st1, yes{}, yes{});
        step(tile + 1, st1, st0, no{}, yes{});
      } else {
        step(tile, st0, st1, no{}, yes{});
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    if (tid == 0) redo = 0;
    __syncthreads();
    if (__ballot(overflow) != 0 && lane == 0) atomicOr(&redo, 1);
    __syncthreads();
    if (pass == 1 || redo == 0) break;
    m_ref = m_true;
    __syncthreads();
  }

  // ---- epilogue: O^T goes through LDS (the stages are free: every wave
  // passed the barrier after its last load and read), then each wave writes
  // its 32 rows one 512-byte row at a time, 4 elements per lane, 8 rows'
  // loads in flight together: the suffix keys' V rows (decode), the
  // normalisation, the gate, the store.  A row's scalars (1/l, the suffix
  // keys' weights, its offsets) come from the lane that owns it by readlane,
  // and the code is branch-free but for the store of rows past the end.
  float* ep = (float*)smem + wave * 32 * Attn3::EpiLd;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const int d0 = dt * 32 + gq * 8 + hi * 4;
      *(f32x4*)(ep + col * Attn3::EpiLd + d0) =
          f32x4{O[dt][gq * 4], O[dt][gq * 4 + 1], O[dt][gq * 4 + 2], O[dt][gq * 4 + 3]};
    }
  // this lane's row: 1/l, the suffix weights (0 for a key the row does not
  // see) and the offsets of its output, gate and suffix V rows
  const float inv_l = l > 0.f ? 1.0f / l : 0.f;
  float pw[NSUF];
#pragma unroll
  for (int j = 0; j < NSUF; ++j) pw[j] = sc[j] == -INFINITY ? 0.f : exp2f(sc[j] - m_ref);
  const int64_t off_o = n * a.so_n + (int64_t)t * a.so_t + (int64_t)h * a.so_h;
  const int64_t off_g = n * a.sg_n + (int64_t)t * a.sg_t + (int64_t)h * a.sg_h;
  const int64_t off_v = n * a.ssv_n + (int64_t)kh * a.ssv_h;
  auto row_i64 = [&](int64_t v, int r) {
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, r);
    const uint32_t hi32 = __builtin_amdgcn_readlane((uint32_t)(v >> 32), r);
    return (int64_t)(((uint64_t)hi32 << 32) | lo);
  };
  // the builtin takes and returns int: a float goes through as its bits
  auto lane_f32 = [](float v, int r) {
    return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(v), r));
  };
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): a wave reads only its own rows
  const int d0 = lane * 4;
  const int64_t row0 = (int64_t)qb_blk * ROWS + wave * 32;
  const int nrows = (int)min<int64_t>(32, rows_total - row0);
  const int tk = CAUSAL ? 0 : min(a.Tk, NSUF);
  // the gate's sigmoid takes the hardware reciprocal (1 ulp) in place of
  // the IEEE divide, the bulk of this VALU-bound tail
  auto rows = [&](auto gated_c, auto suffix_c) {
    constexpr bool kGated = decltype(gated_c)::value;
    constexpr bool kSuffix = decltype(suffix_c)::value;
    constexpr int RB = 8;
    for (int rb = 0; rb < nrows; rb += RB) {
      u32x2 gv[RB], vv[RB][NSUF];
      int64_t oo[RB];
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int rr = min(rb + i, nrows - 1);
        oo[i] = row_i64(off_o, rr);
        if constexpr (kGated) gv[i] = *(const u32x2*)(a.gate + row_i64(off_g, rr) + d0);
        if constexpr (kSuffix) {
          const bf16_t* vrow = a.sv + row_i64(off_v, rr) + d0;
#pragma unroll
          for (int j = 0; j < NSUF; ++j)   // keys past Tk repeat the last one (weight 0)
            vv[i][j] = *(const u32x2*)(vrow + (int64_t)min(j, tk - 1) * a.ssv_t);
        }
      }
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int rr = min(rb + i, nrows - 1);
        const f32x4 ov = *(const f32x4*)(ep + rr * Attn3::EpiLd + d0);
        float o[4] = {ov[0], ov[1], ov[2], ov[3]};
        if constexpr (kSuffix) {
#pragma unroll
          for (int j = 0; j < NSUF; ++j) {
            const float pj = lane_f32(pw[j], rr);
            o[0] += pj * __uint_as_float(vv[i][j][0] << 16);
            o[1] += pj * __uint_as_float(vv[i][j][0] & 0xffff0000u);
            o[2] += pj * __uint_as_float(vv[i][j][1] << 16);
            o[3] += pj * __uint_as_float(vv[i][j][1] & 0xffff0000u);
          }
        }
        const float inv = lane_f32(inv_l, rr);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = round_bf(o[e] * inv);
        if constexpr (kGated) {
          const float g4[4] = {__uint_as_float(gv[i][0] << 16),
                               __uint_as_float(gv[i][0] & 0xffff0000u),
                               __uint_as_float(gv[i][1] << 16),
                               __uint_as_float(gv[i][1] & 0xffff0000u)};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            o[e] = o[e] * round_bf(__builtin_amdgcn_rcpf(1.0f + __expf(-g4[e])));
        }
        u32x2 packed;
        packed[0] = (uint32_t)f2bf(o[0]) | ((uint32_t)f2bf(o[1]) << 16);
        packed[1] = (uint32_t)f2bf(o[2]) | ((uint32_t)f2bf(o[3]) << 16);
        if (rb + i < nrows) *(u32x2*)(a.out + oo[i] + d0) = packed;
      }
    }
  };
  using yes = std::integral_constant<bool, true>;
  using no = std::integral_constant<bool, false>;
  if (a.gate) {
    if (tk > 0) rows(yes{}, yes{}); else rows(yes{}, no{});
  } else {
    if (tk > 0) rows(no{}, yes{}); else rows(no{}, no{});
  }
}

template <bool CAUSAL, int NSUF, bool MASKED>
int launch_attn3_as(const AttnArgs& a, int64_t nblocks, hipStream_t s) {
  const size_t lds = Attn3::lds;
  static bool configured = false;
  if (!configured) {
    if (hipFuncSetAttribute((const void*)attn3_kernel<CAUSAL, NSUF, MASKED>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
      kad_set_error("attention: cannot reserve %zu bytes of LDS", lds);
      return KAD_ERR_HIP;
    }
    configured = true;
  }
  hipLaunchKernelGGL((attn3_kernel<CAUSAL, NSUF, MASKED>), dim3((unsigned)nblocks),
                     dim3(kThreads), lds, s, a);
  return kad_launch_status("attn3_kernel");
}

template <bool CAUSAL, int NSUF>
int launch_attn3(AttnArgs a, int64_t rows, int64_t bh, hipStream_t s) {
  if ((int64_t)kKeys2 * a.sp_l >= 0x7fffffff)
    KAD_UNSUPPORTED("attention: prefix key stride %lld too large", (long long)a.sp_l);
  if ((int64_t)a.L * a.sp_l * 2 >= 0x7fffffff)
    KAD_UNSUPPORTED("attention: prefix of %lld bytes per head too long for 32-bit offsets",
                    (long long)a.L * a.sp_l * 2);
  a.nqblk = (int)kad_cdiv(rows, Attn3::ROWS);
  const int64_t nblocks = bh * a.nqblk;
  KAD_REQUIRE(nblocks < 0x7fffffff, "grid too large");
  if constexpr (!CAUSAL) {
    if (a.mask) return launch_attn3_as<CAUSAL, NSUF, true>(a, nblocks, s);
  }
  return launch_attn3_as<CAUSAL, NSUF, false>(a, nblocks, s);
}

// rows: query rows per (request, KV head); bh: number of (request, KV head)
// (the folds of up to 2, 4 and 8 suffix keys are instantiations of their
// own: a row's arithmetic is the same in each, the keys past Tk scoring -inf)
template <bool CAUSAL, int NSUF>
int dispatch_d(int D, const AttnArgs& a, int64_t rows, int64_t bh, hipStream_t s) {
  if (D == 256) return launch_attn3<CAUSAL, NSUF>(a, rows, bh, s);
  if (D == 128) return launch_attn2<128, CAUSAL, NSUF>(a, rows, bh, s);
  if (D == 64) return launch_attn2<64, CAUSAL, NSUF>(a, rows, bh, s);
  KAD_UNSUPPORTED("attention supports head dim 64, 128, 256; got %d", D);
}

template <bool CAUSAL>
int dispatch(int D, const AttnArgs& a, int64_t rows, int64_t bh, hipStream_t s) {
  if (!CAUSAL && a.Tk > kSuffixFold) return dispatch_d<CAUSAL, kSuffixFoldLong>(D, a, rows, bh, s);
  // one or two suffix keys (the first two search levels): a fold of two, which
  // skips the dot products and V loads of the keys a row cannot have (decode
  // attention 145 -> 139 us at one or two keys)
  if (!CAUSAL && a.Tk <= kSuffixFoldShort) return dispatch_d<CAUSAL, kSuffixFoldShort>(D, a, rows, bh, s);
  return dispatch_d<CAUSAL, kSuffixFold>(D, a, rows, bh, s);
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" int kad_prefix_attention_decode_ex(
    const void* q, int64_t sq_n, int64_t sq_t, int64_t sq_h, const void* prefix_k,
    const void* prefix_v, int64_t sp_b, int64_t sp_l, int64_t sp_h, const void* suffix_k,
    int64_t ssk_n, int64_t ssk_t, int64_t ssk_h, const void* suffix_v, int64_t ssv_n,
    int64_t ssv_t, int64_t ssv_h, const void* prefix_mask, const void* gate, int64_t sg_n,
    int64_t sg_t, int64_t sg_h, void* out, int64_t so_n, int64_t so_t, int64_t so_h, int B,
    int W, int Tq, int Tk, int H, int HK, int L, int D, float scale, kad_stream_t stream) {
  KAD_REQUIRE(q && suffix_k && suffix_v && out, "null pointer argument");
  KAD_REQUIRE(L == 0 || (prefix_k && prefix_v), "null prefix pointer with L > 0");
  KAD_REQUIRE(B > 0 && W > 0 && Tq > 0 && Tq <= Tk && H > 0 && HK > 0 && L >= 0 && D > 0,
              "bad dimensions");
  KAD_REQUIRE(H % HK == 0, "H must be divisible by HK");
  if (Tk > kSuffixFoldLong)
    KAD_UNSUPPORTED("prefix attention supports suffixes of <= %d tokens, got %d", kSuffixFoldLong,
                    Tk);
  KAD_REQUIRE(scale > 0.f && scale < INFINITY, "scale must be positive and finite");
  KAD_REQUIRE(al16(q) && al16(suffix_k) && (L == 0 || (al16(prefix_k) && al16(prefix_v))),
              "q, suffix_k and prefix K/V must be 16-byte aligned");
  KAD_REQUIRE(((uintptr_t)suffix_v | (uintptr_t)out | (uintptr_t)gate) % 8 == 0,
              "suffix_v, out and gate must be 8-byte aligned");
  for (int64_t st : {sq_n, sq_t, sq_h, sp_b, sp_l, sp_h, ssk_n, ssk_t, ssk_h})
    KAD_REQUIRE(st % 8 == 0, "q/k strides must be multiples of 8 elements");
  for (int64_t st : {ssv_n, ssv_t, ssv_h, so_n, so_t, so_h, sg_n, sg_t, sg_h})
    KAD_REQUIRE(st % 4 == 0, "v/out/gate strides must be multiples of 4 elements");
  AttnArgs a{(const bf16_t*)q, sq_n, sq_t, sq_h, (const bf16_t*)prefix_k,
             (const bf16_t*)prefix_v, sp_b, sp_l, sp_h, (const bf16_t*)suffix_k,
             (const bf16_t*)suffix_v, ssk_n, ssk_t, ssk_h, ssv_n, ssv_t, ssv_h,
             (const uint8_t*)prefix_mask, (const bf16_t*)gate, sg_n, sg_t, sg_h, (bf16_t*)out,
             so_n, so_t, so_h, W, Tq, H, HK, L, scale, 0, Tk, Tk - Tq};
  const int64_t rows = (int64_t)W * (H / HK) * Tq;
  return dispatch<false>(D, a, rows, (int64_t)B * HK, (hipStream_t)stream);
}

extern "C" int kad_prefix_attention_decode(
    const void* q, int64_t sq_n, int64_t sq_t, int64_t sq_h, const void* prefix_k,
    const void* prefix_v, int64_t sp_b, int64_t sp_l, int64_t sp_h, const void* suffix_k,
    int64_t ssk_n, int64_t ssk_t, int64_t ssk_h, const void* suffix_v, int64_t ssv_n,
    int64_t ssv_t, int64_t ssv_h, const void* prefix_mask, const void* gate, int64_t sg_n,
    int64_t sg_t, int64_t sg_h, void* out, int64_t so_n, int64_t so_t, int64_t so_h, int B,
    int W, int T, int H, int HK, int L, int D, float scale, kad_stream_t stream) {
  return kad_prefix_attention_decode_ex(q, sq_n, sq_t, sq_h, prefix_k, prefix_v, sp_b, sp_l, sp_h,
                                        suffix_k, ssk_n, ssk_t, ssk_h, suffix_v, ssv_n, ssv_t,
                                        ssv_h, prefix_mask, gate, sg_n, sg_t, sg_h, out, so_n,
                                        so_t, so_h, B, W, T, T, H, HK, L, D, scale, stream);
}

extern "C" int kad_attention_prefill(const void* q, int64_t sq_b, int64_t sq_l, int64_t sq_h,
                                     const void* k, const void* v, int64_t skv_b, int64_t skv_l,
                                     int64_t skv_h, const void* gate, int64_t sg_b, int64_t sg_l,
                                     int64_t sg_h, void* out, int64_t so_b, int64_t so_l,
                                     int64_t so_h, int B, int L, int H, int HK, int D,
                                     float scale, kad_stream_t stream) {
  KAD_REQUIRE(q && k && v && out, "null pointer argument");
  KAD_REQUIRE(B > 0 && L > 0 && H > 0 && HK > 0 && D > 0 && H % HK == 0, "bad dimensions");
  KAD_REQUIRE(scale > 0.f && scale < INFINITY, "scale must be positive and finite");
  KAD_REQUIRE(al16(q) && al16(k) && al16(v), "q, k, v must be 16-byte aligned");
  KAD_REQUIRE(((uintptr_t)out | (uintptr_t)gate) % 8 == 0, "out and gate must be 8-byte aligned");
  for (int64_t st : {sq_b, sq_l, sq_h, skv_b, skv_l, skv_h})
    KAD_REQUIRE(st % 8 == 0, "q/k/v strides must be multiples of 8 elements");
  for (int64_t st : {so_b, so_l, so_h, sg_b, sg_l, sg_h})
    KAD_REQUIRE(st % 4 == 0, "out/gate strides must be multiples of 4 elements");
  AttnArgs a{(const bf16_t*)q, sq_b, sq_l, sq_h, (const bf16_t*)k, (const bf16_t*)v, skv_b, skv_l,
             skv_h, nullptr, nullptr, 0, 0, 0, 0, 0, 0, nullptr, (const bf16_t*)gate, sg_b, sg_l,
             sg_h, (bf16_t*)out, so_b, so_l, so_h, 1, 1, H, HK, L, scale, 0, 0, 0};
  const int64_t rows = (int64_t)L * (H / HK);
  return dispatch<true>(D, a, rows, (int64_t)B * HK, (hipStream_t)stream);
}
