// bf16 GEMM on gfx950 MFMA: C[M,N] = A[M,K] * W[N,K]^T (nn.Linear layout),
// fp32 accumulation, fused epilogues.
//
// Replaces the torch nn.Linear calls of the decode and prefill paths
// (src/kadllm/adapters/qwen3_5.py:146,161-162,169,175,177,181-188,202,234-235
// and the transformers layer modules they call).
//
// Tiling: a workgroup of WAVES_M x WAVES_N waves computes a BM x BN tile; each wave owns (BM/WAVES_M) x (BN/WAVES_N) outputs
// as 32x32 v_mfma_f32_32x32x16_bf16 tiles.  K advances 64 at a time through
// double-buffered LDS tiles (rows padded by 16 bytes so that the 16-byte
// fragment reads of 8 consecutive rows hit distinct bank groups); the next
// K tile is fetched from HBM into registers while the current one feeds the
// MFMAs, with one barrier per K tile.  Tiles are ordered so that the larger
// operand is reused: N-major (each weight slice serves every M tile in turn)
// when the weight is the larger matrix, M-major otherwise, and the linear
// order is remapped so that consecutive tiles share an XCD's L2.
//
// Epilogues (bf16 rounding points follow the reference's torch modules):
//   STORE     C = bf16(acc)
//   RESIDUAL  C = bf16(R + bf16(acc))                 (x + mixed, x + mlp(x))
//   SWIGLU    weight rows interleaved per 32 as [gate 32 | up 32] blocks;
//             C[:, j] = bf16(bf16(silu(bf16(g))) * bf16(u)), N/2 columns

#include <cstdlib>

#include "kad_common.h"

namespace {

constexpr int kBK = 64;
constexpr int kPad = 8;
constexpr int kLdk = kBK + kPad;  // LDS row stride (elements)

// SiLU of the SwiGLU epilogues: x / (1 + e^-x) with the hardware reciprocal
// (1 ulp) in place of the IEEE divide, which is most of the epilogue's VALU
// work; every tile configuration uses it, so they still agree bit for bit
__device__ __forceinline__ float silu_rcp(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x));
}

// SwiGLU of two adjacent outputs, bf16(bf16(silu(bf16(g))) * bf16(u)) for
// (g0, u0) in the low half and (g1, u1) in the high half: each bf16
// rounding of the pair is one packed conversion (the same bits as rounding
// each value on its own, with half the conversions and their widenings)
__device__ __forceinline__ uint32_t swiglu2(float g0, float g1, float u0, float u1) {
  const uint32_t gp = pack_bf16x2(g0, g1), up = pack_bf16x2(u0, u1);
  const float ua = __uint_as_float(up << 16), ub = __uint_as_float(up & 0xffff0000u);
  const uint32_t sp =
      pack_bf16x2(silu_rcp(__uint_as_float(gp << 16)), silu_rcp(__uint_as_float(gp & 0xffff0000u)));
  return pack_bf16x2(__uint_as_float(sp << 16) * ua, __uint_as_float(sp & 0xffff0000u) * ub);
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int EPI>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_bf16_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ Wt, int64_t ldw,
    bf16_t* C, int64_t ldc, const bf16_t* R, int64_t ldr, int M, int N, int K, int n_major) {
  constexpr int NTH = 64 * WAVES_M * WAVES_N;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int MT = WM / 32, NT = WN / 32;
  constexpr int CPR = kBK / 8;  // 16-byte chunks per tile row
  constexpr int A_CH = BM * CPR / NTH, B_CH = BN * CPR / NTH;
  static_assert(A_CH * NTH == BM * CPR && B_CH * NTH == BN * CPR, "tile/thread mismatch");
  __shared__ __attribute__((aligned(16))) bf16_t smem[2][(BM + BN) * kLdk];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int mtiles = (M + BM - 1) / BM, ntiles = (N + BN - 1) / BN;
  const int lid = xcd_logical_id(blockIdx.x, gridDim.x);
  int mi, ni;
  if (n_major) {
    ni = lid / mtiles;
    mi = lid % mtiles;
  } else {
    mi = lid / ntiles;
    ni = lid % ntiles;
  }
  const int m0 = mi * BM, n0 = ni * BN;

  // global -> register staging (16-byte chunks); rows past M/N read a valid row
  const bf16_t* a_src[A_CH];
  const bf16_t* b_src[B_CH];
  int a_dst[A_CH], b_dst[B_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    const int c = tid + i * NTH, row = c / CPR, kc = c % CPR;
    a_src[i] = A + (int64_t)min(m0 + row, M - 1) * lda + kc * 8;
    a_dst[i] = row * kLdk + kc * 8;
  }
#pragma unroll
  for (int i = 0; i < B_CH; ++i) {
    const int c = tid + i * NTH, row = c / CPR, kc = c % CPR;
    b_src[i] = Wt + (int64_t)min(n0 + row, N - 1) * ldw + kc * 8;
    b_dst[i] = BM * kLdk + row * kLdk + kc * 8;
  }
  u32x4 a_reg[A_CH], b_reg[B_CH];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) a_reg[i] = *(const u32x4*)(a_src[i] + k0);
#pragma unroll
    for (int i = 0; i < B_CH; ++i) b_reg[i] = *(const u32x4*)(b_src[i] + k0);
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) *(u32x4*)(&smem[buf][a_dst[i]]) = a_reg[i];
#pragma unroll
    for (int i = 0; i < B_CH; ++i) *(u32x4*)(&smem[buf][b_dst[i]]) = b_reg[i];
  };

  f32x16 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = f32x16{};

  const int KT = K / kBK;
  fetch(0);
  stash(0);
  __syncthreads();
  const int frag_row = lane & 31, frag_k = (lane >> 5) * 8;
  for (int kt = 0; kt < KT; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < KT) fetch((kt + 1) * kBK);
    const bf16_t* As = &smem[buf][(wm * WM + frag_row) * kLdk + frag_k];
    const bf16_t* Bs = &smem[buf][BM * kLdk + (wn * WN + frag_row) * kLdk + frag_k];
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      bf16x8 af[MT], bfr[NT];
#pragma unroll
      for (int i = 0; i < MT; ++i) af[i] = as_bf16x8(*(const u32x4*)(As + i * 32 * kLdk + kk * 16));
#pragma unroll
      for (int j = 0; j < NT; ++j) bfr[j] = as_bf16x8(*(const u32x4*)(Bs + j * 32 * kLdk + kk * 16));
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = mfma32x32x16(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < KT) stash(buf ^ 1);
    __syncthreads();
  }

  // epilogue: lane holds column (lane % 32) and rows (j/4)*8 + (lane/32)*4 + j%4
  const int col_in = lane & 31, row_q = (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int rbase = m0 + wm * WM + i * 32 + row_q;
    if constexpr (EPI == KAD_EPI_SWIGLU) {
#pragma unroll
      for (int j = 0; j < NT; j += 2) {
        const int gcol = n0 + wn * WN + j * 32;  // start of a [gate 32 | up 32] block
        const int ocol = gcol / 2 + col_in;
        if (gcol + col_in >= N) continue;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = rbase + (e / 4) * 8 + (e % 4);
          if (row < M) {
            const float gv = round_bf(acc[i][j][e]);
            const float uv = round_bf(acc[i][j + 1][e]);
            const float s = round_bf(silu_rcp(gv));
            C[(int64_t)row * ldc + ocol] = f2bf(s * uv);
          }
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int col = n0 + wn * WN + j * 32 + col_in;
        if (col >= N) continue;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = rbase + (e / 4) * 8 + (e % 4);
          if (row < M) {
            float v = acc[i][j][e];
            if constexpr (EPI == KAD_EPI_RESIDUAL)
              v = bf2f(R[(int64_t)row * ldr + col]) + round_bf(v);
            C[(int64_t)row * ldc + col] = f2bf(v);
          }
        }
      }
    }
  }
}

// 256 x BN tiles (BN = 256 or 128) for the large GEMMs.
//
// Operand tiles move HBM -> LDS with global_load_lds_dwordx4 (no register
// staging): one wave instruction writes 64 x 16 bytes contiguously, i.e. 8
// tile rows of 128 bytes.  Within a row the 16-byte chunk c of K is stored at
// chunk c ^ ((row >> 1) & 7), so that the fragment reads (16 lanes = 16
// consecutive rows at one chunk) hit 16 distinct 16-byte bank groups; each
// lane of a load therefore fetches the global chunk that belongs at its LDS
// slot.  Two stages of 64-deep K: tile kt+1 is in flight while tile kt feeds
// the MFMAs.
//
// Operands are swapped (weight rows are the MFMA's A operand), so each lane's
// accumulators hold 4 consecutive output columns: the epilogue packs them 8
// bytes at a time into LDS, and the wave then writes its sub-tile with
// 16-byte stores (fusing the residual add or SwiGLU on the way).  Every
// configuration accumulates K in the same order, so results are bit-identical
// across tile shapes.
constexpr int kT = 256;

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

// Origin of this workgroup's BM x BN tile.  Grouped order: `group`
// consecutive tiles along the outer dimension share each inner-dimension
// tile, so an XCD's resident tiles form a 2-D block and both operands are
// reused from its L2.
__device__ __forceinline__ void tile_origin_of(int lid, int M, int N, int BM, int BN, int n_major,
                                              int group, int& m0, int& n0) {
  const int mtiles = (M + BM - 1) / BM, ntiles = (N + BN - 1) / BN;
  const int nx = n_major ? ntiles : mtiles, ny = n_major ? mtiles : ntiles;
  const int gx0 = (lid / (group * ny)) * group, gs = min(nx - gx0, group);
  const int within = lid % (group * ny);
  const int tx = gx0 + within % gs, ty = within / gs;
  const int mi = n_major ? ty : tx, ni = n_major ? tx : ty;
  m0 = mi * BM;
  n0 = ni * BN;
}

__device__ __forceinline__ void tile_origin(int M, int N, int BM, int BN, int n_major, int group,
                                           int& m0, int& n0) {
  tile_origin_of(xcd_logical_id(blockIdx.x, gridDim.x), M, N, BM, BN, n_major, group, m0, n0);
}

__device__ __forceinline__ void dma16(const bf16_t* g, bf16_t* lds_block) {
  __builtin_amdgcn_global_load_lds((global_void_t*)g, (lds_void_t*)lds_block, 16, 0, 0);
}

// The same 16 bytes per lane through a buffer resource: a per-lane 32-bit
// byte offset (voff) plus a wave-uniform one (soff) from the resource's base,
// so that no per-lane 64-bit address is formed.  Raw buffer, no format
// conversion (third dword 0x00020000); an offset past num_records reads 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                          bf16_t* lds_block) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)lds_block, 16, voff, soff, 0, 0);
}

// workgroup barrier without __syncthreads' wait for every outstanding load;
// the empty asm statements keep LDS accesses on their side of it
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(n) lgkmcnt(0), expcnt not waited (vmcnt is bits 3:0 and
// 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int wait_vm_lgkm0(int n) { return 0x0070 | (n & 15) | ((n >> 4) << 14); }

// 16x16x32 MFMA tiles: BM x BN per workgroup, WM x WN waves (an even count,
// so that a wave's DMA rows keep its swizzle phase).  mfma16x16x32(w, a, c):
// lane l supplies row l%16 and K elements 8*(l/16) .. +7 of a 32-deep step of
// each operand; acc[i][j][e] then holds output row i*16 + l%16, column
// j*16 + 4*(l/16) + e of the wave's sub-tile (4 consecutive columns per lane).
// 256 x 256 with 2 x 4 waves is the large-shape tile (two waves per SIMD);
// 128 x 128 with 2 x 2 waves runs two workgroups per CU (64 KB of LDS each),
// whose barriers then do not stall each other.

template <int BM_, int BN_, int WM_, int WN_>
struct TileX16 {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, NW = WM * WN;
  static constexpr int NI = BM / WM / 16, NJ = BN / WN / 16;      // 16 x 16 blocks per wave
  static constexpr int Stage = (BM + BN) * kBK;
  static constexpr int AG = (BM / 8) / NW, WGW = (BN / 8) / NW;   // 8-row groups per wave
  static constexpr int Cols = NJ * 16;                            // wave sub-tile columns
  static constexpr int EpiWave = NI * 16 * (Cols + 8);
  static constexpr int Smem = 2 * Stage > NW * EpiWave ? 2 * Stage : NW * EpiWave;
  static_assert(NW % 2 == 0 && AG * NW * 8 == BM && WGW * NW * 8 == BN, "tile/wave mismatch");
};
using Tile256 = TileX16<256, 256, 2, 4>;

// Epilogue of one wave's (NI*16) x (NJ*16) sub-tile through a wave-private LDS
// region, as epilogue_sub.  SwiGLU: the sub-tile's columns are whole 64-column
// [gate 32 | up 32] groups, blocks 4g, 4g+1 gate and 4g+2, 4g+3 up.
template <int EPI, int NI, int NJ>
__device__ __forceinline__ void epilogue_x16(f32x4 (&acc)[NI][NJ], bf16_t* ep, int lane,
                                             int row0, int col0, bf16_t* C, int64_t ldc,
                                             const bf16_t* R, int64_t ldr, int M, int N) {
  constexpr int kCols = EPI == KAD_EPI_SWIGLU ? NJ * 8 : NJ * 16;
  constexpr int kLd = kCols + 8;
  const int e_row = lane & 15, e_col = (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    if constexpr (EPI == KAD_EPI_SWIGLU) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if ((j & 3) >= 2) continue;
        u32x2 packed;
#pragma unroll
        for (int h = 0; h < 2; ++h)
          packed[h] = swiglu2(acc[i][j][h * 2], acc[i][j][h * 2 + 1], acc[i][j + 2][h * 2],
                              acc[i][j + 2][h * 2 + 1]);
        *(u32x2*)(ep + (i * 16 + e_row) * kLd + (j >> 2) * 32 + (j & 3) * 16 + e_col) = packed;
      }
    } else {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        u32x2 packed;
#pragma unroll
        for (int h = 0; h < 2; ++h)
          packed[h] = (uint32_t)f2bf(acc[i][j][h * 2]) | ((uint32_t)f2bf(acc[i][j][h * 2 + 1]) << 16);
        *(u32x2*)(ep + (i * 16 + e_row) * kLd + j * 16 + e_col) = packed;
      }
    }
  }
  constexpr int kChunks = kCols / 8, kRowsPer = 64 / kChunks;
  const int c_row = lane / kChunks, c_col = (lane % kChunks) * 8;
  const int n_out = EPI == KAD_EPI_SWIGLU ? N / 2 : N;
#pragma unroll 4
  for (int r = c_row; r < NI * 16; r += kRowsPer) {
    const int row = row0 + r, col = col0 + c_col;
    if (row >= M || col >= n_out) continue;
    u32x4 v = *(const u32x4*)(ep + r * kLd + c_col);
    if constexpr (EPI == KAD_EPI_RESIDUAL) {
      const u32x4 rr = *(const u32x4*)(R + (int64_t)row * ldr + col);
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const float lo = __uint_as_float(rr[h] << 16) + __uint_as_float(v[h] << 16);
        const float hi = __uint_as_float(rr[h] & 0xffff0000u) + __uint_as_float(v[h] & 0xffff0000u);
        v[h] = (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
      }
    }
    *(u32x4*)(C + (int64_t)row * ldc + col) = v;
  }
}

// issue order of a half step: NM MFMAs, the first NR each followed by one
// fragment read, the NV global loads spread over the rest
template <int NM, int NR, int NV>
__device__ __forceinline__ void interleave_x16() {
#pragma unroll
  for (int t = 0; t < NM; ++t) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (t < NR) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    } else if constexpr (NV > 0) {
      constexpr int kSlots = NM > NR ? NM - NR : 1;
      const int c = ((t - NR + 1) * NV) / kSlots - ((t - NR) * NV) / kSlots;
#pragma unroll
      for (int q = 0; q < c; ++q) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

// 256 x BN tile, 8 waves, 16x16x32 MFMAs; two 64-deep LDS stages, two 32-deep
// steps per tile.  One barrier per tile, between the two steps (step 1's
// fragments are read during step 0): past it the next tile has landed (each
// wave waited for its own loads) and every wave has read its last fragments
// of the current stage, so the loads of the tile after next go out into that
// stage at once, and step 1's MFMAs cover them and the next tile's step-0
// fragment reads.  (With the barrier in the middle of step 1, only 16 MFMAs
// per wave followed it: 3.6% slower over the search's shapes.)
//
// The two waves of a SIMD share its MFMA unit, and the older one wins the
// issue arbitration: it runs both of its half steps while the younger one's
// post-barrier half step, whose global->LDS loads block issue whenever the
// CU's load queue is full, falls behind; the older wave then idles at the
// next barrier.  Raising the wave priority (s_setprio 1) for the half step
// after the barrier lets a lagging wave's MFMAs and loads go first (2.5%
// faster over the search's shapes, every shape gaining).  This is the
// instruction arbiter's wave priority, not a queue priority.
template <int EPI, class TX>
__global__ __launch_bounds__(64 * TX::NW) void gemm_x16_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ Wt, int64_t ldw,
    bf16_t* C, int64_t ldc, const bf16_t* R, int64_t ldr, int M, int N, int K, int n_major,
    int group) {
  constexpr int BM = TX::BM, BN = TX::BN;
  constexpr int NW = TX::NW, WN = TX::WN, NI = TX::NI, NJ = TX::NJ;
  constexpr int kStage = TX::Stage, AG = TX::AG, WGW = TX::WGW;
  constexpr int kLoads = AG + WGW;
  constexpr int NM = NI * NJ, NR = NI + NJ;
  __shared__ __attribute__((aligned(1024))) bf16_t smem[TX::Smem];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int m0, n0;
  tile_origin(M, N, BM, BN, n_major, group, m0, n0);

  // row groups g = wave + 8 i (8 rows each); lane L -> row g*8 + L/8, LDS
  // chunk L%8 holding global chunk (L%8) ^ ((row>>1)&7)
  const int d_row = lane >> 3;
  const int d_kc = ((lane & 7) ^ ((wave & 1) * 4 + (lane >> 4))) * 8;
  // uniform tile bases plus 32-bit per-lane offsets (a tile spans < 2^31
  // elements: 256 rows of lda, ldw)
  const bf16_t* a_base = A + (int64_t)m0 * lda;
  const bf16_t* b_base = Wt + (int64_t)n0 * ldw;
  int a_off[AG], b_off[WGW];
#pragma unroll
  for (int i = 0; i < AG; ++i) {
    const int r = (wave + NW * i) * 8 + d_row;
    a_off[i] = (int)((int64_t)(min(m0 + r, M - 1) - m0) * lda) + d_kc;
    if (i < WGW) b_off[i] = (int)((int64_t)(min(n0 + r, N - 1) - n0) * ldw) + d_kc;
  }
  auto issue = [&](int stage, int k0) {
    bf16_t* base = smem + stage * kStage + wave * 8 * kBK;
#pragma unroll
    for (int i = 0; i < AG; ++i) dma16(a_base + (a_off[i] + k0), base + i * NW * 8 * kBK);
#pragma unroll
    for (int i = 0; i < WGW; ++i) dma16(b_base + (b_off[i] + k0), base + BM * kBK + i * NW * 8 * kBK);
  };

  // fragment lane l: row block_base + l%16, chunk 4*step + l/16, stored at
  // chunk ^ ((row >> 1) & 7)
  const int f_row = lane & 15, f_sw = (lane & 15) >> 1, f_q = lane >> 4;
  const int fa_row = (wm * NI * 16 + f_row) * kBK;
  const int fw_row = BM * kBK + (wn * NJ * 16 + f_row) * kBK;
  bf16x8 fa[2][NI], fw[2][NJ];
  auto load_frags = [&](int stage, int step, int buf) {
    const bf16_t* base = smem + stage * kStage + (((step * 4 + f_q) ^ f_sw) * 8);
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      fw[buf][j] = as_bf16x8(*(const u32x4*)(base + fw_row + j * 16 * kBK));
#pragma unroll
    for (int i = 0; i < NI; ++i)
      fa[buf][i] = as_bf16x8(*(const u32x4*)(base + fa_row + i * 16 * kBK));
  };
  f32x4 acc[NI][NJ];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{};
  // MFMAs of A blocks [i0, i1)
  auto mfma_rows = [&](int buf, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = mfma16x16x32(fw[buf][j], fa[buf][i], acc[i][j]);
  };

  // past the last tile the loads re-fetch it, which keeps every iteration's
  // wait the same
  const int KT = K / kBK;
  issue(0, 0);
  issue(1, min(1, KT - 1) * kBK);
  __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(kLoads));   // tile 0 landed
  ring_barrier();
  load_frags(0, 0, 0);
  for (int kt = 0; kt < KT; ++kt) {
    __builtin_amdgcn_sched_barrier(0);
    const int stage = kt & 1;
    const int k2 = min(kt + 2, KT - 1) * kBK;
    load_frags(stage, 1, 1);
    mfma_rows(0, 0, NI);
    interleave_x16<NM, NR, 0>();
    // tile kt + 1 landed; every wave is done reading this stage (its step-1
    // fragments are in registers)
    __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));
    ring_barrier();
    // the half step that issues the loads runs at raised wave priority (see
    // the comment above the kernel)
    __builtin_amdgcn_s_setprio(1);
    load_frags(stage ^ 1, 0, 0);
    issue(stage, k2);
    mfma_rows(1, 0, NI);
    interleave_x16<NM, NR, kLoads>();
    __builtin_amdgcn_s_setprio(0);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int col0 = EPI == KAD_EPI_SWIGLU ? (n0 + wn * NJ * 16) / 2 : n0 + wn * NJ * 16;
  epilogue_x16<EPI, NI, NJ>(acc, smem + wave * TX::EpiWave, lane, m0 + wm * NI * 16, col0, C,
                            ldc, R, ldr, M, N);
}

template <int EPI, class TX>
int launch_x16(const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
               const void* R, int64_t ldr, int M, int N, int K, hipStream_t s) {
  const int64_t nblocks = kad_cdiv(M, TX::BM) * kad_cdiv(N, TX::BN);
  if (nblocks > 0x7fffffff) KAD_UNSUPPORTED("gemm grid too large");
  if ((int64_t)TX::BM * (lda > ldw ? lda : ldw) + K >= 0x7fffffff)
    KAD_UNSUPPORTED("gemm rows too long for 32-bit tile offsets");
  const int n_major = (int64_t)N >= (int64_t)M ? 1 : 0;
  hipLaunchKernelGGL((gemm_x16_kernel<EPI, TX>), dim3((unsigned)nblocks), dim3(64 * TX::NW), 0, s,
                     (const bf16_t*)A, lda, (const bf16_t*)W, ldw, (bf16_t*)C, ldc,
                     (const bf16_t*)R, ldr, M, N, K, n_major, 8);
  return kad_launch_status("gemm_x16_kernel");
}

// 256 x 256 tiles as gemm_x16_kernel, but the operand that streams from
// beyond the L2 gets three LDS slots of 64-deep K and the other two (160 KB):
// the streamed operand's tile kt + 3 goes out when tile kt's slot frees, so
// its loads have two tiles of time to land instead of one.  Which operand
// streams follows the tile order: A (the activations) for M-major orders,
// where an XCD keeps its W panels in L2 across rounds and fetches new A
// panels each round; W for N-major ones.  The prefill's long-K projections
// (K = 3,584), whose loads wait 600-800 cycles per tile at the barrier with
// two slots, run 10% faster; at K = 1,024 the per-tile prologue (one
// workgroup per CU: nothing overlaps it) eats the gain.
template <int EPI, class TX, bool STREAM_A>
__global__ __launch_bounds__(64 * TX::NW) void gemm_s3_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ Wt, int64_t ldw,
    bf16_t* C, int64_t ldc, const bf16_t* R, int64_t ldr, int M, int N, int K, int n_major,
    int group) {
  constexpr int BM = TX::BM, BN = TX::BN;
  constexpr int NW = TX::NW, WN = TX::WN, NI = TX::NI, NJ = TX::NJ;
  constexpr int AG = TX::AG, WGW = TX::WGW;
  constexpr int SA = STREAM_A ? 3 : 2, SW = STREAM_A ? 2 : 3;
  constexpr int kASlot = BM * kBK, kWSlot = BN * kBK;
  constexpr int kStages = SA * kASlot + SW * kWSlot;
  constexpr int kSmem = kStages > NW * TX::EpiWave ? kStages : NW * TX::EpiWave;
  constexpr int n3 = STREAM_A ? AG : WGW;   // loads of the 3-slot operand per wave per tile
  constexpr int n2 = STREAM_A ? WGW : AG;
  constexpr int kLoads = AG + WGW;
  constexpr int NM = NI * NJ, NR = NI + NJ;
  __shared__ __attribute__((aligned(1024))) bf16_t smem[kSmem];
  bf16_t* a_lds = smem;
  bf16_t* w_lds = smem + SA * kASlot;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int m0, n0;
  tile_origin(M, N, BM, BN, n_major, group, m0, n0);

  const int d_row = lane >> 3;
  const int d_kc = ((lane & 7) ^ ((wave & 1) * 4 + (lane >> 4))) * 8;
  const bf16_t* a_base = A + (int64_t)m0 * lda;
  const bf16_t* b_base = Wt + (int64_t)n0 * ldw;
  int a_off[AG], b_off[WGW];
#pragma unroll
  for (int i = 0; i < AG; ++i) {
    const int r = (wave + NW * i) * 8 + d_row;
    a_off[i] = (int)((int64_t)(min(m0 + r, M - 1) - m0) * lda) + d_kc;
  }
#pragma unroll
  for (int i = 0; i < WGW; ++i) {
    const int r = (wave + NW * i) * 8 + d_row;
    b_off[i] = (int)((int64_t)(min(n0 + r, N - 1) - n0) * ldw) + d_kc;
  }
  const int KT = K / kBK;
  auto issue_a = [&](int t) {
    const int k0 = min(t, KT - 1) * kBK;
    bf16_t* base = a_lds + (t % SA) * kASlot + wave * 8 * kBK;
#pragma unroll
    for (int i = 0; i < AG; ++i) dma16(a_base + (a_off[i] + k0), base + i * NW * 8 * kBK);
  };
  auto issue_w = [&](int t) {
    const int k0 = min(t, KT - 1) * kBK;
    bf16_t* base = w_lds + (t % SW) * kWSlot + wave * 8 * kBK;
#pragma unroll
    for (int i = 0; i < WGW; ++i) dma16(b_base + (b_off[i] + k0), base + i * NW * 8 * kBK);
  };
  // the 2-slot operand's loads go out before the 3-slot one's, so that
  // vmcnt(n3) at a barrier leaves only the newest 3-slot loads in flight
  auto issue2 = [&](int t) { if (STREAM_A) issue_w(t); else issue_a(t); };
  auto issue3 = [&](int t) { if (STREAM_A) issue_a(t); else issue_w(t); };

  const int f_row = lane & 15, f_sw = (lane & 15) >> 1, f_q = lane >> 4;
  const int fa_row = (wm * NI * 16 + f_row) * kBK;
  const int fw_row = (wn * NJ * 16 + f_row) * kBK;
  bf16x8 fa[2][NI], fw[2][NJ];
  auto load_frags = [&](int t, int step, int buf) {
    const int ch = ((step * 4 + f_q) ^ f_sw) * 8;
    const bf16_t* ab = a_lds + (t % SA) * kASlot + ch;
    const bf16_t* wb = w_lds + (t % SW) * kWSlot + ch;
#pragma unroll
    for (int j = 0; j < NJ; ++j) fw[buf][j] = as_bf16x8(*(const u32x4*)(wb + fw_row + j * 16 * kBK));
#pragma unroll
    for (int i = 0; i < NI; ++i) fa[buf][i] = as_bf16x8(*(const u32x4*)(ab + fa_row + i * 16 * kBK));
  };
  f32x4 acc[NI][NJ];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{};
  auto mfma_rows = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = mfma16x16x32(fw[buf][j], fa[buf][i], acc[i][j]);
  };

  issue2(0);
  issue3(0);
  issue2(1);
  issue3(1);
  issue3(2);
  __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(n2 + 2 * n3));   // tile 0 landed
  ring_barrier();
  load_frags(0, 0, 0);
  for (int kt = 0; kt < KT; ++kt) {
    __builtin_amdgcn_sched_barrier(0);
    load_frags(kt, 1, 1);
    mfma_rows(0);
    interleave_x16<NM, NR, 0>();
    // tile kt + 1 landed (the 3-slot operand's tile kt + 2 may still be in
    // flight); every wave is done reading tile kt's slots
    __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(n3));
    ring_barrier();
    __builtin_amdgcn_s_setprio(1);
    load_frags(kt + 1, 0, 0);
    issue2(kt + 2);
    issue3(kt + 3);
    mfma_rows(1);
    interleave_x16<NM, NR, kLoads>();
    __builtin_amdgcn_s_setprio(0);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int col0 = EPI == KAD_EPI_SWIGLU ? (n0 + wn * NJ * 16) / 2 : n0 + wn * NJ * 16;
  epilogue_x16<EPI, NI, NJ>(acc, smem + wave * TX::EpiWave, lane, m0 + wm * NI * 16, col0, C,
                            ldc, R, ldr, M, N);
}

template <int EPI, class TX>
int launch_s3(const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
              const void* R, int64_t ldr, int M, int N, int K, hipStream_t s) {
  const int64_t nblocks = kad_cdiv(M, TX::BM) * kad_cdiv(N, TX::BN);
  if (nblocks > 0x7fffffff) KAD_UNSUPPORTED("gemm grid too large");
  if ((int64_t)TX::BM * (lda > ldw ? lda : ldw) + K >= 0x7fffffff)
    KAD_UNSUPPORTED("gemm rows too long for 32-bit tile offsets");
  const int n_major = (int64_t)N >= (int64_t)M ? 1 : 0;
  if (n_major)
    hipLaunchKernelGGL((gemm_s3_kernel<EPI, TX, false>), dim3((unsigned)nblocks), dim3(64 * TX::NW),
                       0, s, (const bf16_t*)A, lda, (const bf16_t*)W, ldw, (bf16_t*)C, ldc,
                       (const bf16_t*)R, ldr, M, N, K, n_major, 8);
  else
    hipLaunchKernelGGL((gemm_s3_kernel<EPI, TX, true>), dim3((unsigned)nblocks), dim3(64 * TX::NW),
                       0, s, (const bf16_t*)A, lda, (const bf16_t*)W, ldw, (bf16_t*)C, ldc,
                       (const bf16_t*)R, ldr, M, N, K, n_major, 8);
  return kad_launch_status("gemm_s3_kernel");
}

// Persistent form of the 16x16x32 kernel: one workgroup per CU walks the
// tiles v = blockIdx.x, + gridDim.x, ... (the same grouped, XCD-aware order).
// The K slices of successive tiles form one stream through the two LDS
// stages, so the last two iterations of a tile already load the first two
// slices of the next one; the epilogue then runs while those loads land
// (through a small LDS region of its own), and no workgroup is dispatched
// per tile.
// Epilogue of the persistent kernel: as epilogue_x16, staged one 16-row
// block at a time through a small wave-private LDS region (16 x (cols + 8) elements), so that every global
// store is a 16-byte piece of a full 128-byte row segment.  A wave's LDS
// accesses complete in order, so no barrier is needed.
template <int EPI, int NI, int NJ>
__device__ __forceinline__ void epilogue_x16_chunked(f32x4 (&acc)[NI][NJ], bf16_t* ep, int lane,
                                                     int row0, int col0, bf16_t* C, int64_t ldc,
                                                     const bf16_t* R, int64_t ldr, int M, int N) {
  constexpr int kCols = EPI == KAD_EPI_SWIGLU ? NJ * 8 : NJ * 16;
  constexpr int kLd = kCols + 8;
  constexpr int kChunks = kCols / 8, kRowsPer = 64 / kChunks;
  const int e_row = lane & 15, e_col = (lane >> 4) * 4;
  const int c_row = lane / kChunks, c_col = (lane % kChunks) * 8;
  const int n_out = EPI == KAD_EPI_SWIGLU ? N / 2 : N;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if constexpr (EPI == KAD_EPI_SWIGLU) {
        if ((j & 3) >= 2) continue;
        u32x2 packed;
#pragma unroll
        for (int h = 0; h < 2; ++h)
          packed[h] = swiglu2(acc[i][j][h * 2], acc[i][j][h * 2 + 1], acc[i][j + 2][h * 2],
                              acc[i][j + 2][h * 2 + 1]);
        *(u32x2*)(ep + e_row * kLd + (j >> 2) * 32 + (j & 3) * 16 + e_col) = packed;
      } else {
        u32x2 packed;
#pragma unroll
        for (int h = 0; h < 2; ++h)
          packed[h] = (uint32_t)f2bf(acc[i][j][h * 2]) | ((uint32_t)f2bf(acc[i][j][h * 2 + 1]) << 16);
        *(u32x2*)(ep + e_row * kLd + j * 16 + e_col) = packed;
      }
    }
#pragma unroll
    for (int r = c_row; r < 16; r += kRowsPer) {
      const int row = row0 + i * 16 + r, col = col0 + c_col;
      u32x4 v = *(const u32x4*)(ep + r * kLd + c_col);
      if (row >= M || col >= n_out) continue;
      if constexpr (EPI == KAD_EPI_RESIDUAL) {
        const u32x4 rr = *(const u32x4*)(R + (int64_t)row * ldr + col);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const float lo = __uint_as_float(rr[h] << 16) + __uint_as_float(v[h] << 16);
          const float hi =
              __uint_as_float(rr[h] & 0xffff0000u) + __uint_as_float(v[h] & 0xffff0000u);
          v[h] = (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
        }
      }
      *(u32x4*)(C + (int64_t)row * ldc + col) = v;
    }
  }
}

// Epilogue of the prefill's GDN input projection (kEpiConv): the columns
// below ce.cols are the depthwise causal conv's inputs (q | k | v), and the
// tile leaves them convolved (width 4, SiLU), with conv_prefill_bf16's
// arithmetic operation for operation: each 16-row block is staged in the
// wave's LDS region as bf16 (the projection's rounding), and row r of a
// wave's 128-row sub-tile (which lies inside one sequence) takes its taps from
// rows r-3 .. r-1 of the block or, across blocks, from a 3-row carry of the
// previous block.  Rows 0-2 of a sub-tile need the rows before it: they and
// rows 124-127 go raw to ce.side ([M/128][7][cols]: slots 0-2, then 3-6), and
// conv_fixup_kernel finishes rows 0-2 and the decode's conv state.  Columns
// from ce.cols on are stored plain.
struct ConvEpi {
  const bf16_t* w;   // [cols, 4] conv weights
  bf16_t* side;      // [M / 128][7][cols] raw rows 0-2 and 124-127 of every sub-tile
  int cols;
};
constexpr int kEpiConv = 3;   // internal epilogue code (not part of the C ABI)

template <int NI, int NJ>
__device__ __forceinline__ void epilogue_conv_chunked(f32x4 (&acc)[NI][NJ], bf16_t* ep,
                                                      bf16_t* carry, int lane, int row0,
                                                      int col0, bf16_t* C, int64_t ldc,
                                                      const ConvEpi& ce) {
  static_assert(NI * 16 == 128 && NJ * 16 == 64, "128 x 64 wave sub-tiles");
  constexpr int kCols = NJ * 16, kLd = kCols + 8;
  const int e_row = lane & 15, e_col = (lane >> 4) * 4;
  // 4 channels x 4 consecutive rows per lane (rows 4 rg .. 4 rg + 3 of a
  // block, channels col0 + c_col .. + 3): the 7 input rows of its window are
  // read and widened once
  const int rg = lane >> 4, c_col = (lane & 15) * 4;
  // this lane's 4 channels' taps, packed: word j of wpk[h] holds channel
  // 2h + j/2, taps 2 (j%2) and 2 (j%2) + 1
  u32x4 wpk[2];
  {
    const u32x4* wp = (const u32x4*)(ce.w + (int64_t)(col0 + c_col) * 4);
    wpk[0] = wp[0];
    wpk[1] = wp[1];
  }
  auto wtap = [&](int ch, int d) {
    const int flat = ch * 4 + d;
    const uint32_t word = wpk[flat / 8][(flat % 8) / 2];
    return __uint_as_float((flat & 1) ? (word & 0xffff0000u) : (word << 16));
  };
  bf16_t* side = ce.side + (int64_t)(row0 / 128) * 7 * ce.cols + col0 + c_col;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      u32x2 packed;
#pragma unroll
      for (int h = 0; h < 2; ++h)
        packed[h] = (uint32_t)f2bf(acc[i][j][h * 2]) | ((uint32_t)f2bf(acc[i][j][h * 2 + 1]) << 16);
      *(u32x2*)(ep + e_row * kLd + j * 16 + e_col) = packed;
    }
    // window rows 4 rg - 3 .. 4 rg + 3 (negative: the carry of the block before)
    u32x2 xw[7];
#pragma unroll
    for (int d = 0; d < 7; ++d) {
      const int src = rg * 4 - 3 + d;
      xw[d] = src >= 0 ? *(const u32x2*)(ep + src * kLd + c_col)
                       : *(const u32x2*)(carry + (src + 3) * kLd + c_col);
    }
    if (i == 0 && rg == 0) {
#pragma unroll
      for (int r = 0; r < 3; ++r) *(u32x2*)(side + (int64_t)r * ce.cols) = xw[3 + r];
    }
    if (i == NI - 1 && rg == 3) {
#pragma unroll
      for (int r = 0; r < 4; ++r) *(u32x2*)(side + (int64_t)(3 + r) * ce.cols) = xw[3 + r];
    }
    u32x2 o[4];
#pragma unroll
    for (int e = 0; e < 2; ++e) {   // channel pair 2e, 2e + 1
      float xf[2][7];
#pragma unroll
      for (int d = 0; d < 7; ++d) {
        xf[0][d] = __uint_as_float(xw[d][e] << 16);
        xf[1][d] = __uint_as_float(xw[d][e] & 0xffff0000u);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {   // row 4 rg + q: inputs xf[.][q .. q + 3]
        float a[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          float sacc = 0.f;
#pragma unroll
          for (int d = 0; d < 4; ++d) sacc += wtap(e * 2 + hh, d) * xf[hh][q + d];
          a[hh] = sacc;
        }
        const uint32_t pk = pack_bf16x2(a[0], a[1]);
        o[q][e] = pack_bf16x2(silu_fast(__uint_as_float(pk << 16)),
                              silu_fast(__uint_as_float(pk & 0xffff0000u)));
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = rg * 4 + q;
      if (i == 0 && r < 3) continue;   // finished by conv_fixup_kernel
      *(u32x2*)(C + (int64_t)(row0 + i * 16 + r) * ldc + col0 + c_col) = o[q];
    }
    // rows 13-15 of the block carry into the next (a wave's LDS accesses
    // complete in order, so the block's reads above are done first)
    if (lane < 48) {
      const int cr = lane >> 4, cc = (lane & 15) * 4;
      *(u32x2*)(carry + cr * kLd + cc) = *(const u32x2*)(ep + (13 + cr) * kLd + cc);
    }
  }
}

// Rows 0-2 of every 128-row sub-tile of the fused conv projection (their
// taps are rows 125-127 of the sub-tile before, zeros at a sequence start),
// with conv_prefill_bf16's arithmetic, and the decode's conv state: the last
// 4 inputs of each sequence, [B, cols, 4].  One thread per (sub-tile, 8
// channels).
__global__ __launch_bounds__(256) void conv_fixup_kernel(const bf16_t* __restrict__ side,
                                                         const bf16_t* __restrict__ w,
                                                         bf16_t* __restrict__ C, int64_t ldc,
                                                         bf16_t* __restrict__ state, int nsub,
                                                         int sub_per_seq, int cols) {
  const int C8 = cols / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)nsub * C8) return;
  const int c0 = (int)(idx % C8) * 8;
  const int sb = (int)(idx / C8);
  float wt[8][4];
  {
    const u32x4* wp = (const u32x4*)(w + (int64_t)c0 * 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 r = wp[j];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int flat = j * 8 + e * 2;
        wt[flat / 4][flat % 4] = __uint_as_float(r[e] << 16);
        wt[(flat + 1) / 4][(flat + 1) % 4] = __uint_as_float(r[e] & 0xffff0000u);
      }
    }
  }
  // xv[0..2]: the taps (rows 125-127 before), xv[3..5]: rows 0-2
  u32x4 xv[6];
  const bool seq_start = sb % sub_per_seq == 0;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    xv[k] = seq_start ? u32x4{0u, 0u, 0u, 0u}
                      : *(const u32x4*)(side + ((int64_t)(sb - 1) * 7 + 4 + k) * cols + c0);
    xv[3 + k] = *(const u32x4*)(side + ((int64_t)sb * 7 + k) * cols + c0);
  }
#pragma unroll
  for (int t = 0; t < 3; ++t) {
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float a[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int ch = e * 2 + hh;
        float sacc = 0.f;
#pragma unroll
        for (int d = 0; d < 4; ++d)
          sacc += wt[ch][d] *
                  __uint_as_float(hh ? (xv[t + d][e] & 0xffff0000u) : (xv[t + d][e] << 16));
        a[hh] = sacc;
      }
      const uint32_t pk = pack_bf16x2(a[0], a[1]);
      o[e] = pack_bf16x2(silu_fast(__uint_as_float(pk << 16)),
                         silu_fast(__uint_as_float(pk & 0xffff0000u)));
    }
    *(u32x4*)(C + ((int64_t)sb * 128 + t) * ldc + c0) = o;
  }
  if (state && sb % sub_per_seq == sub_per_seq - 1) {
    const int64_t b = sb / sub_per_seq;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const u32x4 r = *(const u32x4*)(side + ((int64_t)sb * 7 + 3 + j) * cols + c0);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        state[(b * cols + c0 + 2 * e) * 4 + j] = (bf16_t)(r[e] & 0xffffu);
        state[(b * cols + c0 + 2 * e + 1) * 4 + j] = (bf16_t)(r[e] >> 16);
      }
    }
  }
}

template <int EPI, int BN>
__global__ __launch_bounds__(512, 1) void gemm_x16p_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ Wt, int64_t ldw,
    bf16_t* C, int64_t ldc, const bf16_t* R, int64_t ldr, int M, int N, int K, int n_major,
    int group, int ntiles) {
  using TX = TileX16<256, BN, 2, 4>;
  constexpr int NW = TX::NW, WN = TX::WN, NI = TX::NI, NJ = TX::NJ;
  constexpr int kStage = TX::Stage, AG = TX::AG, WGW = TX::WGW;
  constexpr int kLoads = AG + WGW;
  constexpr int NM = NI * NJ, NR = NI + NJ;
  constexpr int kEpiChunk = 16 * ((EPI == KAD_EPI_SWIGLU ? NJ * 8 : NJ * 16) + 8);
  __shared__ __attribute__((aligned(1024))) bf16_t smem[2 * kStage + NW * kEpiChunk];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int KT = K / kBK;
  // this workgroup's tiles: v = blockIdx.x + r * gridDim.x, r < my_tiles
  const int my_tiles = (ntiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  const int my_slices = my_tiles * KT;
  auto origin = [&](int r, int& m0, int& n0) {
    const int v = (int)blockIdx.x + r * (int)gridDim.x;
    tile_origin_of(xcd_logical_id(v, ntiles), M, N, kT, BN, n_major, group, m0, n0);
  };

  // DMA rows: groups g = wave + 8 i (8 rows each); lane L -> row g*8 + L/8,
  // LDS chunk L%8 holding global chunk (L%8) ^ ((row>>1)&7)
  const int d_row = lane >> 3;
  const int d_kc = ((lane & 7) ^ ((wave & 1) * 4 + (lane >> 4))) * 8;
  // load cursor: tile ld_r, slice ld_k of it; it stops at the last slice of
  // the last tile (the loads then re-fetch it, which keeps the wait counts
  // uniform)
  int ld_r = 0, ld_k = 0, ld_g = 0;
  const bf16_t* ld_a = A;
  const bf16_t* ld_b = Wt;
  int ld_amax = 0, ld_bmax = 0;
  auto set_tile = [&](int r) {
    int m0, n0;
    origin(r, m0, n0);
    ld_a = A + (int64_t)m0 * lda + d_kc;
    ld_b = Wt + (int64_t)n0 * ldw + d_kc;
    ld_amax = M - 1 - m0;
    ld_bmax = N - 1 - n0;
  };
  auto issue = [&](int slot) {
    bf16_t* base = smem + (slot & 1) * kStage + wave * 8 * kBK;
    const int k0 = ld_k * kBK;
#pragma unroll
    for (int i = 0; i < AG; ++i) {
      const int rr = min((wave + NW * i) * 8 + d_row, ld_amax);
      dma16(ld_a + (int64_t)rr * lda + k0, base + i * NW * 8 * kBK);
    }
#pragma unroll
    for (int i = 0; i < WGW; ++i) {
      const int rr = min((wave + NW * i) * 8 + d_row, ld_bmax);
      dma16(ld_b + (int64_t)rr * ldw + k0, base + kT * kBK + i * NW * 8 * kBK);
    }
  };
  auto advance = [&]() {
    if (++ld_g < my_slices) {
      if (++ld_k == KT) {
        ld_k = 0;
        set_tile(++ld_r);
      }
    }
  };

  const int f_row = lane & 15, f_sw = (lane & 15) >> 1, f_q = lane >> 4;
  const int fa_row = (wm * NI * 16 + f_row) * kBK;
  const int fw_row = kT * kBK + (wn * NJ * 16 + f_row) * kBK;
  bf16x8 fa[2][NI], fw[2][NJ];
  auto load_frags = [&](int stage, int step, int buf) {
    const bf16_t* base = smem + stage * kStage + (((step * 4 + f_q) ^ f_sw) * 8);
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      fw[buf][j] = as_bf16x8(*(const u32x4*)(base + fw_row + j * 16 * kBK));
#pragma unroll
    for (int i = 0; i < NI; ++i)
      fa[buf][i] = as_bf16x8(*(const u32x4*)(base + fa_row + i * 16 * kBK));
  };
  f32x4 acc[NI][NJ];
  auto mfma_rows = [&](int buf, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = mfma16x16x32(fw[buf][j], fa[buf][i], acc[i][j]);
  };

  if (my_tiles <= 0) return;
  set_tile(0);
  issue(0);
  advance();
  issue(1);
  advance();
  __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(kLoads));   // slice 0 landed
  ring_barrier();
  load_frags(0, 0, 0);
  for (int r = 0; r < my_tiles; ++r) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{};
    const int g0 = r * KT;
    for (int kt = 0; kt < KT; ++kt) {
      __builtin_amdgcn_sched_barrier(0);
      const int g = g0 + kt, stage = g & 1;
      load_frags(stage, 1, 1);
      mfma_rows(0, 0, NI);
      interleave_x16<NM, NR, 0>();
      // slice g + 1 landed; every wave is done reading this stage (its step-1
      // fragments are in registers)
      __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));
      ring_barrier();
      __builtin_amdgcn_s_setprio(1);
      load_frags(stage ^ 1, 0, 0);
      issue(g + 2);
      mfma_rows(1, 0, NI);
      interleave_x16<NM, NR, kLoads>();
      __builtin_amdgcn_s_setprio(0);
      advance();
    }
    int m0, n0;
    origin(r, m0, n0);
    const int col0 = EPI == KAD_EPI_SWIGLU ? (n0 + wn * NJ * 16) / 2 : n0 + wn * NJ * 16;
    epilogue_x16_chunked<EPI, NI, NJ>(acc, smem + 2 * kStage + wave * kEpiChunk, lane,
                                      m0 + wm * NI * 16, col0, C, ldc, R, ldr, M, N);
  }
  // no LDS write may land after the workgroup ends
  __builtin_amdgcn_s_waitcnt(0);
}

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// 256 x 256 tiles, 8 waves in two groups that alternate roles ("ping-pong"),
// persistent.  Waves w and w + 4 share a SIMD; group 0 (waves 0-3) owns
// output rows 0-127 of a tile, group 1 rows 128-255, each wave a 128 x 64
// sub-tile.  Between two workgroup barriers one group issues only MFMAs
// (all 64 of a 64-deep K slice, from fragments already in registers) while
// the other does memory work: the LDS fragment reads of its next slice and
// its part of the global->LDS loads.  So each SIMD's matrix unit is fed by
// one wave at a time and no load stalls an MFMA wave's issue.
//
// Phases (each ends at a barrier): 2g: group 0 reads slice g, group 1
// computes slice g - 1; 2g + 1: group 0 computes slice g, group 1 reads
// slice g.  A stage (g % 2) may be reloaded only once every wave that reads
// the rows is done with them, which the barriers order (a wave waits for
// its own LDS reads before the barrier that ends its read phase).
//
// One workgroup per CU walks the tiles v = blockIdx.x, + gridDim.x, ... (the
// grouped, XCD-aware order); the K slices of its tiles form one stream
// through the two stages, and a group's epilogue for a tile runs in its read
// phase of the next tile's first slice (through a small LDS region of its
// own, as in gemm_x16p_kernel) while the other group's MFMAs run.  Tiles
// must be whole (M, N multiples of 256).  Every K slice accumulates in the
// order of the other configurations, so results are bit-identical to them.
// An instrumented copy (shader-clock timers at each barrier) puts a slice at
// 3,100-3,700 cycles against 2,048 of MFMA work: the read phases (24
// fragment reads per wave, 85 B/clk per CU, where an LDS microbenchmark of
// the same pattern reads 253) set the pace.
template <int EPI>
__global__ __launch_bounds__(512, 1) void gemm_ppp_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ Wt, int64_t ldw,
    bf16_t* C, int64_t ldc, const bf16_t* R, int64_t ldr, int M, int N, int K, int n_major,
    int group, int ntiles, ConvEpi ce) {
  using TX = Tile256;
  constexpr int BM = TX::BM, BN = TX::BN;
  constexpr int NW = TX::NW, WN = TX::WN, NI = TX::NI, NJ = TX::NJ;
  constexpr int kStage = TX::Stage, AG = TX::AG, WGW = TX::WGW;
  constexpr int kLoads = AG + WGW;
  constexpr int kEpiChunk = 16 * ((EPI == KAD_EPI_SWIGLU ? NJ * 8 : NJ * 16) + 8);
  constexpr int kCarry = EPI == kEpiConv ? 3 * (NJ * 16 + 8) : 0;   // per wave
  __shared__ __attribute__((aligned(1024))) bf16_t smem[2 * kStage + NW * (kEpiChunk + kCarry)];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int swave = __builtin_amdgcn_readfirstlane(wave);
  const int grp = swave / WN;
  const int wm = grp, wn = swave % WN;
  const int KT = K / kBK;
  const int my_tiles = (ntiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  if (my_tiles <= 0) return;
  const int total = my_tiles * KT;   // slices in this workgroup's stream
  auto origin = [&](int r, int& m0, int& n0) {
    const int v = (int)blockIdx.x + r * (int)gridDim.x;
    tile_origin_of(xcd_logical_id(v, ntiles), M, N, BM, BN, n_major, group, m0, n0);
  };

  // Loads.  Group 1 reads only A rows 128-255, so the A rows 0-127 of a
  // stage are free once group 0 has read them: group 1 loads those (row
  // groups w + 4i of 8 rows, w = its wave index in the group) during its own
  // read phase, two slices ahead.  Group 0 loads A rows 128-255 and every W
  // row (row groups 16 + w + 4i and w + 4i) during its read phase, one slice
  // ahead, once both groups have read the stage.  So no load is issued in an
  // MFMA phase.  A row group's swizzle phase is its parity, which is that of
  // w for all of a wave's groups.  Load cursor (per wave, uniform): every
  // wave issues its part of slices 0, 1, 2, ... in order; past the last slice
  // it re-fetches that one (uniform wait counts).
  constexpr int kL1 = 4, kL0 = 12;   // loads per slice of a group-1 / group-0 wave
  const int gw = swave & 3;
  const int l_row = lane >> 3;
  const int l_kc = ((lane & 7) ^ ((gw & 1) * 4 + (lane >> 4))) * 8;
  const uint32_t a_lane = (uint32_t)(l_row * (int)lda + l_kc) * 2u;
  const uint32_t b_lane = (uint32_t)(l_row * (int)ldw + l_kc) * 2u;
  int ld_g = 0, ld_k = 0, ld_r = 0;
  __amdgpu_buffer_rsrc_t ld_a, ld_b;
  auto set_tile = [&](int r) {
    int m0, n0;
    origin(r, m0, n0);
    ld_a = buffer_rsrc(A + (int64_t)m0 * lda);
    ld_b = buffer_rsrc(Wt + (int64_t)n0 * ldw);
  };
  set_tile(0);
  const uint32_t a_rg = (uint32_t)(8 * lda * 2), b_rg = (uint32_t)(8 * ldw * 2);  // bytes per row group
  auto issue_loads = [&]() {
    const uint32_t k0 = (uint32_t)ld_k * kBK * 2;
    bf16_t* base = smem + (ld_g & 1) * kStage;
    if (grp == 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rg = gw + 4 * i;
        dma16_buf(ld_a, a_lane, (uint32_t)rg * a_rg + k0, base + rg * 8 * kBK);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rg = 16 + gw + 4 * i;
        dma16_buf(ld_a, a_lane, (uint32_t)rg * a_rg + k0, base + rg * 8 * kBK);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int rg = gw + 4 * i;
        dma16_buf(ld_b, b_lane, (uint32_t)rg * b_rg + k0, base + BM * kBK + rg * 8 * kBK);
      }
    }
  };
  // the stage alternates with every issue; the slice stays at the stream's
  // last one once reached
  auto advance = [&]() {
    ++ld_g;
    if (ld_r * KT + ld_k + 1 < total) {
      if (++ld_k == KT) {
        ld_k = 0;
        set_tile(++ld_r);
      }
    }
  };
  auto issue = [&]() {
    issue_loads();
    advance();
  };

  const int f_row = lane & 15, f_sw = (lane & 15) >> 1, f_q = lane >> 4;
  const int fa_row = (wm * NI * 16 + f_row) * kBK;
  const int fw_row = BM * kBK + (wn * NJ * 16 + f_row) * kBK;
  bf16x8 fa[2][NI], fw[2][NJ];
  auto read_slice = [&](int g) {
#pragma unroll
    for (int step = 0; step < 2; ++step) {
      const bf16_t* base = smem + (g & 1) * kStage + (((step * 4 + f_q) ^ f_sw) * 8);
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        fw[step][j] = as_bf16x8(*(const u32x4*)(base + fw_row + j * 16 * kBK));
#pragma unroll
      for (int i = 0; i < NI; ++i)
        fa[step][i] = as_bf16x8(*(const u32x4*)(base + fa_row + i * 16 * kBK));
    }
  };
  f32x4 acc[NI][NJ];
  auto zero = [&]() {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{};
  };
  auto compute = [&]() {
#pragma unroll
    for (int step = 0; step < 2; ++step)
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = mfma16x16x32(fw[step][j], fa[step][i], acc[i][j]);
  };
  bf16_t* ep = smem + 2 * kStage + swave * kEpiChunk;
  auto epilogue = [&](int r) {
    int m0, n0;
    origin(r, m0, n0);
    const int col0 = EPI == KAD_EPI_SWIGLU ? (n0 + wn * NJ * 16) / 2 : n0 + wn * NJ * 16;
    if constexpr (EPI == kEpiConv) {
      if (n0 < ce.cols)
        epilogue_conv_chunked<NI, NJ>(acc, ep, smem + 2 * kStage + NW * kEpiChunk + swave * kCarry,
                                      lane, m0 + wm * NI * 16, col0, C, ldc, ce);
      else
        epilogue_x16_chunked<KAD_EPI_STORE, NI, NJ>(acc, ep, lane, m0 + wm * NI * 16, col0, C,
                                                    ldc, R, ldr, M, N);
    } else {
      epilogue_x16_chunked<EPI, NI, NJ>(acc, ep, lane, m0 + wm * NI * 16, col0, C, ldc, R, ldr,
                                        M, N);
    }
  };

  zero();
  issue();
  issue();
  if (grp == 0)
    __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(kL0));   // own part of slice 0 landed
  else
    __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(kL1));
  ring_barrier();
  if (grp == 0) {
    for (int g = 0; g < total; ++g) {
      __builtin_amdgcn_sched_barrier(0);
      // phase 2g: the previous tile's epilogue when g starts a tile, the
      // fragments of slice g, this wave's part of slice g + 1 (its stage was
      // last read in phase 2g - 1)
      const int kt = g % KT;
      if (kt == 0 && g > 0) {
        epilogue(g / KT - 1);
        zero();
        // the conv epilogue needs the registers that the next slice's
        // fragments would hold if their reads were hoisted above it
        if constexpr (EPI == kEpiConv) __builtin_amdgcn_sched_barrier(0);
      }
      read_slice(g);
      if (g >= 1) issue();
      __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(63));   // this wave's LDS accesses done
      __builtin_amdgcn_sched_barrier(0);
      ring_barrier();
      // phase 2g + 1: compute slice g, then wait for this wave's part of
      // slice g + 1
      compute();
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));
      ring_barrier();
    }
  } else {
    // phase 2g: compute slice g - 1; phase 2g + 1: the previous tile's
    // epilogue when g starts a tile, the fragments of slice g, this wave's
    // part of slice g + 2 (A rows that only group 0 reads, and it has), and
    // the wait for its part of slice g + 1
    auto read_phase = [&](int g) {
      const int kt = g % KT;
      if (kt == 0 && g > 0) {
        // the epilogue's stores are not ordered with the loads that the
        // counted wait below expects: drain the loads first
        __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));
        epilogue(g / KT - 1);
        zero();
        if constexpr (EPI == kEpiConv) __builtin_amdgcn_sched_barrier(0);
      }
      issue();
      read_slice(g);
      __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(kL1));
      __builtin_amdgcn_sched_barrier(0);
      ring_barrier();
    };
    ring_barrier();
    read_phase(0);
    for (int g = 1; g < total; ++g) {
      __builtin_amdgcn_sched_barrier(0);
      compute();
      __builtin_amdgcn_sched_barrier(0);
      ring_barrier();
      read_phase(g);
    }
    compute();
  }
  epilogue(my_tiles - 1);
  // no LDS write may land after the workgroup ends
  __builtin_amdgcn_s_waitcnt(0);
}

template <int EPI>
int launch_ppp(const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
               const void* R, int64_t ldr, int M, int N, int K, hipStream_t s,
               const ConvEpi& ce = ConvEpi{}) {
  const int64_t ntiles = kad_cdiv(M, 256) * kad_cdiv(N, 256);
  if (ntiles > 0x7fffffff / 2 || ntiles * (K / kBK) > 0x7fffffff)
    KAD_UNSUPPORTED("gemm grid too large");
  if ((int64_t)256 * (lda > ldw ? lda : ldw) + K >= 0x7fffffff)
    KAD_UNSUPPORTED("gemm rows too long for 32-bit tile offsets");
  if (M % 256 || N % 256) KAD_UNSUPPORTED("tile configuration 22 needs M and N multiples of 256");
  int grid = device_cu_count();
  grid -= grid % 8;
  if (grid <= 0) grid = 8;
  if (ntiles < grid) grid = (int)ntiles;
  const int n_major = (int64_t)N >= (int64_t)M ? 1 : 0;
  hipLaunchKernelGGL((gemm_ppp_kernel<EPI>), dim3((unsigned)grid), dim3(512), 0, s,
                     (const bf16_t*)A, lda, (const bf16_t*)W, ldw, (bf16_t*)C, ldc,
                     (const bf16_t*)R, ldr, M, N, K, n_major, 8, (int)ntiles, ce);
  return kad_launch_status("gemm_ppp_kernel");
}

// issue order of a first step that stores the previous tile, NB rows of 8
// blocks: per MFMA the staging of its block (4 accumulator reads, 2 packed
// conversions, one 8-byte LDS write), after each row its 4 staged 16-byte
// reads and stores; the first NR MFMAs each followed by one fragment read,
// the NV global loads spread over the others
template <int NB, int NR, int NV>
__device__ __forceinline__ void interleave_store_step() {
  constexpr int NM = NB * 8;
#pragma unroll
  for (int t = 0; t < NM; ++t) {
    __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
    __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (t < NR) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    } else if constexpr (NV > 0) {
      constexpr int kSlots = NM > NR ? NM - NR : 1;
      const int c = ((t - NR + 1) * NV) / kSlots - ((t - NR) * NV) / kSlots;
#pragma unroll
      for (int q = 0; q < c; ++q) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
    if (t % 8 == 7) {
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
      __builtin_amdgcn_sched_group_barrier(0x040, 4, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

// 256 x 256 tiles with 4 waves, one per SIMD, each owning a 128 x 128
// sub-tile: 256 fp32 accumulators per lane, which the compiler keeps in
// AGPRs (a wave alone on its SIMD may hold 512 registers).  Per 64-deep
// slice a wave reads 32 KB of fragments from LDS, so the CU reads 128 KB per
// slice where the 8-wave tiles read 192 KB, and no second wave competes for
// the SIMD's issue slots.  Persistent (one workgroup per CU walks the
// grouped, XCD-aware tile order); the K slices of successive tiles form one
// load stream through two 64-deep LDS stages, as in gemm_x16p_kernel.  Two
// 32-deep steps per slice: the MFMAs of step 0 run with the fragment reads of
// step 1, those of step 1 with the next slice's step-0 reads and this wave's
// loads of the slice after next; one barrier per slice, between the steps.
//
// Epilogue: straight from the accumulators to global memory, each lane's 4
// consecutive columns of a 16 x 16 block as one 8-byte buffer store (the L2
// merges a row's pieces before they reach HBM).  For plain stores it runs
// inside the first MFMA step of the next tile: each block is converted and
// stored just before the step's MFMA that restarts it from zero, so the
// matrix unit never waits for an epilogue.  The residual and SwiGLU
// epilogues run after the tile's last slice, while the loads of the next
// tile's first two slices land.  Tiles must be whole (M, N multiples of 256).
// Every K slice accumulates in the order of the other configurations, so
// results are bit-identical to them.
template <int EPI>
__global__ __launch_bounds__(256, 1) void gemm_w4e_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ Wt, int64_t ldw,
    bf16_t* C, int64_t ldc, const bf16_t* R, int64_t ldr, int M, int N, int K, int n_major,
    int group, int ntiles) {
  using TX = TileX16<256, 256, 2, 2>;
  constexpr int BM = TX::BM, BN = TX::BN;
  constexpr int NW = TX::NW, WN = TX::WN, NI = TX::NI, NJ = TX::NJ;
  constexpr int kStage = TX::Stage;
  constexpr int kLoads = (BM + BN) / 8 / NW;   // 1 KB row-group loads per wave per slice
  constexpr int NM = NI * NJ, NR = NI + NJ;
  // plain-store and residual epilogues stage a 16-row block of the wave's
  // sub-tile through LDS (rows of 128 columns + 8 padding, so that both the
  // 8-byte writes of the accumulator layout and the 16-byte row reads are
  // free of bank conflicts): every store then writes 4 whole 256-byte rows
  constexpr int kStgLd = NJ * 16 + 8;
  constexpr int kStg = EPI == KAD_EPI_SWIGLU ? 0 : 16 * kStgLd;
  __shared__ __attribute__((aligned(1024))) bf16_t smem[2 * kStage + NW * kStg];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int swave = __builtin_amdgcn_readfirstlane(wave);
  const int wm = swave / WN, wn = swave % WN;
  const int KT = K / kBK;
  const int my_tiles = (ntiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;
  if (my_tiles <= 0) return;
  const int total = my_tiles * KT;
  auto origin = [&](int r, int& m0, int& n0) {
    const int v = (int)blockIdx.x + r * (int)gridDim.x;
    tile_origin_of(xcd_logical_id(v, ntiles), M, N, BM, BN, n_major, group, m0, n0);
  };

  // loads: wave w takes A and W row groups w + 4i (8 rows each), whose
  // swizzle phase (the group's parity) is that of w
  const int l_row = lane >> 3;
  const int l_kc = ((lane & 7) ^ ((swave & 1) * 4 + (lane >> 4))) * 8;
  const uint32_t a_lane = (uint32_t)(l_row * (int)lda + l_kc) * 2u;
  const uint32_t b_lane = (uint32_t)(l_row * (int)ldw + l_kc) * 2u;
  const uint32_t a_rg = (uint32_t)(8 * lda * 2), b_rg = (uint32_t)(8 * ldw * 2);
  int ld_g = 0, ld_k = 0, ld_r = 0;
  __amdgpu_buffer_rsrc_t ld_a, ld_b;
  auto set_tile = [&](int r) {
    int m0, n0;
    origin(r, m0, n0);
    ld_a = buffer_rsrc(A + (int64_t)m0 * lda);
    ld_b = buffer_rsrc(Wt + (int64_t)n0 * ldw);
  };
  set_tile(0);
  // a slice's loads in two halves: its A rows, then its W rows
  auto issue_a = [&]() {
    const uint32_t k0 = (uint32_t)ld_k * kBK * 2;
    bf16_t* base = smem + (ld_g & 1) * kStage;
#pragma unroll
    for (int i = 0; i < BM / 8 / NW; ++i) {
      const int rg = swave + NW * i;
      dma16_buf(ld_a, a_lane, (uint32_t)rg * a_rg + k0, base + rg * 8 * kBK);
    }
  };
  auto issue_b = [&]() {
    const uint32_t k0 = (uint32_t)ld_k * kBK * 2;
    bf16_t* base = smem + (ld_g & 1) * kStage;
#pragma unroll
    for (int i = 0; i < BN / 8 / NW; ++i) {
      const int rg = swave + NW * i;
      dma16_buf(ld_b, b_lane, (uint32_t)rg * b_rg + k0, base + BM * kBK + rg * 8 * kBK);
    }
  };
  constexpr int kHalf = BM / 8 / NW;   // loads per half slice per wave
  static_assert(BN / 8 / NW == kHalf, "both halves issue the same number of loads");
  // the stage alternates with every issue; the slice stays at the stream's
  // last one once reached (the loads then re-fetch it: uniform wait counts)
  auto advance = [&]() {
    ++ld_g;
    if (ld_r * KT + ld_k + 1 < total) {
      if (++ld_k == KT) {
        ld_k = 0;
        set_tile(++ld_r);
      }
    }
  };

  const int f_row = lane & 15, f_sw = (lane & 15) >> 1, f_q = lane >> 4;
  const int fa_row = (wm * NI * 16 + f_row) * kBK;
  const int fw_row = BM * kBK + (wn * NJ * 16 + f_row) * kBK;
  bf16x8 fa[2][NI], fw[2][NJ];
  auto load_frags = [&](int g, int step, int buf) {
    const bf16_t* base = smem + (g & 1) * kStage + (((step * 4 + f_q) ^ f_sw) * 8);
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      fw[buf][j] = as_bf16x8(*(const u32x4*)(base + fw_row + j * 16 * kBK));
#pragma unroll
    for (int i = 0; i < NI; ++i)
      fa[buf][i] = as_bf16x8(*(const u32x4*)(base + fa_row + i * 16 * kBK));
  };
  f32x4 acc[NI][NJ];
  auto mfma_rows = [&](int buf, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = mfma16x16x32(fw[buf][j], fa[buf][i], acc[i][j]);
  };
  auto mfma_first_rows = [&](int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = mfma16x16x32(fw[0][j], fa[0][i], f32x4{});
  };

  // output addressing: a buffer resource at the wave's sub-tile origin per
  // tile.  The epilogue works on pairs of 16 x 16 blocks (32 columns): two
  // lane-row swaps (permlane32, permlane16) turn each lane's 4 + 4 columns
  // into 8 consecutive ones, so lane l stores 16 bytes at row l % 16, columns
  // 8 (l / 16) .. + 7 of the pair, and each row receives 64 contiguous bytes
  // per store instruction (32 with the accumulator layout as it is).
  const uint32_t c_lane = ((uint32_t)(lane & 15) * (uint32_t)ldc + (uint32_t)(lane >> 4) * 8u) * 2u;
  const uint32_t c_row16 = (uint32_t)(16 * ldc * 2);
  auto out_rsrc = [&](int r) {
    int m0, n0;
    origin(r, m0, n0);
    const int col0 = EPI == KAD_EPI_SWIGLU ? (n0 + wn * NJ * 16) / 2 : n0 + wn * NJ * 16;
    return buffer_rsrc(C + (int64_t)(m0 + wm * NI * 16) * ldc + col0);
  };
  // x: a lane's 4 packed columns of the left block (2 words), y: of the
  // right one; returns the lane's 8 consecutive columns of the pair
  auto pair_swap = [&](uint32_t x0, uint32_t x1, uint32_t y0, uint32_t y1) {
    const auto a = __builtin_amdgcn_permlane32_swap(x0, y0, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(x1, y1, false, false);
    const auto c = __builtin_amdgcn_permlane16_swap(a[0], a[1], false, false);
    const auto d = __builtin_amdgcn_permlane16_swap(b[0], b[1], false, false);
    return u32x4{c[0], d[0], c[1], d[1]};
  };
  // staged stores: block (i, j) goes into the wave's LDS block at row
  // lane % 16, columns j * 16 + 4 (lane / 16); lane l then reads 16 bytes of
  // row l / 16 + 4k, columns 8 (l % 16) .. + 7, and stores them
  bf16_t* stg = smem + 2 * kStage + swave * kStg;
  const int stg_w = (lane & 15) * kStgLd + (lane >> 4) * 4;
  const int stg_r = (lane >> 4) * kStgLd + (lane & 15) * 8;
  const uint32_t s_lane = ((uint32_t)(lane >> 4) * (uint32_t)ldc + (uint32_t)(lane & 15) * 8u) * 2u;
  const uint32_t c_row4 = (uint32_t)(4 * ldc * 2);
  auto stage_block = [&](int i, int j) {
    const f32x4& x = acc[i][j];
    *(u32x2*)(stg + stg_w + j * 16) = u32x2{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])};
  };
  auto store_staged = [&](__amdgpu_buffer_rsrc_t rc, int i) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 v = *(const u32x4*)(stg + stg_r + q * 4 * kStgLd);
      __builtin_amdgcn_raw_buffer_store_b128(v, rc, s_lane, (uint32_t)i * c_row16 + q * c_row4, 0);
    }
  };
  // plain-store epilogue of tile r - 1 fused into tile r's first step (a
  // wave's LDS accesses complete in order, so block i + 1's writes never
  // overtake block i's reads)
  auto mfma_first_store = [&](__amdgpu_buffer_rsrc_t rc, int i0, int i1) {
#pragma unroll
    for (int i = i0; i < i1; ++i) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        stage_block(i, j);
        acc[i][j] = mfma16x16x32(fw[0][j], fa[0][i], f32x4{});
      }
      store_staged(rc, i);
    }
  };
  auto epilogue = [&](int r) {
    const __amdgpu_buffer_rsrc_t rc = out_rsrc(r);
    if constexpr (EPI == KAD_EPI_STORE) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) stage_block(i, j);
        store_staged(rc, i);
      }
    } else if constexpr (EPI == KAD_EPI_SWIGLU) {
      // blocks 4g, 4g + 1 gate and 4g + 2, 4g + 3 up of each 64-column
      // group: output blocks 2g, 2g + 1 form the pair
#pragma unroll
      for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int g = 0; g < NJ / 4; ++g) {
          uint32_t w[4];
#pragma unroll
          for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const f32x4& gv = acc[i][4 * g + b];
              const f32x4& uv = acc[i][4 * g + b + 2];
              w[b * 2 + h] = swiglu2(gv[h * 2], gv[h * 2 + 1], uv[h * 2], uv[h * 2 + 1]);
            }
          const u32x4 v = pair_swap(w[0], w[1], w[2], w[3]);
          __builtin_amdgcn_raw_buffer_store_b128(v, rc, c_lane, (uint32_t)i * c_row16 + g * 64, 0);
        }
    } else {
      int m0, n0;
      origin(r, m0, n0);
      const __amdgpu_buffer_rsrc_t rr =
          buffer_rsrc(R + (int64_t)(m0 + wm * NI * 16) * ldr + n0 + wn * NJ * 16);
      const uint32_t r_lane = ((uint32_t)(lane >> 4) * (uint32_t)ldr + (uint32_t)(lane & 15) * 8u) * 2u;
      const uint32_t r_row4 = (uint32_t)(4 * ldr * 2), r_row16 = (uint32_t)(16 * ldr * 2);
      // C = bf16(R + bf16(acc)): the residual rows of half the sub-tile in
      // flight (16-byte pieces of whole rows, as the staged stores)
#pragma unroll
      for (int ih = 0; ih < NI; ih += NI / 2) {
        u32x4 rv[NI / 2][4];
#pragma unroll
        for (int i = 0; i < NI / 2; ++i)
#pragma unroll
          for (int q = 0; q < 4; ++q)
            rv[i][q] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           rr, r_lane, (uint32_t)(ih + i) * r_row16 + q * r_row4, 0));
#pragma unroll
        for (int i = 0; i < NI / 2; ++i) {
#pragma unroll
          for (int j = 0; j < NJ; ++j) stage_block(ih + i, j);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            u32x4 v = *(const u32x4*)(stg + stg_r + q * 4 * kStgLd);
#pragma unroll
            for (int h = 0; h < 4; ++h) {
              const float lo = __uint_as_float(rv[i][q][h] << 16) + __uint_as_float(v[h] << 16);
              const float hi = __uint_as_float(rv[i][q][h] & 0xffff0000u) +
                               __uint_as_float(v[h] & 0xffff0000u);
              v[h] = pack_bf16x2(lo, hi);
            }
            __builtin_amdgcn_raw_buffer_store_b128(v, rc, s_lane,
                                                   (uint32_t)(ih + i) * c_row16 + q * c_row4, 0);
          }
        }
      }
    }
  };

  // Slice g, with two barriers: step 0's first two rows of MFMAs carry the
  // reads of step 1's fragments; once every wave's reads are done (barrier
  // 1) stage g % 2 is free, and the A rows of slice g + 2 go into it during
  // the rest of step 0; barrier 2 (after this wave's loads of slice g + 1
  // landed) makes slice g + 1 visible, and step 1 carries the reads of its
  // step-0 fragments and the W rows of slice g + 2.  So each slice's loads
  // issue over one and three quarter steps instead of one.
  constexpr int kRowsA = 2;   // MFMA rows before barrier 1
  auto mid_barrier1 = [&]() {
    __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(63));   // own fragment reads done
    ring_barrier();
  };
  auto mid_barrier2 = [&]() {
    __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(kHalf));   // own slice g + 1 landed
    ring_barrier();
  };
  auto step1 = [&](int g) {
    load_frags(g + 1, 0, 0);
    issue_b();
    mfma_rows(1, 0, NI);
    interleave_x16<NM, NR, kHalf>();
    advance();
  };

  issue_a();
  issue_b();
  advance();
  issue_a();
  issue_b();
  advance();
  __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(2 * kHalf));   // own rows of slice 0 landed
  ring_barrier();
  load_frags(0, 0, 0);
  // the first tile's fused epilogue stores go to a resource of no records
  // (buffer stores past num_records are dropped), so every tile runs the
  // same branch-free code and the accumulators keep their registers
  __amdgpu_buffer_rsrc_t rc_prev = __builtin_amdgcn_make_buffer_rsrc(C, 0, 0, 0x00020000);
  // the loads of slice 2 (A half) are issued in slice 0's step 0: the stream
  // runs one half slice ahead of the slice count below
  for (int r = 0; r < my_tiles; ++r) {
    __builtin_amdgcn_sched_barrier(0);
    // slice 0: step 0 restarts the accumulators (storing the previous tile
    // for plain stores)
    const int g0 = r * KT;
    load_frags(g0, 1, 1);
    if constexpr (EPI == KAD_EPI_STORE) {
      mfma_first_store(rc_prev, 0, kRowsA);
      interleave_store_step<kRowsA, NR, 0>();
      mid_barrier1();
      issue_a();
      mfma_first_store(rc_prev, kRowsA, NI);
      interleave_store_step<NI - kRowsA, 0, kHalf>();
      rc_prev = out_rsrc(r);
    } else {
      mfma_first_rows(0, kRowsA);
      interleave_x16<kRowsA * NJ, NR, 0>();
      mid_barrier1();
      issue_a();
      mfma_first_rows(kRowsA, NI);
      interleave_x16<(NI - kRowsA) * NJ, 0, kHalf>();
    }
    mid_barrier2();
    step1(g0);
    for (int kt = 1; kt < KT; ++kt) {
      __builtin_amdgcn_sched_barrier(0);
      const int g = g0 + kt;
      load_frags(g, 1, 1);
      mfma_rows(0, 0, kRowsA);
      interleave_x16<kRowsA * NJ, NR, 0>();
      mid_barrier1();
      issue_a();
      mfma_rows(0, kRowsA, NI);
      interleave_x16<(NI - kRowsA) * NJ, 0, kHalf>();
      mid_barrier2();
      step1(g);
    }
    if constexpr (EPI != KAD_EPI_STORE) epilogue(r);
  }
  if constexpr (EPI == KAD_EPI_STORE) epilogue(my_tiles - 1);
  // no LDS write may land after the workgroup ends
  __builtin_amdgcn_s_waitcnt(0);
}

template <int EPI>
int launch_w4e(const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
               const void* R, int64_t ldr, int M, int N, int K, hipStream_t s) {
  const int64_t ntiles = kad_cdiv(M, 256) * kad_cdiv(N, 256);
  if (ntiles > 0x7fffffff / 2 || ntiles * (K / kBK) > 0x7fffffff)
    KAD_UNSUPPORTED("gemm grid too large");
  if ((int64_t)256 * (lda > ldw ? lda : ldw) + K >= 0x7fffffff)
    KAD_UNSUPPORTED("gemm rows too long for 32-bit tile offsets");
  if ((int64_t)256 * (ldc > ldr ? ldc : ldr) >= 0x7fffffff)
    KAD_UNSUPPORTED("gemm output rows too long for 32-bit tile offsets");
  if (M % 256 || N % 256) KAD_UNSUPPORTED("tile configuration 24 needs M and N multiples of 256");
  int grid = device_cu_count();
  grid -= grid % 8;
  if (grid <= 0) grid = 8;
  if (ntiles < grid) grid = (int)ntiles;
  const int n_major = (int64_t)N >= (int64_t)M ? 1 : 0;
  hipLaunchKernelGGL((gemm_w4e_kernel<EPI>), dim3((unsigned)grid), dim3(256), 0, s,
                     (const bf16_t*)A, lda, (const bf16_t*)W, ldw, (bf16_t*)C, ldc,
                     (const bf16_t*)R, ldr, M, N, K, n_major, 8, (int)ntiles);
  return kad_launch_status("gemm_w4e_kernel");
}

template <int EPI, int BN>
int launch_x16p(const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
                const void* R, int64_t ldr, int M, int N, int K, hipStream_t s) {
  const int64_t ntiles = kad_cdiv(M, kT) * kad_cdiv(N, BN);
  if (ntiles > 0x7fffffff / 2 || ntiles * (K / kBK) > 0x7fffffff)
    KAD_UNSUPPORTED("gemm grid too large");
  // whole XCD rounds of workgroups, so that a workgroup's tiles keep one XCD
  int grid = device_cu_count();
  grid -= grid % 8;
  if (grid <= 0) grid = 8;
  if (ntiles < grid) grid = (int)ntiles;
  const int n_major = (int64_t)N >= (int64_t)M ? 1 : 0;
  hipLaunchKernelGGL((gemm_x16p_kernel<EPI, BN>), dim3((unsigned)grid), dim3(512), 0, s,
                     (const bf16_t*)A, lda, (const bf16_t*)W, ldw, (bf16_t*)C, ldc,
                     (const bf16_t*)R, ldr, M, N, K, n_major, 8, (int)ntiles);
  return kad_launch_status("gemm_x16p_kernel");
}

// 16-byte epilogue stores need aligned, 8-column-granular outputs
bool vector_epilogue_ok(const void* C, int64_t ldc, const void* R, int64_t ldr, int N, int epi) {
  const int n_out = epi == KAD_EPI_SWIGLU ? N / 2 : N;
  bool ok = ((uintptr_t)C % 16) == 0 && ldc % 8 == 0 && n_out % 8 == 0;
  if (epi == KAD_EPI_RESIDUAL) ok = ok && ((uintptr_t)R % 16) == 0 && ldr % 8 == 0;
  return ok;
}

template <int BM, int BN, int WM_, int WN_, int EPI>
int launch(const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
           const void* R, int64_t ldr, int M, int N, int K, hipStream_t s) {
  const int64_t mt = kad_cdiv(M, BM), nt = kad_cdiv(N, BN);
  const int64_t nblocks = mt * nt;
  if (nblocks > 0x7fffffff) KAD_UNSUPPORTED("gemm grid too large");
  // reuse the larger operand: weights (N*K) vs activations (M*K)
  const int n_major = (int64_t)N >= (int64_t)M ? 1 : 0;
  hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM_, WN_, EPI>), dim3((unsigned)nblocks),
                     dim3(64 * WM_ * WN_),
                     0, s, (const bf16_t*)A, lda, (const bf16_t*)W, ldw, (bf16_t*)C, ldc,
                     (const bf16_t*)R, ldr, M, N, K, n_major);
  return kad_launch_status("gemm_bf16_kernel");
}

// Outputs of at most 32 columns (the GDN gate projection, N = 2 x value
// heads), read-bound on A.  The generic 64 x 32 tiles leave half the chip
// idle at M = 8,192 and wait for HBM once per 64-deep K tile.  Here a wave
// owns 32 rows and walks the whole of K after one barrier: the weight is
// copied into LDS once per workgroup, step-major (each 16-deep K step's
// 32 x 16 elements form 1 KB, which a wave's fragment read takes whole, free
// of bank conflicts), and the wave's rows of A stream through registers in slices of
// 256 of K, three slices in flight.  The MFMA chain is the generic kernel's
// 32x32x16 one in the same K order, so the results are the same bits.  One
// wave per workgroup when the waves number fewer than two per CU (M =
// 8,192: every CU then holds a wave, 11.4 -> 8.9 us in the search), else four sharing
// the weight's copy.
constexpr int kN32Steps = 16;  // 16-deep MFMA steps per slice

template <int EPI, int NSL, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void gemm_n32_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ Wt, int64_t ldw,
    bf16_t* C, int64_t ldc, const bf16_t* R, int64_t ldr, int M, int N) {
  constexpr int K = NSL * kN32Steps * 16;
  extern __shared__ __attribute__((aligned(16))) bf16_t wsm[];  // [K / 16][32 rows][16]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = (blockIdx.x * WAVES + wave) * 32;
  const int r = lane & 31, kq = (lane >> 5) * 8;
  // rows past M read row M - 1 (their results are not stored)
  const bf16_t* a = A + (int64_t)min(m0 + r, M - 1) * lda + kq;
  u32x4 ar[3][kN32Steps];
  auto fetch = [&](u32x4 (&dst)[kN32Steps], int sl) {
#pragma unroll
    for (int i = 0; i < kN32Steps; ++i) dst[i] = *(const u32x4*)(a + (sl * kN32Steps + i) * 16);
  };
#pragma unroll
  for (int sl = 0; sl < 3; ++sl)
    if (sl < NSL) fetch(ar[sl], sl);
  // the weight into LDS by direct loads, one 16-deep K step (32 rows x 32
  // bytes, 1 KB) per instruction, all in flight at once: lane l fetches row
  // l / 2 (rows past N read row N - 1), bytes 16 (l % 2) .. +15 of the step
  {
    const bf16_t* wg = Wt + (int64_t)min(lane >> 1, N - 1) * ldw + (lane & 1) * 8;
    for (int kt = wave; kt < K / 16; kt += WAVES) dma16(wg + kt * 16, wsm + kt * 512);
  }
  __syncthreads();
  // fragment of step kt: row lane % 32, elements 8 (lane / 32) .. +7
  const bf16_t* wl = wsm + r * 16 + kq;
  f32x16 acc = {};
#pragma unroll
  for (int sl = 0; sl < NSL; ++sl) {
#pragma unroll
    for (int i = 0; i < kN32Steps; ++i) {
      const bf16x8 wf = as_bf16x8(*(const u32x4*)(wl + (sl * kN32Steps + i) * 512));
      acc = mfma32x32x16(as_bf16x8(ar[sl % 3][i]), wf, acc);
    }
    if (sl + 3 < NSL) fetch(ar[sl % 3], sl + 3);
  }
  // lane holds column lane % 32 and rows (e/4)*8 + (lane/32)*4 + e%4
  const int col = lane & 31, row_q = (lane >> 5) * 4;
  if (m0 >= M || col >= N) return;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int row = m0 + row_q + (e / 4) * 8 + (e % 4);
    if (row < M) {
      float v = acc[e];
      if constexpr (EPI == KAD_EPI_RESIDUAL) v = bf2f(R[(int64_t)row * ldr + col]) + round_bf(v);
      C[(int64_t)row * ldc + col] = f2bf(v);
    }
  }
}

// whole-K rows of A and the weight in 16-byte units, K a multiple of 256 up
// to 2,048 (the weight's LDS copy at most 128 KB)
bool n32_ok(const void* A, int64_t lda, const void* W, int64_t ldw, int N, int K, int epi) {
  return epi != KAD_EPI_SWIGLU && N <= 32 && K % 256 == 0 && K >= 256 && K <= 2048 &&
         ((uintptr_t)A % 16) == 0 && ((uintptr_t)W % 16) == 0 && lda % 8 == 0 && ldw % 8 == 0;
}

template <int EPI, int NSL, int WAVES>
int launch_n32_w(const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
                 const void* R, int64_t ldr, int M, int N, hipStream_t s) {
  const size_t lds = (size_t)32 * NSL * kN32Steps * 16 * 2;
  static bool configured = false;
  if (!configured) {
    if (hipFuncSetAttribute((const void*)gemm_n32_kernel<EPI, NSL, WAVES>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
      kad_set_error("gemm: cannot reserve %zu bytes of LDS", lds);
      return KAD_ERR_HIP;
    }
    configured = true;
  }
  const int64_t nblocks = kad_cdiv(M, 32 * WAVES);
  hipLaunchKernelGGL((gemm_n32_kernel<EPI, NSL, WAVES>), dim3((unsigned)nblocks), dim3(64 * WAVES),
                     lds, s, (const bf16_t*)A, lda, (const bf16_t*)W, ldw, (bf16_t*)C, ldc,
                     (const bf16_t*)R, ldr, M, N);
  return kad_launch_status("gemm_n32_kernel");
}

template <int EPI, int NSL>
int launch_n32_at(const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
                  const void* R, int64_t ldr, int M, int N, hipStream_t s) {
  if (kad_cdiv(M, 32) < 2 * (int64_t)device_cu_count())
    return launch_n32_w<EPI, NSL, 1>(A, lda, W, ldw, C, ldc, R, ldr, M, N, s);
  return launch_n32_w<EPI, NSL, 4>(A, lda, W, ldw, C, ldc, R, ldr, M, N, s);
}

template <int EPI>
int launch_n32(const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
               const void* R, int64_t ldr, int M, int N, int K, hipStream_t s) {
  if (!n32_ok(A, lda, W, ldw, N, K, EPI))
    KAD_UNSUPPORTED("tile configuration 13 needs N <= 32, K a multiple of 256 up to 2,048, "
                    "16-byte aligned A and W rows and no SwiGLU epilogue");
  switch (K / 256) {
    case 1: return launch_n32_at<EPI, 1>(A, lda, W, ldw, C, ldc, R, ldr, M, N, s);
    case 2: return launch_n32_at<EPI, 2>(A, lda, W, ldw, C, ldc, R, ldr, M, N, s);
    case 3: return launch_n32_at<EPI, 3>(A, lda, W, ldw, C, ldc, R, ldr, M, N, s);
    case 4: return launch_n32_at<EPI, 4>(A, lda, W, ldw, C, ldc, R, ldr, M, N, s);
    case 5: return launch_n32_at<EPI, 5>(A, lda, W, ldw, C, ldc, R, ldr, M, N, s);
    case 6: return launch_n32_at<EPI, 6>(A, lda, W, ldw, C, ldc, R, ldr, M, N, s);
    case 7: return launch_n32_at<EPI, 7>(A, lda, W, ldw, C, ldc, R, ldr, M, N, s);
    default: return launch_n32_at<EPI, 8>(A, lda, W, ldw, C, ldc, R, ldr, M, N, s);
  }
}

// tile configurations (tile_config argument of kad_gemm_bf16_tiled): the
// forms the automatic choice uses; the numbers are part of the C ABI
enum { CFG_AUTO = 0, CFG_32x256 = 1, CFG_128x128 = 2, CFG_256x256_8W = 5, CFG_64x32 = 11,
       CFG_32x64 = 12, CFG_N32 = 13,
       CFG_256x256_X16 = 16, CFG_256x256_X16P = 18, CFG_128x128_X16 = 19,
       CFG_256x256_S3 = 20, CFG_256x256_PPP = 22, CFG_256x256_W4E = 24 };

template <int EPI>
int pick(int cfg, const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
         const void* R, int64_t ldr, int M, int N, int K, hipStream_t s) {
  if (cfg == CFG_AUTO) {
    // the 8-wave 256x256 kernels on 16x16x32 MFMAs when their tiles still
    // fill every CU (and the output suits 16-byte stores): the ping-pong
    // kernel for plain products of at least four whole tiles per CU, a third
    // LDS slot for the streamed operand for K >= 3072 (residual outputs
    // from K = 2048: the prefill mixer output projection 2% faster), else
    // persistent, except for the SwiGLU epilogue in launches of fewer than
    // eight rounds, where one workgroup per tile with a split last round is
    // faster (decode SwiGLU 111.9 against 114.8 us; at M = 32,768 the
    // persistent form is 2% faster, interleaved medians); then the
    // 128x128 form, two workgroups per CU, when its tiles fill two rounds
    // (N = 1,024 at M = 8,192: 5-7% faster than 8-wave 256x128 tiles, and
    // 14% slower than 256x256 where those fill the chip); 64x32 for outputs
    // of at most 32 columns (the GDN gate projection); the register-staged
    // 128x128 kernel otherwise (all measured on the decode/prefill shapes)
    const int64_t tiles256 = kad_cdiv(M, 256) * kad_cdiv(N, 256);
    const int64_t tiles128 = kad_cdiv(M, 128) * kad_cdiv(N, 128);
    const bool vec = vector_epilogue_ok(C, ldc, R, ldr, N, EPI);
    if (M <= 64)
      cfg = N <= 2048 && EPI != KAD_EPI_SWIGLU ? CFG_32x64 : CFG_32x256;
    else if (N <= 32)
      // whole-K waves of 32 rows (the GDN gate projection at M = 8,192 and
      // 32,768), else 64x32 tiles
      cfg = n32_ok(A, lda, W, ldw, N, K, EPI) ? CFG_N32 : CFG_64x32;
    else if (tiles256 >= 256 && !vec)
      cfg = CFG_256x256_8W;
    else if (EPI == KAD_EPI_STORE && M % 256 == 0 && N % 256 == 0 && K <= 2048 &&
             tiles256 >= 4 * device_cu_count())
      // plain products of whole tiles, at least four per CU: the ping-pong
      // kernel (the GDN input projections 1-6%, the vocabulary head 3%
      // faster than configuration 18, interleaved A/B medians on one box)
      cfg = CFG_256x256_PPP;
    else if (EPI != KAD_EPI_STORE && M % 256 == 0 && N % 256 == 0 &&
             (EPI == KAD_EPI_RESIDUAL ? K >= 2048 && tiles256 >= 2 * device_cu_count()
                                      : tiles256 >= 8 * device_cu_count()))
      // the 4-wave kernel for whole-tile residual outputs from K = 2,048 (the
      // prefill mixer output and down projections 14% and 13% faster than
      // configuration 20) and SwiGLU launches of eight rounds or more (the
      // prefill gate/up projection 2% faster than configuration 18)
      cfg = CFG_256x256_W4E;
    else if (tiles256 >= 256 && (K >= 3072 || (EPI == KAD_EPI_RESIDUAL && K >= 2048)))
      cfg = CFG_256x256_S3;
    else if (tiles256 >= 256)
      cfg = EPI == KAD_EPI_SWIGLU && tiles256 < 8 * device_cu_count() ? CFG_256x256_X16
                                                                        : CFG_256x256_X16P;
    else if (vec && tiles128 >= 512)
      cfg = CFG_128x128_X16;
    else
      cfg = CFG_128x128;
    // A last round of 256 x 256 workgroups that would leave more than a
    // quarter of the CUs idle, in a launch of few rounds (the decode SwiGLU
    // projection at M = 8,192: 3.5 rounds): the columns past the last whole
    // round go to 128 x 128 tiles, two workgroups per CU, in a second launch
    // (114.8 -> 111.9 us there).  Every configuration accumulates K in the
    // same order, so the split does not change a bit of the result.  The
    // persistent kernel gains nothing from it (its workgroups take the
    // leftover tiles in turn: the decode QKV projection at 2.5 rounds ran
    // 79.2 us either way, the vocabulary head 0.6% slower split).
    if (cfg == CFG_256x256_X16) {
      const int64_t mt = kad_cdiv(M, 256), nt = kad_cdiv(N, 256);
      const int64_t cus = device_cu_count();
      const int64_t rem = tiles256 % cus;
      if (rem != 0 && rem * 4 < cus * 3 && tiles256 < 8 * cus) {
        int64_t n1 = nt - 1;
        while (n1 > 0 && (mt * n1) % cus != 0) --n1;
        if (n1 > 0) {
          const int N1 = (int)(n1 * 256);
          const int64_t c_off = EPI == KAD_EPI_SWIGLU ? N1 / 2 : N1;
          const int rc = pick<EPI>(cfg, A, lda, W, ldw, C, ldc, R, ldr, M, N1, K, s);
          if (rc) return rc;
          return pick<EPI>(CFG_128x128_X16, A, lda, (const bf16_t*)W + (int64_t)N1 * ldw, ldw,
                           (bf16_t*)C + c_off, ldc, R ? (const bf16_t*)R + N1 : nullptr, ldr, M,
                           N - N1, K, s);
        }
      }
    }
  }
  switch (cfg) {
    case CFG_32x256: return launch<32, 256, 1, 4, EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_32x64:
      // a few rows against a narrow weight (the pruned last prefill layer's
      // output and down projections, M = 32, N = 1,024): four times the
      // workgroups of 32x256 tiles (13.2 against 25.8 us at K = 2,048)
      if (EPI == KAD_EPI_SWIGLU) KAD_UNSUPPORTED("tile configuration 12 has no SwiGLU epilogue");
      return launch<32, 64, 1, 2, EPI == KAD_EPI_SWIGLU ? KAD_EPI_STORE : EPI>(
          A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_128x128: return launch<128, 128, 2, 2, EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_N32:
      if (EPI == KAD_EPI_SWIGLU) KAD_UNSUPPORTED("tile configuration 13 has no SwiGLU epilogue");
      return launch_n32<EPI == KAD_EPI_SWIGLU ? KAD_EPI_STORE : EPI>(A, lda, W, ldw, C, ldc, R, ldr,
                                                                     M, N, K, s);
    case CFG_64x32:
      // two waves of 32x32: twice the workgroups of 128x32 tiles for this
      // read-bound shape (12.1 against 14.0 us at M = 32,768, N = 32)
      if (EPI == KAD_EPI_SWIGLU) KAD_UNSUPPORTED("tile configuration 11 has no SwiGLU epilogue");
      return launch<64, 32, 2, 1, EPI == KAD_EPI_SWIGLU ? KAD_EPI_STORE : EPI>(
          A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_256x256_8W:
      return launch<256, 256, 2, 4, EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_256x256_X16:
    case CFG_256x256_X16P:
    case CFG_128x128_X16:
    case CFG_256x256_S3:
    case CFG_256x256_PPP:
    case CFG_256x256_W4E:
      if (!vector_epilogue_ok(C, ldc, R, ldr, N, EPI))
        KAD_UNSUPPORTED("tile configuration %d needs 16-byte aligned outputs in 8-column units",
                        cfg);
      if (cfg == CFG_256x256_X16)
        return launch_x16<EPI, Tile256>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
      if (cfg == CFG_256x256_S3)
        return launch_s3<EPI, Tile256>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
      if (cfg == CFG_256x256_W4E)
        return launch_w4e<EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
      if (cfg == CFG_256x256_PPP)
        return launch_ppp<EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
      if (cfg == CFG_128x128_X16)
        return launch_x16<EPI, TileX16<128, 128, 2, 2>>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K,
                                                        s);
      return launch_x16p<EPI, 256>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    default: KAD_UNSUPPORTED("unknown gemm tile configuration %d", cfg);
  }
}

}  // namespace

extern "C" int kad_gemm_bf16_tiled(const void* A, int64_t lda, const void* W, int64_t ldw,
                                   void* C, int64_t ldc, const void* R, int64_t ldr, int M, int N,
                                   int K, int epilogue, int tile_config, kad_stream_t stream) {
  KAD_REQUIRE(A && W && C, "null pointer argument");
  KAD_REQUIRE(M > 0 && N > 0 && K > 0, "dimensions must be positive");
  if (K % kBK) KAD_UNSUPPORTED("gemm requires K %% %d == 0, got K=%d", kBK, K);
  KAD_REQUIRE(lda >= K && ldw >= K && lda % 8 == 0 && ldw % 8 == 0,
              "lda/ldw must be >= K and multiples of 8");
  KAD_REQUIRE(((uintptr_t)A | (uintptr_t)W) % 16 == 0, "A and W must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  const int cfg = tile_config;
  switch (epilogue) {
    case KAD_EPI_STORE:
      KAD_REQUIRE(ldc >= N, "ldc must be >= N");
      return pick<KAD_EPI_STORE>(cfg, A, lda, W, ldw, C, ldc, nullptr, 0, M, N, K, s);
    case KAD_EPI_RESIDUAL:
      KAD_REQUIRE(R != nullptr && ldr >= N && ldc >= N, "residual epilogue needs R, ldr >= N");
      return pick<KAD_EPI_RESIDUAL>(cfg, A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case KAD_EPI_SWIGLU:
      KAD_REQUIRE(N % 64 == 0, "swiglu epilogue needs N %% 64 == 0 ([gate 32 | up 32] blocks)");
      KAD_REQUIRE(ldc >= N / 2, "ldc must be >= N/2");
      return pick<KAD_EPI_SWIGLU>(cfg, A, lda, W, ldw, C, ldc, nullptr, 0, M, N, K, s);
    default:
      KAD_REQUIRE(false, "unknown epilogue %d", epilogue);
  }
}

extern "C" int kad_gemm_bf16(const void* A, int64_t lda, const void* W, int64_t ldw, void* C,
                             int64_t ldc, const void* R, int64_t ldr, int M, int N, int K,
                             int epilogue, kad_stream_t stream) {
  return kad_gemm_bf16_tiled(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, epilogue, 0, stream);
}

extern "C" int kad_gemm_bf16_conv_workspace_bytes(int M, int conv_cols, int64_t* bytes) {
  KAD_REQUIRE(bytes, "null pointer argument");
  KAD_REQUIRE(M > 0 && conv_cols > 0, "dimensions must be positive");
  *bytes = (int64_t)((M + 127) / 128) * 7 * conv_cols * 2;
  return KAD_OK;
}

extern "C" int kad_gemm_bf16_conv(const void* A, int64_t lda, const void* W, int64_t ldw, void* C,
                                  int64_t ldc, int M, int N, int K, int conv_cols,
                                  const void* conv_weight, int seq_len, void* conv_state,
                                  void* workspace, int64_t workspace_bytes, kad_stream_t stream) {
  KAD_REQUIRE(A && W && C && conv_weight && workspace, "null pointer argument");
  KAD_REQUIRE(M > 0 && N > 0 && K > 0 && conv_cols > 0 && seq_len > 0,
              "dimensions must be positive");
  KAD_REQUIRE(lda >= K && ldw >= K && lda % 8 == 0 && ldw % 8 == 0,
              "lda/ldw must be >= K and multiples of 8");
  KAD_REQUIRE(((uintptr_t)A | (uintptr_t)W) % 16 == 0, "A and W must be 16-byte aligned");
  KAD_REQUIRE(ldc >= N && ldc % 8 == 0 && ((uintptr_t)C % 16) == 0,
              "C rows must be 16-byte aligned with ldc >= N");
  KAD_REQUIRE(((uintptr_t)conv_weight % 16) == 0, "the conv weight must be 16-byte aligned");
  KAD_REQUIRE(M % seq_len == 0, "M must be a whole number of sequences");
  int64_t need = 0;
  kad_gemm_bf16_conv_workspace_bytes(M, conv_cols, &need);
  KAD_REQUIRE(workspace_bytes >= need, "workspace of %lld bytes is smaller than %lld",
              (long long)workspace_bytes, (long long)need);
  KAD_REQUIRE(((uintptr_t)workspace % 16) == 0, "workspace must be 16-byte aligned");
  if (K % kBK || M % 256 || N % 256 || conv_cols % 256 || conv_cols > N || seq_len % 128)
    KAD_UNSUPPORTED("the conv projection takes M, N, conv_cols multiples of 256 (conv_cols <= N), "
                    "K %% %d == 0 and sequences of a multiple of 128 rows (got M=%d N=%d K=%d "
                    "conv_cols=%d seq_len=%d)", kBK, M, N, K, conv_cols, seq_len);
  hipStream_t s = (hipStream_t)stream;
  const ConvEpi ce{(const bf16_t*)conv_weight, (bf16_t*)workspace, conv_cols};
  if (const int rc = launch_ppp<kEpiConv>(A, lda, W, ldw, C, ldc, nullptr, 0, M, N, K, s, ce))
    return rc;
  const int nsub = M / 128;
  const int64_t threads = (int64_t)nsub * (conv_cols / 8);
  hipLaunchKernelGGL(conv_fixup_kernel, dim3((unsigned)kad_cdiv(threads, 256)), dim3(256), 0, s,
                     (const bf16_t*)workspace, (const bf16_t*)conv_weight, (bf16_t*)C, ldc,
                     (bf16_t*)conv_state, nsub, seq_len / 128, conv_cols);
  return kad_launch_status("conv_fixup_kernel");
}
