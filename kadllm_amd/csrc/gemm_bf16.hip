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

// 256 x BN tiles (BN = 256 or 128), 4 waves (2 x 2), each wave a 128 x BN/2
// sub-tile: 4 * BN/64 MFMA 32x32x16 per 16-deep K step against 4 + BN/64
// fragment loads.  256x256 gives the highest MFMA-to-LDS ratio the
// 512-register file allows (a second wave per SIMD would halve it); 256x128
// fills the chip on narrow outputs (N = 1024 at M = 8192 is 256 tiles).
//
// Operand tiles move HBM -> LDS with global_load_lds_dwordx4 (no register
// staging): one wave instruction writes 64 x 16 bytes contiguously, i.e. 8
// tile rows of 128 bytes.  Within a row the 16-byte chunk c of K is stored at
// chunk c ^ ((row >> 1) & 7), so that the fragment reads (16 lanes = 16
// consecutive rows at one chunk) hit 16 distinct 16-byte bank groups; each
// lane of a load therefore fetches the global chunk that belongs at its LDS
// slot.  Two stages of 64-deep K: tile kt+1 is in flight while tile kt feeds
// the MFMAs.  Each 16-deep step is its own scheduling region with its MFMAs
// interleaved with the next step's fragment reads and the next tile's loads
// (MODE 0: all in step 0; MODE 2: split over steps 0 and 1, which measured
// 2-5% faster).  MODE 1 stages the same loads through registers
// (global_load_dwordx4 in step 0, ds_write_b128 in step 2 to the same
// swizzled positions).
//
// Operands are swapped (weight rows are the MFMA's A operand), so each lane's
// accumulators hold 4 consecutive output columns: the epilogue packs them 8
// bytes at a time into LDS, and the wave then writes its sub-tile with
// 16-byte stores (fusing the residual add or SwiGLU on the way).  Every
// configuration accumulates K in the same order, so results are bit-identical
// across tile shapes.
constexpr int kT = 256;

template <int BN>
struct Tile256 {
  static constexpr int NJ = BN / 64;                 // 32-column blocks per wave
  static constexpr int Stage = (kT + BN) * kBK;      // elements per stage: A rows then W rows
  static constexpr int EpiLd = BN / 2 + 8;           // epilogue LDS row stride (elements)
  static constexpr int Smem = 2 * Stage > 4 * 128 * EpiLd ? 2 * Stage : 4 * 128 * EpiLd;
};

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

// Origin of this workgroup's 256 x BN tile.  Grouped order: `group`
// consecutive tiles along the outer dimension share each inner-dimension
// tile, so an XCD's resident tiles form a 2-D block and both operands are
// reused from its L2.
__device__ __forceinline__ void tile_origin_of(int lid, int M, int N, int BN, int n_major,
                                              int group, int& m0, int& n0) {
  const int mtiles = (M + kT - 1) / kT, ntiles = (N + BN - 1) / BN;
  const int nx = n_major ? ntiles : mtiles, ny = n_major ? mtiles : ntiles;
  const int gx0 = (lid / (group * ny)) * group, gs = min(nx - gx0, group);
  const int within = lid % (group * ny);
  const int tx = gx0 + within % gs, ty = within / gs;
  const int mi = n_major ? ty : tx, ni = n_major ? tx : ty;
  m0 = mi * kT;
  n0 = ni * BN;
}

__device__ __forceinline__ void tile_origin(int M, int N, int BN, int n_major, int group, int& m0,
                                           int& n0) {
  tile_origin_of(xcd_logical_id(blockIdx.x, gridDim.x), M, N, BN, n_major, group, m0, n0);
}

__device__ __forceinline__ void dma16(const bf16_t* g, bf16_t* lds_block) {
  __builtin_amdgcn_global_load_lds((global_void_t*)g, (lds_void_t*)lds_block, 16, 0, 0);
}

// Epilogue.  acc[i][j][e]: row m = i*32 + lane%32, column
// n = j*32 + (e/4)*8 + (lane/32)*4 + e%4 of the wave's 128 x BN/2 sub-tile
// (waves 2 x 2).  The accumulators go through LDS (smem free on entry) and
// leave as 16-byte row stores, fusing the residual add or SwiGLU.
template <int EPI, int BN>
__device__ __forceinline__ void epilogue_tile(f32x16 (&acc)[4][Tile256<BN>::NJ], bf16_t* smem,
                                              int lane, int wave, int m0, int n0, bf16_t* C,
                                              int64_t ldc, const bf16_t* R, int64_t ldr, int M,
                                              int N) {
  constexpr int NJ = Tile256<BN>::NJ, kEpiLd = Tile256<BN>::EpiLd;
  const int wm = wave >> 1, wn = wave & 1;
  bf16_t* ep = smem + wave * 128 * kEpiLd;
  const int e_row = lane & 31, e_col = (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (EPI == KAD_EPI_SWIGLU) {
#pragma unroll
      for (int j = 0; j < NJ; j += 2) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u32x2 packed;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            uint32_t two = 0;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              const int e = g * 4 + h * 2 + q;
              const float gv = round_bf(acc[i][j][e]);
              const float uv = round_bf(acc[i][j + 1][e]);
              two |= (uint32_t)f2bf(round_bf(silu_rcp(gv)) * uv) << (16 * q);
            }
            packed[h] = two;
          }
          *(u32x2*)(ep + (i * 32 + e_row) * kEpiLd + (j / 2) * 32 + g * 8 + e_col) = packed;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u32x2 packed;
#pragma unroll
          for (int h = 0; h < 2; ++h)
            packed[h] = (uint32_t)f2bf(acc[i][j][g * 4 + h * 2]) |
                        ((uint32_t)f2bf(acc[i][j][g * 4 + h * 2 + 1]) << 16);
          *(u32x2*)(ep + (i * 32 + e_row) * kEpiLd + j * 32 + g * 8 + e_col) = packed;
        }
      }
    }
  }
  __syncthreads();
  constexpr int kCols = EPI == KAD_EPI_SWIGLU ? BN / 4 : BN / 2;  // wave sub-tile output columns
  constexpr int kChunks = kCols / 8, kRowsPer = 64 / kChunks;
  const int c_row = lane / kChunks, c_col = (lane % kChunks) * 8;
  const int out_n0 = EPI == KAD_EPI_SWIGLU ? n0 / 2 + wn * kCols : n0 + wn * kCols;
  const int n_out = EPI == KAD_EPI_SWIGLU ? N / 2 : N;
#pragma unroll 4
  for (int r = c_row; r < 128; r += kRowsPer) {
    const int row = m0 + wm * 128 + r, col = out_n0 + c_col;
    if (row >= M || col >= n_out) continue;
    u32x4 v = *(const u32x4*)(ep + r * kEpiLd + c_col);
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

// issue order inside one 16-deep step: NM MFMAs, each followed by up to one
// fragment read (NR in all), and the step's NV global loads and NW LDS writes
// spread one per MFMA (two when there are at least NM of them)
template <int NM, int NR, int NV, int NW>
__device__ __forceinline__ void interleave_step() {
  constexpr int PV = NV >= NM ? 2 : 1, PW = NW >= NM ? 2 : 1;
#pragma unroll
  for (int t = 0; t < NM; ++t) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (t < NR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    if (t * PV < NV) __builtin_amdgcn_sched_group_barrier(0x020, PV, 0);
    if (t * PW < NW) __builtin_amdgcn_sched_group_barrier(0x200, PW, 0);
  }
  __builtin_amdgcn_sched_barrier(0);  // steps are separate scheduling regions
}

// issue order inside one 16-deep step when the step's fragment reads come
// before its global loads in program order (the loads write LDS, so they
// cannot be hoisted above reads that might alias): NR MFMAs each followed by
// one fragment read, then the NV global loads spread evenly over the
// remaining NM - NR MFMAs
template <int NM, int NR, int NV>
__device__ __forceinline__ void interleave_reads_then_loads() {
#pragma unroll
  for (int t = 0; t < NM; ++t) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (t < NR) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    } else {
      constexpr int kSlots = NM - NR;
      const int c = ((t - NR + 1) * NV) / kSlots - ((t - NR) * NV) / kSlots;
#pragma unroll
      for (int q = 0; q < c; ++q) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

template <int EPI, int BN, int MODE>
__global__ __launch_bounds__(256, 1) void gemm256_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ Wt, int64_t ldw,
    bf16_t* C, int64_t ldc, const bf16_t* R, int64_t ldr, int M, int N, int K, int n_major,
    int group) {
  using TL = Tile256<BN>;
  constexpr int NJ = TL::NJ, kStage = TL::Stage;
  constexpr int WG = BN / 32;          // W row groups of 8 rows per wave
  constexpr bool DMA = MODE != 1;
  constexpr int NM = 4 * NJ, NR = 4 + NJ;  // MFMAs and fragment reads per step
  __shared__ __attribute__((aligned(1024))) bf16_t smem[TL::Smem];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int m0, n0;
  tile_origin(M, N, BN, n_major, group, m0, n0);

  // this wave loads row groups g = wave + 4 i (8 rows each) of both tiles;
  // lane L -> row g*8 + L/8, LDS chunk L%8, global chunk (L%8) ^ ((row>>1)&7)
  const int d_row = lane >> 3;
  const int d_kc = ((lane & 7) ^ ((wave & 1) * 4 + (lane >> 4))) * 8;
  const bf16_t* a_src[8];
  const bf16_t* b_src[WG];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = (wave + 4 * i) * 8 + d_row;
    a_src[i] = A + (int64_t)min(m0 + r, M - 1) * lda + d_kc;
    if (i < WG) b_src[i] = Wt + (int64_t)min(n0 + r, N - 1) * ldw + d_kc;
  }
  // row groups [i0, i1) of the A tile and [i0 * WG / 8, i1 * WG / 8) of the W tile
  auto issue = [&](int stage, int k0, int i0, int i1) {
    bf16_t* base = smem + stage * kStage + wave * 8 * kBK;
#pragma unroll
    for (int i = i0; i < i1; ++i) dma16(a_src[i] + k0, base + i * 32 * kBK);
#pragma unroll
    for (int i = i0 * WG / 8; i < i1 * WG / 8; ++i)
      dma16(b_src[i] + k0, base + kT * kBK + i * 32 * kBK);
  };
  u32x4 ra[DMA ? 1 : 8], rb[DMA ? 1 : WG];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < (DMA ? 0 : 8); ++i) {
      ra[i] = *(const u32x4*)(a_src[i] + k0);
      if (i < WG) rb[i] = *(const u32x4*)(b_src[i] + k0);
    }
  };
  auto stash = [&](int stage) {
    bf16_t* base = smem + stage * kStage + wave * 8 * kBK + lane * 8;
#pragma unroll
    for (int i = 0; i < (DMA ? 0 : 8); ++i) {
      *(u32x4*)(base + i * 32 * kBK) = ra[i];
      if (i < WG) *(u32x4*)(base + kT * kBK + i * 32 * kBK) = rb[i];
    }
  };

  // fragments: lane reads row lane%32 of a 32-row block at K chunk
  // kk*2 + lane/32, stored at chunk ^ ((row >> 1) & 7)
  const int f_row = lane & 31, f_sw = (lane >> 1) & 7, f_hi = lane >> 5;
  const int fa_row = (wm * 128 + f_row) * kBK;
  const int fw_row = kT * kBK + (wn * (BN / 2) + f_row) * kBK;
  bf16x8 fa[2][4], fw[2][NJ];
  auto load_frags = [&](int stage, int kk, int slot) {
    const bf16_t* base = smem + stage * kStage + (((kk * 2 + f_hi) ^ f_sw) * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      fa[slot][i] = as_bf16x8(*(const u32x4*)(base + fa_row + i * 32 * kBK));
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      fw[slot][j] = as_bf16x8(*(const u32x4*)(base + fw_row + j * 32 * kBK));
  };

  f32x16 acc[4][NJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x16{};
  auto mfma_step = [&](int slot) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = mfma32x32x16(fw[slot][j], fa[slot][i], acc[i][j]);
  };

  constexpr int kLoads = 8 + WG;  // global loads per wave per K tile
  const int KT = K / kBK;
  if constexpr (DMA) {
    issue(0, 0, 0, 8);
  } else {
    fetch(0);
    stash(0);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  load_frags(0, 0, 0);
  for (int kt = 0; kt < KT; ++kt) {
    __builtin_amdgcn_sched_barrier(0);
    const int stage = kt & 1;
    // loads of the next tile (the last iteration re-fetches the final tile,
    // keeping the loop body one basic block)
    const int kn = min(kt + 1, KT - 1) * kBK;
    if constexpr (MODE == 4) {
      load_frags(stage, 1, 1);
      issue(stage ^ 1, kn, 0, 4);
      mfma_step(0);
      interleave_reads_then_loads<NM, NR, kLoads / 2>();
      load_frags(stage, 2, 0);
      issue(stage ^ 1, kn, 4, 8);
      mfma_step(1);
      interleave_reads_then_loads<NM, NR, kLoads / 2>();
    } else if constexpr (MODE == 2) {
      issue(stage ^ 1, kn, 0, 4);
      load_frags(stage, 1, 1);
      mfma_step(0);
      interleave_step<NM, NR, kLoads / 2, 0>();
      issue(stage ^ 1, kn, 4, 8);
      load_frags(stage, 2, 0);
      mfma_step(1);
      interleave_step<NM, NR, kLoads / 2, 0>();
    } else {
      if constexpr (DMA)
        issue(stage ^ 1, kn, 0, 8);
      else
        fetch(kn);
      load_frags(stage, 1, 1);
      mfma_step(0);
      interleave_step<NM, NR, kLoads, 0>();
      load_frags(stage, 2, 0);
      mfma_step(1);
      interleave_step<NM, NR, 0, 0>();
    }
    load_frags(stage, 3, 1);
    if constexpr (!DMA) stash(stage ^ 1);  // nobody reads the idle stage
    mfma_step(0);
    interleave_step<NM, NR, 0, DMA ? 0 : kLoads>();
    // step 3: every read of this stage and the next tile's writes have
    // completed once all waves pass the barrier; prefetch the next stage's
    // step 0
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    load_frags(stage ^ 1, 0, 0);
    mfma_step(1);
    interleave_step<NM, NR, 0, 0>();
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  epilogue_tile<EPI, BN>(acc, smem, lane, wave, m0, n0, C, ldc, R, ldr, M, N);
}

template <int EPI, int BN, int MODE>
int launch_tile(const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
                const void* R, int64_t ldr, int M, int N, int K, hipStream_t s) {
  const int64_t nblocks = kad_cdiv(M, kT) * kad_cdiv(N, BN);
  if (nblocks > 0x7fffffff) KAD_UNSUPPORTED("gemm grid too large");
  const int n_major = (int64_t)N >= (int64_t)M ? 1 : 0;
  static const int group = [] {
    const char* e = getenv("KAD_GEMM_GROUP");
    return e ? atoi(e) : 8;
  }();
  hipLaunchKernelGGL((gemm256_kernel<EPI, BN, MODE>), dim3((unsigned)nblocks), dim3(256), 0, s,
                     (const bf16_t*)A, lda, (const bf16_t*)W, ldw, (bf16_t*)C, ldc,
                     (const bf16_t*)R, ldr, M, N, K, n_major, group < 1 ? 1 : group);
  return kad_launch_status("gemm256_kernel");
}

// Epilogue of one wave's (NI*32) x (NJ*32) sub-tile through a wave-private
// LDS region: accumulators packed as bf16 (SwiGLU applied), then 16-byte row
// stores with the residual add.  acc[i][j][e]: row i*32 + lane%32, column
// j*32 + (e/4)*8 + (lane/32)*4 + e%4.  No workgroup barrier: the caller has
// synchronised once after the main loop, and each wave only touches its own
// region.
template <int EPI, int NI, int NJ>
__device__ __forceinline__ void epilogue_sub(f32x16 (&acc)[NI][NJ], bf16_t* ep, int lane,
                                             int row0, int col0, bf16_t* C, int64_t ldc,
                                             const bf16_t* R, int64_t ldr, int M, int N) {
  constexpr int kCols = EPI == KAD_EPI_SWIGLU ? NJ * 16 : NJ * 32;  // output columns
  constexpr int kLd = kCols + 8;
  const int e_row = lane & 31, e_col = (lane >> 5) * 4;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    if constexpr (EPI == KAD_EPI_SWIGLU) {
#pragma unroll
      for (int j = 0; j < NJ; j += 2) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u32x2 packed;
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            uint32_t two = 0;
#pragma unroll
            for (int q = 0; q < 2; ++q) {
              const int e = g * 4 + h * 2 + q;
              const float gv = round_bf(acc[i][j][e]);
              const float uv = round_bf(acc[i][j + 1][e]);
              two |= (uint32_t)f2bf(round_bf(silu_rcp(gv)) * uv) << (16 * q);
            }
            packed[h] = two;
          }
          *(u32x2*)(ep + (i * 32 + e_row) * kLd + (j / 2) * 32 + g * 8 + e_col) = packed;
        }
      }
    } else {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u32x2 packed;
#pragma unroll
          for (int h = 0; h < 2; ++h)
            packed[h] = (uint32_t)f2bf(acc[i][j][g * 4 + h * 2]) |
                        ((uint32_t)f2bf(acc[i][j][g * 4 + h * 2 + 1]) << 16);
          *(u32x2*)(ep + (i * 32 + e_row) * kLd + j * 32 + g * 8 + e_col) = packed;
        }
      }
    }
  }
  // the wave's own LDS writes are visible to its later reads (in order)
  constexpr int kChunks = kCols / 8, kRowsPer = 64 / kChunks;
  const int c_row = lane / kChunks, c_col = (lane % kChunks) * 8;
  const int n_out = EPI == KAD_EPI_SWIGLU ? N / 2 : N;
#pragma unroll 4
  for (int r = c_row; r < NI * 32; r += kRowsPer) {
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

// The split-load schedule with 8 waves (2 per SIMD) on a 256 x BN tile:
// waves WM (M) x 8/WM (N), each an (NI*32) x (NJ*32) sub-tile.  The second
// wave of each SIMD issues its MFMAs while the other waits on its fragment
// reads.  BN = 256: waves 2 x 4 of 128 x 64; BN = 128: waves 4 x 2 of 64 x 64.
template <int BN>
struct TileW8 {
  static constexpr int NW = 8, WM = BN == 256 ? 2 : 4, WN = NW / WM;
  static constexpr int NI = kT / WM / 32, NJ = BN / WN / 32;
  static constexpr int Stage = (kT + BN) * kBK;
  static constexpr int AG = (kT / 8) / NW, WGW = (BN / 8) / NW;   // 8-row groups per wave
  static constexpr int EpiWave = NI * 32 * (NJ * 32 + 8);         // elements per wave
  static constexpr int Smem = 2 * Stage > NW * EpiWave ? 2 * Stage : NW * EpiWave;
};

template <int EPI, int BN>
__global__ __launch_bounds__(512, 1) void gemm256w8_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ Wt, int64_t ldw,
    bf16_t* C, int64_t ldc, const bf16_t* R, int64_t ldr, int M, int N, int K, int n_major,
    int group) {
  using TW = TileW8<BN>;
  constexpr int NW = TW::NW, WN = TW::WN, NI = TW::NI, NJ = TW::NJ;
  constexpr int kStage = TW::Stage, AG = TW::AG, WGW = TW::WGW;
  constexpr int kLoads = AG + WGW;
  constexpr int NM = NI * NJ, NR = NI + NJ;
  __shared__ __attribute__((aligned(1024))) bf16_t smem[TW::Smem];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int m0, n0;
  tile_origin(M, N, BN, n_major, group, m0, n0);

  // row groups g = wave + 8 i (8 rows each); lane L -> row g*8 + L/8, LDS
  // chunk L%8 holding global chunk (L%8) ^ ((row>>1)&7)
  const int d_row = lane >> 3;
  const int d_kc = ((lane & 7) ^ ((wave & 1) * 4 + (lane >> 4))) * 8;
  const bf16_t* a_src[AG];
  const bf16_t* b_src[WGW];
#pragma unroll
  for (int i = 0; i < AG; ++i) {
    const int r = (wave + NW * i) * 8 + d_row;
    a_src[i] = A + (int64_t)min(m0 + r, M - 1) * lda + d_kc;
    if (i < WGW) b_src[i] = Wt + (int64_t)min(n0 + r, N - 1) * ldw + d_kc;
  }
  // A groups [i0, i1) and W groups [i0 * WGW / AG, i1 * WGW / AG)
  auto issue = [&](int stage, int k0, int i0, int i1) {
    bf16_t* base = smem + stage * kStage + wave * 8 * kBK;
#pragma unroll
    for (int i = i0; i < i1; ++i) dma16(a_src[i] + k0, base + i * NW * 8 * kBK);
#pragma unroll
    for (int i = i0 * WGW / AG; i < i1 * WGW / AG; ++i)
      dma16(b_src[i] + k0, base + kT * kBK + i * NW * 8 * kBK);
  };

  const int f_row = lane & 31, f_sw = (lane >> 1) & 7, f_hi = lane >> 5;
  const int fa_row = (wm * NI * 32 + f_row) * kBK;
  const int fw_row = kT * kBK + (wn * NJ * 32 + f_row) * kBK;
  bf16x8 fa[2][NI], fw[2][NJ];
  auto load_frags = [&](int stage, int kk, int slot) {
    const bf16_t* base = smem + stage * kStage + (((kk * 2 + f_hi) ^ f_sw) * 8);
#pragma unroll
    for (int i = 0; i < NI; ++i)
      fa[slot][i] = as_bf16x8(*(const u32x4*)(base + fa_row + i * 32 * kBK));
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      fw[slot][j] = as_bf16x8(*(const u32x4*)(base + fw_row + j * 32 * kBK));
  };
  f32x16 acc[NI][NJ];
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x16{};
  auto mfma_step = [&](int slot) {
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = mfma32x32x16(fw[slot][j], fa[slot][i], acc[i][j]);
  };

  const int KT = K / kBK;
  issue(0, 0, 0, AG);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  load_frags(0, 0, 0);
  for (int kt = 0; kt < KT; ++kt) {
    __builtin_amdgcn_sched_barrier(0);
    const int stage = kt & 1;
    const int kn = min(kt + 1, KT - 1) * kBK;
    issue(stage ^ 1, kn, 0, AG / 2);
    load_frags(stage, 1, 1);
    mfma_step(0);
    interleave_step<NM, NR, kLoads / 2, 0>();
    issue(stage ^ 1, kn, AG / 2, AG);
    load_frags(stage, 2, 0);
    mfma_step(1);
    interleave_step<NM, NR, kLoads / 2, 0>();
    load_frags(stage, 3, 1);
    mfma_step(0);
    interleave_step<NM, NR, 0, 0>();
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    load_frags(stage ^ 1, 0, 0);
    mfma_step(1);
    interleave_step<NM, NR, 0, 0>();
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int col0 = EPI == KAD_EPI_SWIGLU ? (n0 + wn * NJ * 32) / 2 : n0 + wn * NJ * 32;
  epilogue_sub<EPI, NI, NJ>(acc, smem + wave * TW::EpiWave, lane, m0 + wm * NI * 32, col0, C,
                            ldc, R, ldr, M, N);
}

template <int EPI, int BN>
int launch_w8(const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
              const void* R, int64_t ldr, int M, int N, int K, hipStream_t s) {
  const int64_t nblocks = kad_cdiv(M, kT) * kad_cdiv(N, BN);
  if (nblocks > 0x7fffffff) KAD_UNSUPPORTED("gemm grid too large");
  const int n_major = (int64_t)N >= (int64_t)M ? 1 : 0;
  hipLaunchKernelGGL((gemm256w8_kernel<EPI, BN>), dim3((unsigned)nblocks), dim3(512), 0, s,
                     (const bf16_t*)A, lda, (const bf16_t*)W, ldw, (bf16_t*)C, ldc,
                     (const bf16_t*)R, ldr, M, N, K, n_major, 8);
  return kad_launch_status("gemm256w8_kernel");
}

// 256 x BN tile fed through a ring of 4 LDS slots of 32-deep K slices.  The
// loads of slice t + 3 are issued while slice t is consumed, half in each of
// its two 16-deep steps and spread between MFMAs, so they have two slices of
// time to land and never arrive in a burst.  One barrier per slice, in its
// middle: past it, slice t + 1 has landed (each wave waits for its own loads
// with a partial vmcnt, the barrier makes every wave's part visible) and
// every wave has finished reading slice t - 1, whose slot the next loads
// reuse.
constexpr int kRK = 32;    // K depth of a slot
constexpr int kRing = 4;   // slots

template <int BN>
struct Ring256 {
  static constexpr int NJ = BN / 64;              // 32-column blocks per wave
  static constexpr int WG = BN / 64;              // W 16-row groups per wave
  static constexpr int Loads = 4 + WG;            // DMA instructions per wave per slot
  static constexpr int Slot = (kT + BN) * kRK;    // elements per slot: A rows then W rows
  static constexpr int Smem = kRing * Slot > 4 * 128 * Tile256<BN>::EpiLd
                                  ? kRing * Slot
                                  : 4 * 128 * Tile256<BN>::EpiLd;
};

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

template <int EPI, int BN>
__global__ __launch_bounds__(256, 1) void gemm_ring_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ Wt, int64_t ldw,
    bf16_t* C, int64_t ldc, const bf16_t* R, int64_t ldr, int M, int N, int K, int n_major,
    int group) {
  using RL = Ring256<BN>;
  constexpr int NJ = RL::NJ, WG = RL::WG, kLoads = RL::Loads, kSlot = RL::Slot;
  constexpr int NM = 4 * NJ, NR = 4 + NJ;   // MFMAs and fragment reads per step
  constexpr int kHalf = kLoads / 2;
  __shared__ __attribute__((aligned(1024))) bf16_t smem[RL::Smem];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int m0, n0;
  tile_origin(M, N, BN, n_major, group, m0, n0);

  // one DMA instruction fills 16 rows of 64 bytes; this wave loads the
  // 16-row groups g = wave + 4 i of the A slice (i < 4) and of the W slice
  // (i < WG).  Lane L -> row g*16 + L/4, LDS chunk L%4 holding global chunk
  // (L%4) ^ (L/16): a row's 16-byte chunk c sits at c ^ ((row >> 2) & 3)
  const int d_row = lane >> 2;
  const int d_kc = ((lane & 3) ^ (lane >> 4)) * 8;
  const bf16_t* a_src[4];
  const bf16_t* b_src[WG];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (wave + 4 * i) * 16 + d_row;
    a_src[i] = A + (int64_t)min(m0 + r, M - 1) * lda + d_kc;
    if (i < WG) b_src[i] = Wt + (int64_t)min(n0 + r, N - 1) * ldw + d_kc;
  }
  // loads [j0, j1) of one slot: j < 4 are A groups, the rest W groups
  auto issue = [&](int slot, int k0, int j0, int j1) {
    bf16_t* base = smem + slot * kSlot + wave * 16 * kRK;
#pragma unroll
    for (int j = j0; j < j1; ++j) {
      if (j < 4)
        dma16(a_src[j] + k0, base + j * 64 * kRK);
      else
        dma16(b_src[j - 4] + k0, base + kT * kRK + (j - 4) * 64 * kRK);
    }
  };

  // fragments: lane reads row lane%32 of a 32-row block at K chunk
  // step*2 + lane/32, stored at chunk ^ ((row >> 2) & 3)
  const int f_row = lane & 31, f_sw = (lane >> 2) & 3, f_hi = lane >> 5;
  const int fa_row = (wm * 128 + f_row) * kRK;
  const int fw_row = kT * kRK + (wn * (BN / 2) + f_row) * kRK;
  bf16x8 fa[2][4], fw[2][NJ];
  auto load_frags = [&](int slot, int step, int buf) {
    const bf16_t* base = smem + slot * kSlot + (((step * 2 + f_hi) ^ f_sw) * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      fa[buf][i] = as_bf16x8(*(const u32x4*)(base + fa_row + i * 32 * kRK));
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      fw[buf][j] = as_bf16x8(*(const u32x4*)(base + fw_row + j * 32 * kRK));
  };

  f32x16 acc[4][NJ];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x16{};
  auto mfma_step = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) acc[i][j] = mfma32x32x16(fw[buf][j], fa[buf][i], acc[i][j]);
  };

  // past the last slice the loads re-fetch it, which keeps every
  // iteration's wait counts the same
  const int KT = K / kRK;
  issue(0, 0, 0, kLoads);
  issue(1, min(1, KT - 1) * kRK, 0, kLoads);
  issue(2, min(2, KT - 1) * kRK, 0, kLoads);
  __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(2 * kLoads));   // slice 0 landed
  ring_barrier();
  load_frags(0, 0, 0);
  for (int t = 0; t < KT; ++t) {
    __builtin_amdgcn_sched_barrier(0);
    const int slot = t & (kRing - 1), slot3 = (t + 3) & (kRing - 1);
    const int k3 = min(t + 3, KT - 1) * kRK;
    load_frags(slot, 1, 1);
    issue(slot3, k3, 0, kHalf);
    mfma_step(0);
    interleave_reads_then_loads<NM, NR, kHalf>();
    // slice t + 1 landed: only slice t + 2's loads and the first half of
    // slice t + 3's may still be in flight
    __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(kLoads + kHalf));
    ring_barrier();
    load_frags((t + 1) & (kRing - 1), 0, 0);
    issue(slot3, k3, kHalf, kLoads);
    mfma_step(1);
    interleave_reads_then_loads<NM, NR, kLoads - kHalf>();
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  epilogue_tile<EPI, BN>(acc, smem, lane, wave, m0, n0, C, ldc, R, ldr, M, N);
}

template <int EPI, int BN>
int launch_ring(const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
                const void* R, int64_t ldr, int M, int N, int K, hipStream_t s) {
  if (K % kRK) KAD_UNSUPPORTED("ring gemm needs K %% 32 == 0, got %d", K);
  const int64_t nblocks = kad_cdiv(M, kT) * kad_cdiv(N, BN);
  if (nblocks > 0x7fffffff) KAD_UNSUPPORTED("gemm grid too large");
  const int n_major = (int64_t)N >= (int64_t)M ? 1 : 0;
  hipLaunchKernelGGL((gemm_ring_kernel<EPI, BN>), dim3((unsigned)nblocks), dim3(256), 0, s,
                     (const bf16_t*)A, lda, (const bf16_t*)W, ldw, (bf16_t*)C, ldc,
                     (const bf16_t*)R, ldr, M, N, K, n_major, 8);
  return kad_launch_status("gemm_ring_kernel");
}

// 16x16x32 MFMA form of the 8-wave tile.  mfma16x16x32(w, a, c): lane l
// supplies row l%16 and K elements 8*(l/16) .. +7 of a 32-deep step of each
// operand; acc[i][j][e] then holds output row i*16 + l%16, column
// j*16 + 4*(l/16) + e of the wave's sub-tile (4 consecutive columns per lane).

template <int BN>
struct TileX16 {
  static constexpr int NW = 8, WM = BN == 256 ? 2 : 4, WN = NW / WM;
  static constexpr int NI = kT / WM / 16, NJ = BN / WN / 16;      // 16 x 16 blocks per wave
  static constexpr int Stage = (kT + BN) * kBK;
  static constexpr int AG = (kT / 8) / NW, WGW = (BN / 8) / NW;   // 8-row groups per wave
  static constexpr int Cols = NJ * 16;                            // wave sub-tile columns
  static constexpr int EpiWave = NI * 16 * (Cols + 8);
  static constexpr int Smem = 2 * Stage > NW * EpiWave ? 2 * Stage : NW * EpiWave;
};

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
        for (int h = 0; h < 2; ++h) {
          uint32_t two = 0;
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const float gv = round_bf(acc[i][j][h * 2 + q]);
            const float uv = round_bf(acc[i][j + 2][h * 2 + q]);
            two |= (uint32_t)f2bf(round_bf(silu_rcp(gv)) * uv) << (16 * q);
          }
          packed[h] = two;
        }
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
      constexpr int kSlots = NM - NR;
      const int c = ((t - NR + 1) * NV) / kSlots - ((t - NR) * NV) / kSlots;
#pragma unroll
      for (int q = 0; q < c; ++q) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

// 256 x BN tile, 8 waves, 16x16x32 MFMAs; two 64-deep LDS stages, two 32-deep
// steps per tile.  One barrier per tile, in the middle of step 1: past it the
// next tile has landed (each wave waited for its own loads) and every wave has
// read its last fragments of the current stage, so the loads of the tile
// after next go out into that stage at once and have a whole tile of time
// to land.
template <int EPI, int BN>
__global__ __launch_bounds__(512, 1) void gemm_x16_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ Wt, int64_t ldw,
    bf16_t* C, int64_t ldc, const bf16_t* R, int64_t ldr, int M, int N, int K, int n_major,
    int group) {
  using TX = TileX16<BN>;
  constexpr int NW = TX::NW, WN = TX::WN, NI = TX::NI, NJ = TX::NJ;
  constexpr int kStage = TX::Stage, AG = TX::AG, WGW = TX::WGW;
  constexpr int kLoads = AG + WGW;
  constexpr int NM = NI * NJ, NR = NI + NJ;
  __shared__ __attribute__((aligned(1024))) bf16_t smem[TX::Smem];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  int m0, n0;
  tile_origin(M, N, BN, n_major, group, m0, n0);

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
    for (int i = 0; i < WGW; ++i) dma16(b_base + (b_off[i] + k0), base + kT * kBK + i * NW * 8 * kBK);
  };

  // fragment lane l: row block_base + l%16, chunk 4*step + l/16, stored at
  // chunk ^ ((row >> 1) & 7)
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
    mfma_rows(1, 0, NI / 2);
    interleave_x16<NM / 2, 0, 0>();
    // tile kt + 1 landed; every wave is done reading this stage
    __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));
    ring_barrier();
    load_frags(stage ^ 1, 0, 0);
    issue(stage, k2);
    mfma_rows(1, NI / 2, NI);
    interleave_x16<NM / 2, NR, kLoads>();
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const int col0 = EPI == KAD_EPI_SWIGLU ? (n0 + wn * NJ * 16) / 2 : n0 + wn * NJ * 16;
  epilogue_x16<EPI, NI, NJ>(acc, smem + wave * TX::EpiWave, lane, m0 + wm * NI * 16, col0, C,
                            ldc, R, ldr, M, N);
}

template <int EPI, int BN>
int launch_x16(const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
               const void* R, int64_t ldr, int M, int N, int K, hipStream_t s) {
  const int64_t nblocks = kad_cdiv(M, kT) * kad_cdiv(N, BN);
  if (nblocks > 0x7fffffff) KAD_UNSUPPORTED("gemm grid too large");
  if ((int64_t)kT * (lda > ldw ? lda : ldw) + K >= 0x7fffffff)
    KAD_UNSUPPORTED("gemm rows too long for 32-bit tile offsets");
  const int n_major = (int64_t)N >= (int64_t)M ? 1 : 0;
  hipLaunchKernelGGL((gemm_x16_kernel<EPI, BN>), dim3((unsigned)nblocks), dim3(512), 0, s,
                     (const bf16_t*)A, lda, (const bf16_t*)W, ldw, (bf16_t*)C, ldc,
                     (const bf16_t*)R, ldr, M, N, K, n_major, 8);
  return kad_launch_status("gemm_x16_kernel");
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
        for (int h = 0; h < 2; ++h) {
          uint32_t two = 0;
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const float gv = round_bf(acc[i][j][h * 2 + q]);
            const float uv = round_bf(acc[i][j + 2][h * 2 + q]);
            two |= (uint32_t)f2bf(round_bf(silu_rcp(gv)) * uv) << (16 * q);
          }
          packed[h] = two;
        }
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

template <int EPI, int BN>
__global__ __launch_bounds__(512, 1) void gemm_x16p_kernel(
    const bf16_t* __restrict__ A, int64_t lda, const bf16_t* __restrict__ Wt, int64_t ldw,
    bf16_t* C, int64_t ldc, const bf16_t* R, int64_t ldr, int M, int N, int K, int n_major,
    int group, int ntiles) {
  using TX = TileX16<BN>;
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
    tile_origin_of(xcd_logical_id(v, ntiles), M, N, BN, n_major, group, m0, n0);
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
      mfma_rows(1, 0, NI / 2);
      interleave_x16<NM / 2, 0, 0>();
      // slice g + 1 landed; every wave is done reading this stage
      __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(0));
      ring_barrier();
      load_frags(stage ^ 1, 0, 0);
      issue(g + 2);
      mfma_rows(1, NI / 2, NI);
      interleave_x16<NM / 2, NR, kLoads>();
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

// tile configurations (tile_config argument of kad_gemm_bf16_tiled)
enum { CFG_AUTO = 0, CFG_32x256 = 1, CFG_128x128 = 2, CFG_128x256 = 3, CFG_256x256 = 4,
       CFG_256x256_8W = 5, CFG_256x128_8W = 6, CFG_256x256_PIPE = 7, CFG_256x256_PIPE_REG = 8,
       CFG_256x256_SPREAD = 9, CFG_256x128_PIPE = 10,
       CFG_128x32 = 11, CFG_256x256_RDFIRST = 12, CFG_256x256_RING = 13, CFG_256x256_W8 = 14,
       CFG_256x128_W8 = 15,
       CFG_256x256_X16 = 16, CFG_256x128_X16 = 17, CFG_256x256_X16P = 18,
       CFG_256x128_X16P = 19 };

template <int EPI>
int pick(int cfg, const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
         const void* R, int64_t ldr, int M, int N, int K, hipStream_t s) {
  if (cfg == CFG_AUTO) {
    // the 8-wave 256x256 kernel on 16x16x32 MFMAs when its tiles still fill
    // every CU (and the output suits 16-byte stores), persistent except for
    // the SwiGLU epilogue, where both forms measured the same; then the
    // 256x128 variant; 128x32 for outputs of at most 32 columns (the GDN gate
    // projection); 128x128 otherwise (all measured on the decode/prefill
    // shapes)
    const int64_t tiles256 = kad_cdiv(M, 256) * kad_cdiv(N, 256);
    const int64_t tiles128 = kad_cdiv(M, 256) * kad_cdiv(N, 128);
    const bool vec = vector_epilogue_ok(C, ldc, R, ldr, N, EPI);
    if (M <= 64)
      cfg = CFG_32x256;
    else if (N <= 32)
      cfg = CFG_128x32;
    else if (tiles256 >= 256 && !vec)
      cfg = CFG_256x256_8W;
    else if (tiles256 >= 256)
      cfg = EPI == KAD_EPI_SWIGLU ? CFG_256x256_X16 : CFG_256x256_X16P;
    else if (vec && tiles128 >= 256)
      cfg = CFG_256x128_X16;
    else
      cfg = CFG_128x128;
  }
  switch (cfg) {
    case CFG_32x256: return launch<32, 256, 1, 4, EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_128x128: return launch<128, 128, 2, 2, EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_128x32:
      if (EPI == KAD_EPI_SWIGLU) KAD_UNSUPPORTED("tile configuration 11 has no SwiGLU epilogue");
      return launch<128, 32, 4, 1, EPI == KAD_EPI_SWIGLU ? KAD_EPI_STORE : EPI>(
          A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_128x256: return launch<128, 256, 2, 2, EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_256x256: return launch<256, 256, 2, 2, EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_256x256_8W:
      return launch<256, 256, 2, 4, EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_256x256_PIPE:
    case CFG_256x256_PIPE_REG:
    case CFG_256x256_SPREAD:
    case CFG_256x128_PIPE:
      if (!vector_epilogue_ok(C, ldc, R, ldr, N, EPI))
        KAD_UNSUPPORTED("tile configuration %d needs 16-byte aligned outputs in 8-column units",
                        cfg);
      if (cfg == CFG_256x256_PIPE)
        return launch_tile<EPI, 256, 0>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
      if (cfg == CFG_256x256_PIPE_REG)
        return launch_tile<EPI, 256, 1>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
      if (cfg == CFG_256x256_SPREAD)
        return launch_tile<EPI, 256, 2>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
      return launch_tile<EPI, 128, 2>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_256x256_W8:
    case CFG_256x128_W8:
      if (!vector_epilogue_ok(C, ldc, R, ldr, N, EPI))
        KAD_UNSUPPORTED("tile configuration %d needs 16-byte aligned outputs in 8-column units",
                        cfg);
      if (cfg == CFG_256x256_W8)
        return launch_w8<EPI, 256>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
      return launch_w8<EPI, 128>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_256x256_X16:
    case CFG_256x128_X16:
      if (!vector_epilogue_ok(C, ldc, R, ldr, N, EPI))
        KAD_UNSUPPORTED("tile configuration %d needs 16-byte aligned outputs in 8-column units",
                        cfg);
      if (cfg == CFG_256x256_X16)
        return launch_x16<EPI, 256>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
      return launch_x16<EPI, 128>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_256x256_X16P:
    case CFG_256x128_X16P:
      if (!vector_epilogue_ok(C, ldc, R, ldr, N, EPI))
        KAD_UNSUPPORTED("tile configuration %d needs 16-byte aligned outputs in 8-column units",
                        cfg);
      if (cfg == CFG_256x256_X16P)
        return launch_x16p<EPI, 256>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
      return launch_x16p<EPI, 128>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_256x256_RDFIRST:
    case CFG_256x256_RING:
      if (!vector_epilogue_ok(C, ldc, R, ldr, N, EPI))
        KAD_UNSUPPORTED("tile configuration %d needs 16-byte aligned outputs in 8-column units",
                        cfg);
      if (cfg == CFG_256x256_RDFIRST)
        return launch_tile<EPI, 256, 4>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
      return launch_ring<EPI, 256>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_256x128_8W:
      return launch<256, 128, 4, 2, EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
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
