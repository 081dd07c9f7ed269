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

#include "kad_common.h"

namespace {

constexpr int kBK = 64;
constexpr int kPad = 8;
constexpr int kLdk = kBK + kPad;  // LDS row stride (elements)

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
            const float s = round_bf(silu_f(gv));
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
       CFG_256x256_8W = 5, CFG_256x128_8W = 6 };

template <int EPI>
int pick(int cfg, const void* A, int64_t lda, const void* W, int64_t ldw, void* C, int64_t ldc,
         const void* R, int64_t ldr, int M, int N, int K, hipStream_t s) {
  if (cfg == CFG_AUTO) {
    // 256x256 tiles with 8 waves (two per SIMD) when they still fill every CU;
    // 128x128 otherwise (measured on the decode/prefill projection shapes)
    const int64_t tiles256 = kad_cdiv(M, 256) * kad_cdiv(N, 256);
    cfg = M <= 64 ? CFG_32x256 : (tiles256 >= 256 ? CFG_256x256_8W : CFG_128x128);
  }
  switch (cfg) {
    case CFG_32x256: return launch<32, 256, 1, 4, EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_128x128: return launch<128, 128, 2, 2, EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_128x256: return launch<128, 256, 2, 2, EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_256x256: return launch<256, 256, 2, 2, EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
    case CFG_256x256_8W:
      return launch<256, 256, 2, 4, EPI>(A, lda, W, ldw, C, ldc, R, ldr, M, N, K, s);
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
