// Library-wide host utilities: error reporting, ABI version, MFMA self-test.

#include "kad_common.h"

static thread_local char g_last_error[512] = "";

void kad_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int kad_launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    kad_set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return KAD_ERR_HIP;
  }
  return KAD_OK;
}

extern "C" const char* kad_last_error(void) { return g_last_error; }
extern "C" int kad_abi_version(void) { return 2; }

// ---------------------------------------------------------------------------
// MFMA operand-layout self-test.  One wave loads row-major A, B into the
// fragment layout the kernels assume, issues one MFMA and stores C back
// row-major with the assumed output layout.  All indexes stay inside the
// 16x32 / 32x16 / 16x16 (or 32x16 / 16x32 / 32x32) buffers.

__global__ __launch_bounds__(64) void selftest16(const bf16_t* a, const bf16_t* b, float* c) {
  const int l = threadIdx.x;
  bf16x8 fa, fb;
  for (int i = 0; i < 8; ++i) {
    // A[16][32]: lane l holds row l%16, k = (l/16)*8 + i
    fa[i] = __builtin_bit_cast(__bf16, a[(l % 16) * 32 + (l / 16) * 8 + i]);
    // B[32][16]: lane l holds column l%16, k = (l/16)*8 + i
    fb[i] = __builtin_bit_cast(__bf16, b[((l / 16) * 8 + i) * 16 + (l % 16)]);
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  acc = mfma16x16x32(fa, fb, acc);
  for (int i = 0; i < 4; ++i) c[((l / 16) * 4 + i) * 16 + (l % 16)] = acc[i];
}

__global__ __launch_bounds__(64) void selftest32(const bf16_t* a, const bf16_t* b, float* c) {
  const int l = threadIdx.x;
  bf16x8 fa, fb;
  for (int i = 0; i < 8; ++i) {
    // A[32][16]: lane l holds row l%32, k = (l/32)*8 + i
    fa[i] = __builtin_bit_cast(__bf16, a[(l % 32) * 16 + (l / 32) * 8 + i]);
    // B[16][32]: lane l holds column l%32, k = (l/32)*8 + i
    fb[i] = __builtin_bit_cast(__bf16, b[((l / 32) * 8 + i) * 32 + (l % 32)]);
  }
  f32x16 acc = {};
  acc = mfma32x32x16(fa, fb, acc);
  for (int j = 0; j < 16; ++j) c[((j / 4) * 8 + (l / 32) * 4 + (j % 4)) * 32 + (l % 32)] = acc[j];
}

extern "C" int kad_selftest_mfma16(const void* a, const void* b, float* c, kad_stream_t stream) {
  KAD_REQUIRE(a && b && c, "null pointer argument");
  hipLaunchKernelGGL(selftest16, dim3(1), dim3(64), 0, (hipStream_t)stream, (const bf16_t*)a,
                     (const bf16_t*)b, c);
  return kad_launch_status("selftest16");
}

extern "C" int kad_selftest_mfma32(const void* a, const void* b, float* c, kad_stream_t stream) {
  KAD_REQUIRE(a && b && c, "null pointer argument");
  hipLaunchKernelGGL(selftest32, dim3(1), dim3(64), 0, (hipStream_t)stream, (const bf16_t*)a,
                     (const bf16_t*)b, c);
  return kad_launch_status("selftest32");
}

// ---------------------------------------------------------------------------
// HBM streaming probe: the bandwidth a plain streaming kernel reaches on this
// device, which the HBM-bound kernels are reported against beside the 8 TB/s
// datasheet figure.  mode 0 copies src to dst (read + write), 1 reads src (a
// lane writes only when its running XOR equals `magic`, which keeps the loads
// live), 2 writes dst.  16 bytes per lane per access, kProbeUnroll accesses in
// flight per lane, grid-stride over the buffer; every index is below n16.
constexpr int kProbeUnroll = 4;

__global__ __launch_bounds__(256) void hbm_probe_kernel(const u32x4* __restrict__ src,
                                                        u32x4* __restrict__ dst, int64_t n16,
                                                        int mode, uint32_t magic) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  const u32x4 fill = {magic, magic ^ 1u, magic ^ 2u, magic ^ 3u};
  int64_t i = gid;
  for (; i + (kProbeUnroll - 1) * stride < n16; i += kProbeUnroll * stride) {
    if (mode == 2) {
#pragma unroll
      for (int u = 0; u < kProbeUnroll; ++u) dst[i + u * stride] = fill;
      continue;
    }
    u32x4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * stride);
    if (mode == 0) {
#pragma unroll
      for (int u = 0; u < kProbeUnroll; ++u) dst[i + u * stride] = v[u];
    } else {
#pragma unroll
      for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u];
    }
  }
  for (; i < n16; i += stride) {
    if (mode == 2) dst[i] = fill;
    else if (mode == 0) dst[i] = src[i];
    else acc ^= src[i];
  }
  if (mode == 1 && acc[0] == magic && acc[1] == magic && gid < n16) dst[gid] = acc;
}

extern "C" int kad_hbm_probe(const void* src, void* dst, int64_t bytes, int mode,
                             kad_stream_t stream) {
  KAD_REQUIRE(mode >= 0 && mode <= 2, "probe mode must be 0 (copy), 1 (read) or 2 (write)");
  KAD_REQUIRE(bytes > 0 && bytes % 16 == 0, "probe size must be a positive multiple of 16");
  KAD_REQUIRE(dst && (mode == 2 || src), "null pointer argument");
  KAD_REQUIRE(((uintptr_t)dst % 16) == 0 && ((uintptr_t)src % 16) == 0,
              "probe buffers must be 16-byte aligned");
  const int64_t n16 = bytes / 16;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t want = (int64_t)cus * 8;  // 8 workgroups of 256 lanes per CU
  const int64_t blocks = want < kad_cdiv(n16, 256) ? want : kad_cdiv(n16, 256);
  hipLaunchKernelGGL(hbm_probe_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const u32x4*)src, (u32x4*)dst, n16, mode, 0x9e3779b9u);
  return kad_launch_status("hbm_probe_kernel");
}

// ---------------------------------------------------------------------------
// Cache prefetch: reads up to two ranges with ordinary (cache-allocating)
// loads and discards the data, so that the next kernels on the stream find
// them in the 256 MB last-level cache instead of HBM.  A GEMM whose weight
// arrives cold pays far more than the weight's bytes at HBM rate: its
// workgroups miss on the same panels together and wait out HBM latency.  The
// loads stay live through an empty asm statement that takes their XOR; the
// kernel writes nothing.  The two ranges form one index space, and each lane
// issues all its kPrefetchDepth loads before it uses one, so that a launch of
// a few tens of megabytes takes one memory round trip per lane: indices past
// the end are clamped to the last piece (re-read, not skipped: a guarded load
// would make the compiler wait for each one in turn).  Every load's index is
// below n0 + n1 and maps into its own range.
constexpr int kPrefetchDepth = 8;

__global__ __launch_bounds__(256) void cache_prefetch_kernel(const u32x4* __restrict__ p0,
                                                             int64_t n0,
                                                             const u32x4* __restrict__ p1,
                                                             int64_t n1) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  const int64_t n = n0 + n1;
  uint32_t acc = 0u;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += kPrefetchDepth * stride) {
    u32x4 v[kPrefetchDepth];
#pragma unroll
    for (int u = 0; u < kPrefetchDepth; ++u) {
      const int64_t j = min(i + u * stride, n - 1);
      v[u] = *(j < n0 ? p0 + j : p1 + (j - n0));
    }
#pragma unroll
    for (int u = 0; u < kPrefetchDepth; ++u) acc ^= v[u][0];
  }
  asm volatile("" ::"v"(acc));
}

extern "C" int kad_cache_prefetch(const void* p0, int64_t bytes0, const void* p1, int64_t bytes1,
                                  kad_stream_t stream) {
  KAD_REQUIRE(bytes0 >= 0 && bytes1 >= 0, "prefetch sizes must not be negative");
  KAD_REQUIRE((bytes0 == 0 || p0) && (bytes1 == 0 || p1), "null pointer argument");
  KAD_REQUIRE(((uintptr_t)p0 % 16) == 0 && ((uintptr_t)p1 % 16) == 0,
              "prefetch ranges must be 16-byte aligned");
  const int64_t n0 = bytes0 / 16, n1 = bytes1 / 16;   // whole 16-byte pieces
  if (n0 + n1 == 0) return KAD_OK;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t want = (int64_t)cus * 8;  // 8 workgroups of 256 lanes per CU
  const int64_t need = kad_cdiv(n0 + n1, 256);
  const int64_t blocks = want < need ? want : need;
  hipLaunchKernelGGL(cache_prefetch_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     (hipStream_t)stream, (const u32x4*)p0, n0, (const u32x4*)p1, n1);
  return kad_launch_status("cache_prefetch_kernel");
}
