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
