// Sustained bf16 MFMA rate of the whole GPU, for reading the attention
// kernels' roofline fraction against what the part delivers under load.
//
// Every wave of 2 x CUs workgroups (2 waves per SIMD) issues back-to-back
// v_mfma_f32_32x32x16_bf16 on 4 independent accumulators.  The operands are
// either pseudo-random bf16 values (the switching activity of real data) or
// zeros; the difference measures how much the board's power management lowers
// the shader clock for data-dependent MFMA work.  Each wave also reads the
// shader clock (s_memtime) and the 100 MHz reference clock (s_memrealtime) at
// its start and end, so the clock the work ran at is reported with the rate.
//
// Not part of the attention ABI: built into its own library (libmt_probe.so)
// and used only by bench.py.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kChains = 4;

__global__ __launch_bounds__(256, 2) void mfma_probe_kernel(int iters, int random_operands, float* sink,
                                                             unsigned long long* clocks) {
  bf16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    uint32_t h = (threadIdx.x * 2654435761u) ^ (blockIdx.x * 40503u) ^ (uint32_t(e) * 2246822519u);
    h ^= h >> 13;
    h *= 0x5bd1e995u;
    h ^= h >> 15;
    const float x = random_operands ? float(int(h & 0xffffu) - 32768) * (1.0f / 32768.0f) : 0.f;
    const float y = random_operands ? float(int(h >> 16) - 32768) * (1.0f / 32768.0f) : 0.f;
    a[e] = (__bf16)x;
    b[e] = (__bf16)y;
  }
  f32x16 acc[kChains] = {};
  const unsigned long long m0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < kChains; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
  }
  const unsigned long long m1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < kChains; ++c) s += acc[c][threadIdx.x & 15];
  sink[blockIdx.x * 256 + threadIdx.x] = s;
  if ((threadIdx.x & 63) == 0) {
    const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
    clocks[2 * w] = m1 - m0;
    clocks[2 * w + 1] = r1 - r0;
  }
}

}  // namespace

// Run the probe once on `stream` (synchronously) with `iters` iterations per
// wave.  Outputs: elapsed milliseconds, MFMA TFLOP/s over that time, and the
// average shader clock in MHz seen by the waves.  Returns 0 or a hipError_t.
extern "C" int mt_probe_mfma(int iters, int random_operands, void* stream, float* ms_out, float* tflops_out,
                             float* mhz_out) {
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return (int)e;
  if (iters < 1 || cus < 1) return (int)hipErrorInvalidValue;
  const int blocks = 2 * cus;
  float* sink = nullptr;
  unsigned long long* clocks = nullptr;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  hipStream_t st = (hipStream_t)stream;
  e = hipMalloc(&sink, (size_t)blocks * 256 * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&clocks, (size_t)blocks * 4 * 2 * sizeof(unsigned long long));
  if (e == hipSuccess) e = hipEventCreate(&t0);
  if (e == hipSuccess) e = hipEventCreate(&t1);
  if (e == hipSuccess) e = hipEventRecord(t0, st);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(mfma_probe_kernel, dim3(blocks), dim3(256), 0, st, iters, random_operands, sink, clocks);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipEventRecord(t1, st);
  if (e == hipSuccess) e = hipEventSynchronize(t1);
  float ms = 0.f;
  if (e == hipSuccess) e = hipEventElapsedTime(&ms, t0, t1);
  double mhz = 0.0;
  if (e == hipSuccess) {
    const int waves = blocks * 4;
    unsigned long long* h = new unsigned long long[2 * waves];
    e = hipMemcpy(h, clocks, (size_t)waves * 2 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
    double sm = 0.0, sr = 0.0;
    for (int i = 0; i < waves; ++i) {
      sm += (double)h[2 * i];
      sr += (double)h[2 * i + 1];
    }
    delete[] h;
    mhz = sr > 0.0 ? sm / sr * 100.0 : 0.0;
  }
  if (t0) (void)hipEventDestroy(t0);
  if (t1) (void)hipEventDestroy(t1);
  if (sink) (void)hipFree(sink);
  if (clocks) (void)hipFree(clocks);
  if (e != hipSuccess) return (int)e;
  const double flops = (double)blocks * 4 * iters * kChains * 32768.0;
  *ms_out = ms;
  *tflops_out = (float)(flops / (ms * 1e-3) / 1e12);
  *mhz_out = (float)mhz;
  return 0;
}
