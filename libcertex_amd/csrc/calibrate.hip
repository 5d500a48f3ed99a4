// MFMA throughput calibration for the roofline of the screens (not part of the search path).
//
// Streams of independent v_mfma_i32_16x16x64_i8 / v_mfma_f32_16x16x32_f16 instructions on
// operands held in registers, 2 waves per SIMD, no memory traffic: the rate the matrix cores
// sustain on this card. With constant operands it is the clock-limited rate; with random operands
// (every bit pattern changing from one instruction to the next, as in a screen of real rows) the
// card's power limit lowers the shader clock, and the rate falls with it. The shader clock is read
// in the kernel (s_memtime counts shader cycles, s_memrealtime a constant 100 MHz).
//
// extern "C" certex_calibrate_mfma(kind, random, out[3]): out = {ops/s, shader MHz, ms}; and
// certex_calibrate_mfma_rows(a, na, b, nb, row_bytes, out[3]): the int8 stream on stored rows.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

__device__ inline uint32_t mix(uint32_t x)
{
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

constexpr int kSlots = 8;  // independent accumulators (and operand registers) per lane

/** One timed stream: `iters` rounds of kSlots x kSlots MFMAs; operands rotate through kSlots
 * registers (random) or stay fixed. Block 0 records the shader cycles and 100 MHz ticks. */
template <bool F16, bool RANDOM>
__global__ __launch_bounds__(256, 2) void mfma_stream(int iters, float* sink,
                                                      unsigned long long* clock)
{
  v4i ra[kSlots], rb[kSlots];
  for (int i = 0; i < kSlots; ++i) {
    const uint32_t t = (blockIdx.x * 256u + threadIdx.x) * 64u + uint32_t(i) * 8u;
    for (int j = 0; j < 4; ++j) {
      uint32_t a = RANDOM ? mix(t + j) : 0x01020304u, b = RANDOM ? mix(t + 4 + j) : 0x03010207u;
      if constexpr (F16) {
        a &= 0xbfffbfffu;  // finite halves of magnitude < 2: no overflow over the stream
        b &= 0xbfffbfffu;
      }
      ra[i][j] = int(a);
      rb[i][j] = int(b);
    }
  }
  v4i acc_i[kSlots];
  v4f acc_f[kSlots];
  for (int i = 0; i < kSlots; ++i) {
    acc_i[i] = v4i{0, 0, 0, 0};
    acc_f[i] = v4f{0, 0, 0, 0};
  }
  const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
#pragma unroll
      for (int i = 0; i < kSlots; ++i) {
        const v4i a = ra[i], b = rb[(i + j) % kSlots];
        if constexpr (F16) {
          acc_f[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a),
                                                            __builtin_bit_cast(v8h, b), acc_f[i],
                                                            0, 0, 0);
        } else {
          acc_i[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc_i[i], 0, 0, 0);
        }
      }
    }
  }
  const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.0f;
  for (int i = 0; i < kSlots; ++i) {
    for (int j = 0; j < 4; ++j) { s += F16 ? acc_f[i][j] : float(acc_i[i][j]); }
  }
  sink[blockIdx.x * 256 + threadIdx.x] = s;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    clock[0] = c1 - c0;
    clock[1] = r1 - r0;
  }
}

/** The int8 stream on operands taken from stored data: slot i of a lane holds the 16-byte piece
 * (lane / 16) of row (16 i + lane % 16 + a block offset) of A (rows of row_bytes bytes; the first
 * 64 bytes of each row), and likewise of B; the MFMA fragments of a screen over those rows. */
__global__ __launch_bounds__(256, 2) void mfma_rows_stream(const int8_t* A, int64_t na,
                                                           const int8_t* B, int64_t nb,
                                                           int row_bytes, int iters, float* sink,
                                                           unsigned long long* clock)
{
  const int lane = threadIdx.x & 63;
  const int64_t base =
      (int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6)) * 16 * kSlots + (lane & 15);
  v4i ra[kSlots], rb[kSlots];
  for (int i = 0; i < kSlots; ++i) {
    const int64_t r = base + 16 * i;
    ra[i] = *reinterpret_cast<const v4i*>(A + (r % na) * row_bytes + (lane >> 4) * 16);
    rb[i] = *reinterpret_cast<const v4i*>(B + ((r * 7) % nb) * row_bytes + (lane >> 4) * 16);
  }
  v4i acc[kSlots];
  for (int i = 0; i < kSlots; ++i) { acc[i] = v4i{0, 0, 0, 0}; }
  const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < kSlots; ++j) {
#pragma unroll
      for (int i = 0; i < kSlots; ++i) {
        acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ra[i], rb[(i + j) % kSlots], acc[i], 0, 0, 0);
      }
    }
  }
  const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.0f;
  for (int i = 0; i < kSlots; ++i) {
    for (int j = 0; j < 4; ++j) { s += float(acc[i][j]); }
  }
  sink[blockIdx.x * 256 + threadIdx.x] = s;
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    clock[0] = c1 - c0;
    clock[1] = r1 - r0;
  }
}

template <bool F16, bool RANDOM>
void launch(int blocks, int iters, float* sink, unsigned long long* clock, hipStream_t s)
{
  mfma_stream<F16, RANDOM><<<blocks, 256, 0, s>>>(iters, sink, clock);
}

/** Times run(s) once after a warm-up launch; fills out[] as certex_calibrate_mfma does. */
template <typename Run>
int timed_stream(Run run, int blocks, int iters, double per_mfma, double* out)
{
  hipError_t e = hipSuccess;
  hipStream_t s = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  float* sink = nullptr;
  unsigned long long* clock = nullptr;
  if ((e = hipMalloc(&sink, size_t(blocks) * 256 * sizeof(float))) != hipSuccess) { return int(e); }
  if ((e = hipMalloc(&clock, 2 * sizeof(unsigned long long))) != hipSuccess) {
    (void)hipFree(sink);
    return int(e);
  }
  float ms                = 0.0f;
  unsigned long long c[2] = {0, 1};
  if ((e = hipEventCreate(&e0)) == hipSuccess && (e = hipEventCreate(&e1)) == hipSuccess) {
    run(sink, clock, s);  // warm-up (clocks ramp)
    e = hipEventRecord(e0, s);
    if (e == hipSuccess) {
      run(sink, clock, s);
      e = hipEventRecord(e1, s);
    }
    if (e == hipSuccess) { e = hipEventSynchronize(e1); }
    if (e == hipSuccess) { e = hipGetLastError(); }
    if (e == hipSuccess) { e = hipEventElapsedTime(&ms, e0, e1); }
    if (e == hipSuccess) { e = hipMemcpy(c, clock, sizeof(c), hipMemcpyDeviceToHost); }
  }
  if (e0 != nullptr) { (void)hipEventDestroy(e0); }
  if (e1 != nullptr) { (void)hipEventDestroy(e1); }
  (void)hipFree(sink);
  (void)hipFree(clock);
  if (e != hipSuccess) { return int(e); }
  const double mfmas = double(blocks) * 4 * double(iters) * kSlots * kSlots;
  out[0]             = mfmas * per_mfma / (double(ms) * 1e-3);
  out[1]             = double(c[0]) / double(c[1]) * 100.0;
  out[2]             = double(ms);
  return 0;
}

int stream_blocks(int* blocks)
{
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) { e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev); }
  *blocks = cus * 2 * 8;  // 2 workgroups of 4 waves per CU, 8 rounds
  return int(e);
}

}  // namespace

/**
 * kind 0: int8 (16x16x64), 1: fp16 (16x16x32); random 0/1. out[0] = dense ops per second,
 * out[1] = shader clock in MHz over block 0's stream, out[2] = milliseconds of the timed launch.
 * Returns 0, or the HIP error code.
 */
extern "C" __attribute__((visibility("default"))) int certex_calibrate_mfma(int kind, int random,
                                                                            double* out)
{
  int blocks = 0;
  if (const int e = stream_blocks(&blocks); e != 0) { return e; }
  const int iters = 2000;
  auto run        = [&](float* sink, unsigned long long* clock, hipStream_t s) {
    if (kind == 1) {
      random ? launch<true, true>(blocks, iters, sink, clock, s)
             : launch<true, false>(blocks, iters, sink, clock, s);
    } else {
      random ? launch<false, true>(blocks, iters, sink, clock, s)
             : launch<false, false>(blocks, iters, sink, clock, s);
    }
  };
  return timed_stream(run, blocks, iters, kind == 1 ? 2.0 * 16 * 16 * 32 : 2.0 * 16 * 16 * 64, out);
}

/**
 * The int8 stream on operands from device memory: a (na rows) and b (nb rows) of row_bytes bytes
 * each (row_bytes >= 64), already in the signed form the screen multiplies (uint8 codes ^ 0x80).
 * out[] as for certex_calibrate_mfma. Returns 0, or the HIP error code (hipErrorInvalidValue for
 * bad sizes).
 */
extern "C" __attribute__((visibility("default"))) int certex_calibrate_mfma_rows(
    const void* a, int64_t na, const void* b, int64_t nb, int row_bytes, double* out)
{
  if (a == nullptr || b == nullptr || na <= 0 || nb <= 0 || row_bytes < 64 || row_bytes % 16 != 0) {
    return int(hipErrorInvalidValue);
  }
  int blocks = 0;
  if (const int e = stream_blocks(&blocks); e != 0) { return e; }
  const int iters = 2000;
  auto run        = [&](float* sink, unsigned long long* clock, hipStream_t s) {
    mfma_rows_stream<<<blocks, 256, 0, s>>>(static_cast<const int8_t*>(a), na,
                                            static_cast<const int8_t*>(b), nb, row_bytes, iters,
                                            sink, clock);
  };
  return timed_stream(run, blocks, iters, 2.0 * 16 * 16 * 64, out);
}
