// lds_patterns.hip - the LDS access patterns of the large-tile prefill GEMM
// (gemm_q4_big_kernel), each alone in a kernel of the same shape (256
// workgroups of 512 threads, 32 steps), for attributing SQ_LDS_BANK_CONFLICT:
//   a_reads<1>  the activation reads, chunks swizzled by bits 1..3 of the row
//               (the kernel's form);
//   a_reads<0>  the same, swizzled by the row's low three bits;
//   a_reads<2>  the same, unswizzled (16 rows of a read on one chunk);
//   code_reads  the code and gain reads of read_codes;
//   mfma_only   the step's 64 products on register operands;
//   a_dma       the activation DMA (global_load_lds, 16 bytes a lane).
// Build and count (repo root):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//     tests/probes/lds_patterns.hip -o /tmp/lds_patterns
//   rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_INSTS_LDS SQ_INSTS_MFMA \
//     --output-format csv -d gpurun_out/lds_patterns -o pmc -- /tmp/lds_patterns
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <cstdint>
#define CK(...) do { hipError_t e_ = (__VA_ARGS__); if (e_ != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1); } } while (0)
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));
typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;
constexpr int kSteps = 32;
// A reads: 8 row tiles x 2 k-halves of 16 bytes a lane, rows r = wm*128 + 16 i + n, chunk (2 gq + q) ^ swz(r)
template <int SWZ>
__global__ __launch_bounds__(512) void a_reads(uint32_t *out) {
  __shared__ __attribute__((aligned(16))) _Float16 as[256 * 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave >> 2, gq = lane >> 4, n = lane & 15;
  for (int i = tid; i < 256 * 64; i += 512) as[i] = (_Float16)(i & 7);
  __syncthreads();
  uint32_t x = 0;
  for (int s = 0; s < kSteps; ++s) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int r = wm * 128 + 16 * i + n;
        const int p = SWZ == 2 ? 2 * gq + q : (2 * gq + q) ^ (SWZ ? ((r >> 1) & 7) : (r & 7));
        const half8_t v = *reinterpret_cast<const half8_t *>(as + r * 64 + 8 * p);
        const uint4_t u = __builtin_bit_cast(uint4_t, v);
        x ^= (u[0] + u[1]) ^ (u[2] + u[3]) ^ s;
      }
    __builtin_amdgcn_s_barrier();
  }
  out[blockIdx.x * 512 + tid] = x;
}
// code and gain reads as read_codes issues them
__global__ __launch_bounds__(512) void code_reads(uint32_t *out) {
  __shared__ __attribute__((aligned(16))) uint8_t st[256 * 32 + 256 * 8];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wn = wave & 3, gq = lane >> 4, n = lane & 15;
  for (int i = tid; i < (int)sizeof(st) / 4; i += 512) reinterpret_cast<uint32_t *>(st)[i] = i;
  __syncthreads();
  uint32_t x = 0;
  const float *gs = reinterpret_cast<const float *>(st + 256 * 32);
  for (int s = 0; s < kSteps; ++s) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = wn * 64 + 16 * j + n;
      const int half = (gq >> 1) ^ ((n >> 3) & 1);
      const uint2_t b = *reinterpret_cast<const uint2_t *>(st + row * 32 + 16 * half + 8 * (gq & 1));
      x ^= b[0] + b[1] + __float_as_uint(gs[row * 2 + (gq >> 1)]) + s;
    }
    __builtin_amdgcn_s_barrier();
  }
  out[blockIdx.x * 512 + tid] = x;
}
// 64 MFMAs a step on register operands, no LDS
__global__ __launch_bounds__(512) void mfma_only(float *out) {
  const int tid = threadIdx.x;
  half8_t a, b;
  for (int e = 0; e < 8; ++e) { a[e] = (_Float16)(tid & 3); b[e] = (_Float16)(e); }
  float4_t acc[8][4];
  for (int i = 0; i < 8; ++i) for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0, 0, 0, 0};
  for (int s = 0; s < kSteps; ++s) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(b, a, acc[i][j], 0, 0, 0);
  }
  float t = 0;
  for (int i = 0; i < 8; ++i) for (int j = 0; j < 4; ++j) t += acc[i][j][0];
  out[blockIdx.x * 512 + tid] = t;
}
// the activation DMA: four 16-byte global_load_lds a wave a step into 1 KB slabs
__global__ __launch_bounds__(512) void a_dma(const _Float16 *src, uint32_t *out) {
  __shared__ __attribute__((aligned(16))) uint8_t st[3 * 32768];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = 2048;
  for (int s = 0; s < kSteps; ++s) {
    uint8_t *dst = st + (s % 3) * 32768;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 8 * (4 * wave + i) + (lane >> 3);
      const int c = (lane & 7) ^ ((r >> 1) & 7);
      const _Float16 *p = src + (size_t)(blockIdx.x % 8 * 256 + r) * K + 64 * s + 8 * c;
      __builtin_amdgcn_global_load_lds((global_void_t *)p, (lds_void_t *)(dst + (4 * wave + i) * 1024), 16, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0x0070);
    __builtin_amdgcn_s_barrier();
  }
  out[blockIdx.x * 512 + tid] = reinterpret_cast<uint32_t *>(st)[tid];
}
int main() {
  uint32_t *out; _Float16 *src;
  CK(hipMalloc(&out, 256 * 512 * 4)); CK(hipMalloc(&src, (size_t)2048 * 2048 * 2)); CK(hipMemset(src, 0, (size_t)2048 * 2048 * 2));
  for (int rep = 0; rep < 3; ++rep) {
    hipLaunchKernelGGL((a_reads<1>), dim3(256), dim3(512), 0, 0, out);
    hipLaunchKernelGGL((a_reads<0>), dim3(256), dim3(512), 0, 0, out);
    hipLaunchKernelGGL((a_reads<2>), dim3(256), dim3(512), 0, 0, out);
    hipLaunchKernelGGL(code_reads, dim3(256), dim3(512), 0, 0, out);
    hipLaunchKernelGGL(mfma_only, dim3(256), dim3(512), 0, 0, (float *)out);
    hipLaunchKernelGGL(a_dma, dim3(256), dim3(512), 0, 0, src, out);
    CK(hipGetLastError());
  }
  CK(hipDeviceSynchronize());
  printf("lds patterns done\n");
  return 0;
}
