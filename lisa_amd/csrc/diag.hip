// Measurement aid (no counterpart in the reference): a read-only stream of a
// buffer, the memory side of the matvec kernels without any of their work.
// Wave w of the grid reads L consecutive 1 KB pieces (lane l: 16 bytes at
// 1024 * (w * L + i) + 16 * l), nontemporal, as the weight loads of the
// matvec kernels do; the pieces' XOR goes to *sink only when it equals a
// value no buffer of ones can produce, so the loads cannot be dropped and
// nothing is written.  bench.py --read-floor times it in the same graph
// replay as the matvec to give the floor a kernel of that size can reach.
#include "lisaq_common.h"
#include "qmv_dev.h"

namespace lisaq {

using namespace qmvdev;

template <int L>
__global__ __launch_bounds__(256) void read_stream_kernel(const unsigned char* src, uint32_t bytes, uint32_t* sink) {
  const __amdgpu_buffer_rsrc_t r = make_rsrc(src, bytes);
  const uint32_t lane = threadIdx.x & 63, w = blockIdx.x * 4 + (threadIdx.x >> 6);
  u32x4 v[L];
#pragma unroll
  for (int i = 0; i < L; ++i)
    v[i] = __builtin_bit_cast(u32x4,
                              __builtin_amdgcn_raw_buffer_load_b128(r, ((w * L + i) * 64 + lane) * 16, 0, kNt));
  u32x4 acc = v[0];
#pragma unroll
  for (int i = 1; i < L; ++i) acc ^= v[i];
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x9E3779B9u) sink[0] = acc[0];
}

int launch_read_stream(hipStream_t st, const void* src, size_t bytes, int loads_per_lane, uint32_t* sink) {
  if (bytes == 0) return LISAQ_OK;
  if (bytes >= ((size_t)1 << 31) || bytes % 16)
    return set_error(LISAQ_EINVAL_SHAPE, "read_stream: %zu bytes (a multiple of 16 below 2 GiB)", bytes);
  typedef void (*fn_t)(const unsigned char*, uint32_t, uint32_t*);
  fn_t fn = loads_per_lane == 1 ? read_stream_kernel<1>
            : loads_per_lane == 2 ? read_stream_kernel<2>
            : loads_per_lane == 4 ? read_stream_kernel<4>
            : loads_per_lane == 8 ? read_stream_kernel<8>
            : loads_per_lane == 16 ? read_stream_kernel<16> : nullptr;
  if (!fn) return set_error(LISAQ_EINVAL_SHAPE, "read_stream: loads per lane %d (1, 2, 4, 8 or 16)", loads_per_lane);
  const size_t per_block = (size_t)4 * 1024 * loads_per_lane;
  hipLaunchKernelGGL(fn, dim3((unsigned)((bytes + per_block - 1) / per_block)), dim3(256), 0, st,
                     (const unsigned char*)src, (uint32_t)bytes, sink);
  return check_launch("read_stream");
}

// The GPU's constant 100 MHz clock (s_memrealtime), stored by one lane:
// stream-ordered, so two of them around a run of kernels time that run on the
// device, without the host's submission of it (bench.py brackets the timed
// graph's steps with them inside the graph).
__global__ __launch_bounds__(64) void timestamp_kernel(uint64_t* dst) {
  const uint64_t t = __builtin_amdgcn_s_memrealtime();
  if (threadIdx.x == 0) dst[0] = t;
}

int launch_timestamp(hipStream_t st, uint64_t* dst) {
  hipLaunchKernelGGL(timestamp_kernel, dim3(1), dim3(64), 0, st, dst);
  return check_launch("timestamp");
}

}  // namespace lisaq
