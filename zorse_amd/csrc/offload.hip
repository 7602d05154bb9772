// Copies between device memory and pinned host memory for the stage's
// activation offload, as kernels on the caller's stream.
//
// hipMemcpyAsync was measured unfit for this on gfx950 under a busy compute
// stream: device -> host it runs a copy kernel spread over every CU, which
// took CU slots from the GEMMs beside it for the whole PCIe-bound transfer
// (0.6 ms per 32 MiB); host -> device, with the copy stream waiting on the
// compute stream, the call itself blocked the host for up to ~10 ms, so no
// further work was enqueued and the GPU ran dry.  A kernel launch returns at
// once and the stream orders it like any other launch.  The transfer is
// bounded by the link (about 55 GB/s), not by the waves issuing it, so the
// copy runs from a few workgroups: each thread keeps four 16-byte accesses
// in flight (enough outstanding requests to cover the link's latency from
// 16 workgroups), and the compute kernels it overlaps keep all but those few
// CUs' worth of slots.
#include "zk_common.h"

namespace zk {

static constexpr int kCopyUnroll = 4;

__global__ __launch_bounds__(256) void copy16_kernel(const u32x4* __restrict__ src,
                                                     u32x4* __restrict__ dst, int64_t n16,
                                                     const uint8_t* __restrict__ src_tail,
                                                     uint8_t* __restrict__ dst_tail, int tail) {
  const int64_t step = static_cast<int64_t>(gridDim.x) * 256 * kCopyUnroll;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 * kCopyUnroll + threadIdx.x; i < n16;
       i += step) {
    u32x4 v[kCopyUnroll];
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int64_t j = i + 256 * u;
      if (j < n16) v[u] = src[j];
    }
#pragma unroll
    for (int u = 0; u < kCopyUnroll; ++u) {
      const int64_t j = i + 256 * u;
      if (j < n16) __builtin_nontemporal_store(v[u], dst + j);
    }
  }
  if (blockIdx.x == 0 && threadIdx.x < tail) dst_tail[threadIdx.x] = src_tail[threadIdx.x];
}

// [p, p + bytes) inside one allocation known to HIP.  Used for the pinned
// host side only: a device pointer from torch's caching allocator can sit in
// a block whose reported range (hipPointerGetAttribute) ends before the
// block does, so device extents are checked by the callers' tensor sizes.
static bool in_allocation(const void* p, int64_t bytes) {
  hipDeviceptr_t start = nullptr;
  size_t size = 0;
  if (hipPointerGetAttribute(&start, HIP_POINTER_ATTRIBUTE_RANGE_START_ADDR,
                             reinterpret_cast<hipDeviceptr_t>(const_cast<void*>(p))) != hipSuccess ||
      hipPointerGetAttribute(&size, HIP_POINTER_ATTRIBUTE_RANGE_SIZE,
                             reinterpret_cast<hipDeviceptr_t>(const_cast<void*>(p))) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  const uintptr_t a = reinterpret_cast<uintptr_t>(start), b = reinterpret_cast<uintptr_t>(p);
  return b >= a && b - a + static_cast<uint64_t>(bytes) <= size;
}

}  // namespace zk

using namespace zk;

static int copy_host(const char* what, void* dst, const void* src, int64_t bytes, int blocks,
                     bool to_host, zk_stream_t stream) {
  ZK_REQUIRE(bytes >= 0, ZK_EINVAL, "%s: negative size", what);
  if (bytes == 0) return ZK_OK;
  ZK_REQUIRE(dst && src, ZK_EINVAL, "%s: null pointer", what);
  ZK_REQUIRE(blocks >= 1 && blocks <= 1024, ZK_EINVAL, "%s: blocks %d outside [1, 1024]", what,
             blocks);
  ZK_REQUIRE(aligned(dst, 16) && aligned(src, 16), ZK_EALIGN,
             "%s: pointers must be 16-byte aligned", what);
  void* host = to_host ? dst : const_cast<void*>(src);
  const void* devp = to_host ? src : dst;
  hipPointerAttribute_t ha, da;
  const bool host_ok = hipPointerGetAttributes(&ha, host) == hipSuccess &&
                       ha.type == hipMemoryTypeHost;
  const bool dev_ok = hipPointerGetAttributes(&da, devp) == hipSuccess &&
                      da.type == hipMemoryTypeDevice;
  (void)hipGetLastError();
  ZK_REQUIRE(host_ok, ZK_EINVAL, "%s: host side is not pinned host memory", what);
  ZK_REQUIRE(dev_ok, ZK_EINVAL, "%s: device side is not device memory", what);
  ZK_REQUIRE(in_allocation(host, bytes), ZK_EINVAL,
             "%s: %lld bytes run past the end of the host allocation", what,
             static_cast<long long>(bytes));
  void* host_dev = nullptr;
  ZK_REQUIRE(hipHostGetDevicePointer(&host_dev, host, 0) == hipSuccess && host_dev, ZK_EINVAL,
             "%s: no device mapping of the host buffer", what);
  const uint8_t* s8 = reinterpret_cast<const uint8_t*>(to_host ? src : host_dev);
  uint8_t* d8 = reinterpret_cast<uint8_t*>(to_host ? host_dev : dst);
  const int64_t n16 = bytes / 16;
  const int tail = static_cast<int>(bytes - 16 * n16);
  const int64_t per_block = 256LL * kCopyUnroll;
  const int64_t need = (n16 + per_block - 1) / per_block;
  const int grid = static_cast<int>(need < blocks ? (need > 0 ? need : 1) : blocks);
  hipLaunchKernelGGL(copy16_kernel, dim3(grid), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const u32x4*>(s8), reinterpret_cast<u32x4*>(d8), n16,
                     s8 + 16 * n16, d8 + 16 * n16, tail);
  return launch_status(what);
}

extern "C" int zk_copy_to_host(void* host_dst, const void* src, int64_t bytes, int blocks,
                               zk_stream_t stream) {
  return copy_host("zk_copy_to_host", host_dst, src, bytes, blocks, true, stream);
}

extern "C" int zk_copy_from_host(void* dst, const void* host_src, int64_t bytes, int blocks,
                                 zk_stream_t stream) {
  return copy_host("zk_copy_from_host", dst, host_src, bytes, blocks, false, stream);
}
