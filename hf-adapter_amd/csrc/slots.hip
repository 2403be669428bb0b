// Recurrent-state slot copies for the serving state pool
// (docs/integrations/RWKV7_STATE_CACHE_ABI.md:52-133: layer-major pools
// S_pool [L, capacity, H, N, N], xpa / xpf [L, capacity, D], v_first
// [capacity, A]; gather / scatter / clone / reset of scheduled slots).
//
// One launch moves rows of every layer: row r of layer l goes from
//   src + l * src_layer_stride + src_rows[r] * src_row_stride
// to
//   dst + l * dst_layer_stride + dst_rows[r] * dst_row_stride
// (strides in bytes; a null row-index array means the identity), skipping
// rows whose active flag is 0, and writing zeros when src is null.  A row is
// row_bytes long (a multiple of 16, 16-byte aligned): each thread moves 16
// bytes per pass with plain vector loads and stores.  Grid: (row chunks,
// rows, layers).  Byte copies, no arithmetic.
#include "common.h"

namespace rwkv7mi {

struct SlotCopy {
  const char* src;
  char* dst;
  const int64_t* src_rows;
  const int64_t* dst_rows;
  const uint8_t* active;
  int64_t src_layer, dst_layer, src_row, dst_row;
  int64_t row16;  // 16-byte units per row
};

__global__ __launch_bounds__(256) void slot_copy_kernel(const SlotCopy C) {
  const int64_t r = blockIdx.y;
  const int64_t l = blockIdx.z;
  if (C.active && !C.active[r]) return;
  const int64_t sr = C.src_rows ? C.src_rows[r] : r;
  const int64_t dr = C.dst_rows ? C.dst_rows[r] : r;
  uint4* d = reinterpret_cast<uint4*>(C.dst + l * C.dst_layer + dr * C.dst_row);
  const uint4* s = C.src ? reinterpret_cast<const uint4*>(C.src + l * C.src_layer + sr * C.src_row) : nullptr;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < C.row16; i += (int64_t)gridDim.x * 256)
    d[i] = s ? s[i] : make_uint4(0u, 0u, 0u, 0u);
}

}  // namespace rwkv7mi

using namespace rwkv7mi;

extern "C" int rwkv7mi_slot_copy(const void* src, int64_t src_layer_stride, int64_t src_row_stride,
                                 const int64_t* src_rows, void* dst, int64_t dst_layer_stride,
                                 int64_t dst_row_stride, const int64_t* dst_rows, const uint8_t* active,
                                 int64_t nrows, int64_t row_bytes, int64_t nlayers, void* stream) {
  if (nrows < 0 || nlayers < 0 || row_bytes <= 0 || row_bytes % 16)
    return fail(RWKV7MI_EINVAL, "slot_copy: row_bytes must be a positive multiple of 16");
  if (nrows == 0 || nlayers == 0) return RWKV7MI_OK;
  if (!dst) return fail(RWKV7MI_EINVAL, "slot_copy: null destination");
  if (nrows > 65535 || nlayers > 65535) return fail(RWKV7MI_EINVAL, "slot_copy: at most 65535 rows and layers");
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst) | (uintptr_t)src_layer_stride |
       (uintptr_t)src_row_stride | (uintptr_t)dst_layer_stride | (uintptr_t)dst_row_stride) & 15)
    return fail(RWKV7MI_EINVAL, "slot_copy: pointers and strides must be 16-byte aligned");
  SlotCopy c{reinterpret_cast<const char*>(src), reinterpret_cast<char*>(dst), src_rows, dst_rows, active,
             src_layer_stride, dst_layer_stride, src_row_stride, dst_row_stride, row_bytes / 16};
  const int64_t chunks = std::min<int64_t>((c.row16 + 255) / 256, 64);
  hipLaunchKernelGGL(slot_copy_kernel, dim3((unsigned)chunks, (unsigned)nrows, (unsigned)nlayers), dim3(256), 0,
                     as_stream(stream), c);
  return check_launch("slot_copy_kernel");
}
