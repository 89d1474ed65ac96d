// Host entry of the many-row quantized matmul kernel (qgemm.hip), used by the
// dequant-matmul C-ABI (qmatmul.hip) when M is large enough.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mkq {

// K % 64 == 0 and N % 64 == 0 (the kernel's 64 x 64 weight tile).
bool qgemm_supported(int64_t M, int64_t K, int64_t N);

// int4: w uint8 [K/2, N], s bf16 [K/64, N], z uint8 [K/64, N];
// int8: w int8 [K, N], s f32 [N], z unused.  x bf16 [M, K], y bf16 [M, N].
// aux / epi: the bf16 store epilogue (epilogue.h), MK_EPI_NONE for none.
hipError_t qgemm_launch(bool int4, const void* x, const void* w, const void* s, const void* z, void* y, int64_t M,
                        int64_t K, int64_t N, const void* aux, int epi, hipStream_t stream);

}  // namespace mkq
