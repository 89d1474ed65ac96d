// Host entry of the many-row quantized matmul kernel (qgemm.hip), used by the
// dequant-matmul C-ABI (qmatmul.hip) when M is large enough.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mkq {

// Workspace layout when K is split: [0, kQgPartOffset) per-tile arrival
// counters (zero between calls; the same region the wide int4 kernel uses),
// then the f32 partial tiles.
constexpr int kQgCounters = 16384;
constexpr int64_t kQgPartOffset = 64 * 1024;

// K % 64 == 0 and N % 128 == 0 (the kernel's 64 x 128 weight tile).
bool qgemm_supported(int64_t M, int64_t K, int64_t N);

// The K split the kernel uses for this shape: 2 when the grid would
// otherwise hold fewer than 192 tiles and the partials fit workspace_cap
// bytes, else 1 (MK_QG_KS=1 / 2 forces it, within the same limits).
int qgemm_ks(int64_t M, int64_t K, int64_t N, int64_t workspace_cap);

// Workspace bytes for that split (0 for ks == 1).
int64_t qgemm_workspace_bytes(int64_t M, int64_t K, int64_t N, int ks);

// int4: w uint8 [K/2, N], s bf16 [K/64, N], z uint8 [K/64, N];
// int8: w int8 [K, N], s f32 [N], z unused.  x bf16 [M, K], y bf16 [M, N].
// aux / epi: the bf16 store epilogue (epilogue.h), MK_EPI_NONE for none.
// ks > 1 needs qgemm_workspace_bytes of workspace with zeroed counters.
// xch_local: the caller has seen the dispatcher deal workgroups to the XCDs
// round-robin on this device, so a tile's K parts (consecutive logical ids)
// share one XCD when qgemm_tile_on_one_xcd holds for the grid, and the
// split-K exchange can stay in that XCD's L2.
hipError_t qgemm_launch(bool int4, const void* x, const void* w, const void* s, const void* z, void* y, int64_t M,
                        int64_t K, int64_t N, const void* aux, int epi, int ks, void* workspace,
                        hipStream_t stream, bool xch_local);

// Workgroups of the kernel's grid for this shape and split.
unsigned qgemm_grid(int64_t M, int64_t N, int ks);

// Whether a grid of gx workgroups keeps each tile's ks K parts on one XCD
// under round-robin dealing (see xcd_logical_id).
bool qgemm_tile_on_one_xcd(unsigned gx, int ks);

}  // namespace mkq
