// dsa_gather_floor.hip - measurement probe, built as libdsa_gather_floor.so
// (not part of libdsa_mla.so and not a drop-in entry point).
//
// It moves a decode step's gathered latent rows from HBM into LDS exactly as
// the forward kernels do (16-byte LDS-DMA loads, 32-row tiles, a ring of tile
// slots, 256 threads per query token) and does no attention work, so its run
// time is the memory floor of the step's gather.  The rows are given as a
// flat list of physical row ids per query token (block tables already
// applied); each workgroup folds every 32-bit word it gathered into a sum per
// token, which the caller checks against the same sum taken on the host side
// (it proves every byte landed and keeps the loads live).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dsa_lds.h"

namespace {

constexpr int NTHREADS = 256;
constexpr int NWAVE = NTHREADS / 64;
constexpr int TILE_ROWS = 32;
constexpr int MAX_ROWS = 2048;   // row ids of one token staged in LDS

// One tile of ROW_BYTES-wide rows is 32 * ROW_BYTES / 16 pieces of 16 bytes;
// every wave issues LOADS LDS-DMA instructions per tile (64 pieces each), the
// pieces past the tile's end load row 0 into the slot's padding, so the
// per-wave vmcnt count of a tile is the same constant for every wave.
template <int ROW_BYTES>
struct TileShape {
    static_assert(ROW_BYTES % 16 == 0, "rows are whole 16-byte pieces");
    static constexpr int PIECES_PER_ROW = ROW_BYTES / 16;
    static constexpr int PIECES = TILE_ROWS * PIECES_PER_ROW;
    static constexpr int LOADS = (PIECES + NTHREADS - 1) / NTHREADS;
    static constexpr int SLOT_BYTES = LOADS * NTHREADS * 16;
};

template <int ROW_BYTES, int SLOTS>
__global__ __launch_bounds__(NTHREADS) void dsa_gather_floor_kernel(
    const uint8_t* __restrict__ kv, const int32_t* __restrict__ rows, int nrows,
    uint32_t* __restrict__ sums) {
    using T = TileShape<ROW_BYTES>;
    constexpr int AHEAD = SLOTS - 1;
    extern __shared__ __align__(16) uint8_t smem[];
    int32_t* row_ids = reinterpret_cast<int32_t*>(smem);
    lds_ptr slots = (lds_ptr)(smem + MAX_ROWS * 4);

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int32_t* list = rows + (int64_t)blockIdx.x * nrows;
    {   // all of a thread's row ids are loaded before any is stored: one memory round trip
        constexpr int PER = MAX_ROWS / NTHREADS;
        int32_t v[PER];
#pragma unroll
        for (int k = 0; k < PER; ++k) v[k] = tid + k * NTHREADS < nrows ? list[tid + k * NTHREADS] : 0;
#pragma unroll
        for (int k = 0; k < PER; ++k)
            if (tid + k * NTHREADS < nrows) row_ids[tid + k * NTHREADS] = v[k];
    }
    __syncthreads();
    const int ntiles = nrows / TILE_ROWS;

    auto issue = [&](int t) {
        lds_ptr slot = slots + (t % SLOTS) * T::SLOT_BYTES;
        const uint8_t* src[T::LOADS];
#pragma unroll
        for (int k = 0; k < T::LOADS; ++k) {    // every row id is read before the first load issues
            const int piece = (k * NWAVE + w) * 64 + lane;
            const bool in_tile = piece < T::PIECES;
            const int r = in_tile ? piece / T::PIECES_PER_ROW : 0;
            const int off = in_tile ? (piece - r * T::PIECES_PER_ROW) * 16 : 0;
            src[k] = kv + (int64_t)row_ids[t * TILE_ROWS + r] * ROW_BYTES + off;
        }
#pragma unroll
        for (int k = 0; k < T::LOADS; ++k) lds_dma16(src[k], slot + (k * NWAVE + w) * 1024);
    };

    uint32_t sum = 0;
    for (int t = 0; t < AHEAD && t < ntiles; ++t) issue(t);
    for (int t = 0; t < ntiles; ++t) {
        if (t + AHEAD < ntiles) {
            issue(t + AHEAD);
            wait_vm<T::LOADS * AHEAD>();     // tile t's loads of this wave have landed
        } else {
            wait_vm<0>();
        }
        tile_barrier();                      // ... and every other wave's
        lds_cptr slot = slots + (t % SLOTS) * T::SLOT_BYTES;
#pragma unroll
        for (int k = 0; k < T::LOADS; ++k) {
            const int piece = (k * NWAVE + w) * 64 + lane;
            if (piece < T::PIECES) {
                const u32x4 v = lds_ld<u32x4>(slot + (k * NWAVE + w) * 1024 + lane * 16);
                sum += v.x + v.y + v.z + v.w;
            }
        }
        tile_barrier();                      // slot t is read before tile t + SLOTS refills it
    }

    for (int m = 32; m >= 1; m >>= 1) sum += __shfl_xor(sum, m);
    __syncthreads();
    uint32_t* wsum = reinterpret_cast<uint32_t*>(smem);
    if (lane == 0) wsum[w] = sum;
    __syncthreads();
    if (tid == 0) sums[blockIdx.x] = wsum[0] + wsum[1] + wsum[2] + wsum[3];
}

template <int ROW_BYTES, int SLOTS>
hipError_t launch(const void* kv, const int32_t* rows, int ntok, int nrows, uint32_t* sums,
                  hipStream_t st) {
    using T = TileShape<ROW_BYTES>;
    const size_t lds = MAX_ROWS * 4 + (size_t)SLOTS * T::SLOT_BYTES;
    auto k = dsa_gather_floor_kernel<ROW_BYTES, SLOTS>;
    hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k, dim3(ntok), dim3(NTHREADS), lds, st,
                       static_cast<const uint8_t*>(kv), rows, nrows, sums);
    return hipGetLastError();
}

}  // namespace

extern "C" {

// Gather nrows rows of row_bytes (656: fp8 rows, 1152: bf16 rows) for each of
// ntok query tokens; rows[ntok][nrows] are physical row ids into kv, nrows a
// multiple of 32 and at most 2048; slots = tiles in LDS at once (2..4).
// sums[tok] = sum of the gathered 32-bit words modulo 2^32.
// Returns 0, or -1 for arguments outside those limits, or a hipError_t.
int dsa_gather_floor(const void* kv, const int32_t* rows, int ntok, int nrows, int row_bytes,
                     int slots, uint32_t* sums, void* stream) {
    if (!kv || !rows || !sums || ntok <= 0 || nrows <= 0 || nrows > MAX_ROWS ||
        nrows % TILE_ROWS != 0)
        return -1;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (row_bytes == 656) {
        if (slots == 2) return launch<656, 2>(kv, rows, ntok, nrows, sums, st);
        if (slots == 3) return launch<656, 3>(kv, rows, ntok, nrows, sums, st);
        if (slots == 4) return launch<656, 4>(kv, rows, ntok, nrows, sums, st);
    } else if (row_bytes == 1152) {
        if (slots == 2) return launch<1152, 2>(kv, rows, ntok, nrows, sums, st);
        if (slots == 3) return launch<1152, 3>(kv, rows, ntok, nrows, sums, st);
    }
    return -1;
}

}  // extern "C"
