// dsa_rows.h - the rules that turn an index-list entry into a physical cache
// row, shared by the forward kernel (device) and its CPU unit test (host).
//
// Every rule returns a row id >= 0 for an entry the attention must read and
// -1 for one it must skip, and checks the row against the pool it will be
// read from, so no accepted entry can address memory outside its pool.
//
// Row ids name a pool as well as a row: bit 30 (POOL2) tags a row of the
// second pool (the V4 extend rows), the low 30 bits hold the row.  A pool
// is therefore limited to MAX_POOL_ROWS rows, which the host entry points
// check before any launch.  Only v4_extend_row() sets the tag, and only on
// an id it has checked against the second pool, so a first-pool id (however
// large) can never be taken for a second-pool row.
//
// hipcc compiles these for host and device; a host-only test defines
// __host__ and __device__ as empty before including this file.
#ifndef DSA_ROWS_H_
#define DSA_ROWS_H_

#include <stdint.h>

namespace dsa_rows {

constexpr int32_t POOL2 = 1 << 30;            // row-id tag: a row of the second pool
constexpr int64_t MAX_POOL_ROWS = POOL2;      // rows a pool may hold (ids below 2^30)

__host__ __device__ inline bool row_in_pool2(int32_t id) { return (id & POOL2) != 0; }
__host__ __device__ inline int32_t row_index(int32_t id) { return id & (POOL2 - 1); }

// V4 prefill, prefix list: id j is row j of the first pool (unified_kv)
// when 0 <= j < rows (mla_v4_host.cc:482-532 reads it unchecked; a row
// outside the pool is skipped here).
__host__ __device__ inline int32_t v4_prefix_row(int32_t j, int64_t rows) {
    return j >= 0 && (int64_t)j < rows ? j : -1;
}

// V4 prefill, extend list: id j is row j of the second pool (kv), tagged.
__host__ __device__ inline int32_t v4_extend_row(int32_t j, int64_t rows) {
    return j >= 0 && (int64_t)j < rows ? (j | POOL2) : -1;
}

// CSR form (page size 1): kv_indices holds physical rows
// (opus_attn/dsa_v32/common/host.cc:482,526).
__host__ __device__ inline int32_t csr_row(int32_t j, int64_t rows) {
    return j >= 0 && (int64_t)j < rows ? j : -1;
}

// Top-k form: logical position j of a sequence whose valid positions are
// [0, jmax) (jmax folds in seq_len and the causal bound).  Paged: bt_row is
// the sequence's block-table row, the physical row is
// bt_row[j / block_size] * block_size + j % block_size (bs_shift =
// log2(block_size) for a power of two, else -1).  Flat (bt_row == NULL):
// flat_base + j.  A physical row outside [0, rows) is skipped, so a bad
// block table cannot address memory outside the cache.
//
// The rule in two steps, so that a caller resolving several entries can
// issue all their block-table reads before it waits for any: topk_block()
// gives the block-table slot of position j (-1: j is skipped), topk_finish()
// the row from that slot's entry (read only when paged).
__host__ __device__ inline int32_t topk_block(int32_t j, int64_t jmax, int32_t block_size, int32_t bs_shift) {
    if (j < 0 || (int64_t)j >= jmax) return -1;
    return bs_shift >= 0 ? (j >> bs_shift) : (j / block_size);
}
__host__ __device__ inline int64_t topk_finish(int32_t j, int32_t blk_i, int32_t bt_entry, bool paged,
                                               int32_t block_size, int32_t bs_shift, int64_t flat_base,
                                               int64_t rows) {
    if (blk_i < 0) return -1;
    int64_t row;
    if (paged) {
        const int32_t in_blk = bs_shift >= 0 ? (j & (block_size - 1)) : (j % block_size);
        row = (int64_t)bt_entry * block_size + in_blk;
    } else {
        row = flat_base + j;
    }
    return row >= 0 && row < rows ? row : -1;
}
__host__ __device__ inline int64_t topk_row(int32_t j, int64_t jmax, const int32_t* bt_row, int32_t block_size,
                                            int32_t bs_shift, int64_t flat_base, int64_t rows) {
    const int32_t blk = topk_block(j, jmax, block_size, bs_shift);
    return topk_finish(j, blk, bt_row && blk >= 0 ? bt_row[blk] : 0, bt_row != nullptr, block_size, bs_shift,
                       flat_base, rows);
}

}  // namespace dsa_rows

#endif  // DSA_ROWS_H_
