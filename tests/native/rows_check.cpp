// Host build of opfoundry_amd/csrc/dsa_rows.h (the kernels' index rules) for
// tests/test_rows_cpu.py: the two HIP qualifiers are defined empty, so g++
// compiles exactly the functions the device code runs.
#define __host__
#define __device__
#include "../../opfoundry_amd/csrc/dsa_rows.h"

extern "C" {

int32_t rows_v4_prefix(int32_t j, int64_t rows) { return dsa_rows::v4_prefix_row(j, rows); }
int32_t rows_v4_extend(int32_t j, int64_t rows) { return dsa_rows::v4_extend_row(j, rows); }
int32_t rows_csr(int32_t j, int64_t rows) { return dsa_rows::csr_row(j, rows); }
int rows_in_pool2(int32_t id) { return dsa_rows::row_in_pool2(id) ? 1 : 0; }
int32_t rows_index(int32_t id) { return dsa_rows::row_index(id); }
int64_t rows_max_pool(void) { return dsa_rows::MAX_POOL_ROWS; }
int64_t rows_topk(int32_t j, int64_t jmax, const int32_t* bt_row, int32_t block_size, int32_t bs_shift,
                  int64_t flat_base, int64_t rows) {
    return dsa_rows::topk_row(j, jmax, bt_row, block_size, bs_shift, flat_base, rows);
}

// The V4 list a workgroup compacts: prefix entries then extend entries,
// each resolved against its own pool, skipped rows dropped.  Writes the
// (pool, row) pair the gather would read for every kept entry; returns the
// count.
int rows_v4_list(const int32_t* pre, int n_pre, const int32_t* ext, int n_ext, int64_t pages, int64_t tokens,
                 int32_t* pool_out, int32_t* row_out) {
    int n = 0;
    for (int k = 0; k < n_pre + n_ext; ++k) {
        const bool e = k >= n_pre;
        const int32_t id = e ? dsa_rows::v4_extend_row(ext[k - n_pre], tokens) : dsa_rows::v4_prefix_row(pre[k], pages);
        if (id < 0) continue;
        pool_out[n] = dsa_rows::row_in_pool2(id) ? 2 : 1;
        row_out[n] = dsa_rows::row_index(id);
        ++n;
    }
    return n;
}

}
