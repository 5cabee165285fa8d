// runtime.h -- internal host runtime shared by the entry points.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/hses.h"
#include "bm_exact.h"

namespace hses {

// Error reporting: every entry point returns an hses_status and leaves a
// message retrievable with hses_last_error() (thread-local).
int set_error(int code, const std::string& msg);
int check_hip(hipError_t e, const char* what);
#define HSES_CHECK_HIP(expr)                                    \
    do {                                                        \
        hipError_t _e = (expr);                                 \
        if (_e != hipSuccess) return ::hses::check_hip(_e, #expr); \
    } while (0)
#define HSES_REQUIRE(cond, msg)                                          \
    do {                                                                 \
        if (!(cond)) return ::hses::set_error(HSES_ERR_INVALID_ARG, msg); \
    } while (0)

// Host-side construction of the Box-Muller tables (bm_tables.cpp).
struct HostBmTables {
    BmTables small;
    std::vector<uint32_t> log_exc;  // kBitmapAlloc words (zero past kBitmapWords)
    std::vector<uint32_t> cos_exc;
    uint32_t n_log_exc = 0, n_cos_exc = 0;
    uint32_t n_log_danger = 0, n_cos_danger = 0;
};
// Builds the tables from the running glibc.  Returns an empty string on
// success, otherwise a description of the inconsistency.
std::string build_bm_tables(HostBmTables* out, int nthreads);

// GF(2) jump matrices over xorshift64: column-major 64 x uint64.
struct Gf2 {
    uint64_t c[64];
};
Gf2 gf2_identity();
Gf2 gf2_step();                          // one xorshift64 step
Gf2 gf2_mul(const Gf2& A, const Gf2& B);  // A * B
Gf2 gf2_pow(const Gf2& M, uint64_t n);

// Per-device state.
struct DeviceState {
    int device = -1;
    BmTables* d_tables = nullptr;   // device copy of the small tables
    uint32_t* d_log_exc = nullptr;  // 2 MB bitmaps
    uint32_t* d_cos_exc = nullptr;
    // Row-start jump tables, one per row length L (normals per row), each
    // matrix in nibble form (kJumpNib entries):
    // [0,16): M^(2L*j0); [16, 16+n1): M^(2L*16*j1).
    struct Jump {
        int64_t row_len = 0;
        int32_t n1 = 0;
        uint64_t* d_cols = nullptr;
    };
    std::vector<Jump> jumps;
    int num_cus = 0;
    size_t max_lds = 0;
};

// Returns the state of the current device, initialising it on first use.
int get_state(DeviceState** out);
// Device pointer of the jump table for row length L covering `rows` rows.
int get_jump_table(DeviceState* st, int64_t row_len, int64_t rows, const uint64_t** out);

constexpr int kJumpG = 16;  // rows per first-level jump group

}  // namespace hses
