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

// Row-start jump tables.  For every row length L in [1, kJumpMaxL] (normals
// per stream row) one block of kJumpPerL matrices in nibble form (kJumpNib
// entries each), with R = M^(2L) the xorshift64 advance over one row:
// [0, 16): R^j0; [16, 32): R^(16 j1); [32, 32 + kJumpN2): R^(256 j2), so the
// start of row j < kJumpMaxRows is three table products (row_start_state).
// Built once on the host, uploaded at hses_init, immutable afterwards.
constexpr int kJumpMaxL = 256;
constexpr int kJumpN2 = 64;
constexpr int kJumpPerL = 32 + kJumpN2;
constexpr int64_t kJumpMaxRows = 256ll * kJumpN2;
void build_jump_tables(std::vector<uint64_t>* out, int nthreads);

// Per-device state, created by hses_init.
struct DeviceState {
    int device = -1;
    BmTables* d_tables = nullptr;   // device copy of the small tables
    uint32_t* d_log_exc = nullptr;  // 2 MB bitmaps
    uint32_t* d_cos_exc = nullptr;
    uint64_t* d_jump = nullptr;     // kJumpMaxL blocks of kJumpPerL nibble matrices
    void* es_scratch = nullptr;     // this device's address of es_update.hip's scratch array
    int num_cus = 0;
    size_t max_lds = 0;
};

// Size of the file-scope scratch array of the allocation-free ES update
// (es_update.hip), and its per-device address lookup, run by hses_init with
// the device current.
constexpr size_t kEsScratchBytes = 32u << 20;
int es_scratch_setup(DeviceState* st);

// The state of the current device.  Fails (nothing is allocated here) when
// hses_init has not been called for it.
int get_state(DeviceState** out);
// Device pointer of the jump-table block for row length L, checked to cover
// `rows` rows.  Pure lookup: no allocation, no copy.
int get_jump_table(DeviceState* st, int64_t row_len, int64_t rows, const uint64_t** out);

}  // namespace hses
