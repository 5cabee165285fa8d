// runtime.cpp -- error reporting, per-device state and lazy initialisation.
#include "runtime.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <thread>

namespace hses {

namespace {
thread_local std::string g_err;
std::mutex g_mu;
std::vector<DeviceState*> g_states;  // indexed by device id
HostBmTables* g_host_tables = nullptr;
}  // namespace

int set_error(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int check_hip(hipError_t e, const char* what) {
    char buf[512];
    snprintf(buf, sizeof buf, "HIP error %d (%s) in %s", (int)e, hipGetErrorString(e), what);
    return set_error(HSES_ERR_HIP, buf);
}

static int init_device_locked(int dev, DeviceState** out) {
    if (dev < 0) return set_error(HSES_ERR_INVALID_ARG, "negative device id");
    if ((int)g_states.size() <= dev) g_states.resize(dev + 1, nullptr);
    if (g_states[dev]) {
        *out = g_states[dev];
        return HSES_OK;
    }
    if (!g_host_tables) {
        HostBmTables* t = new HostBmTables();
        unsigned hc = std::thread::hardware_concurrency();
        int nt = (int)std::min<unsigned>(hc ? hc : 1, 16u);
        std::string err = build_bm_tables(t, nt);
        if (!err.empty()) {
            delete t;
            return set_error(HSES_ERR_INTERNAL, "Box-Muller table construction failed: " + err);
        }
        g_host_tables = t;
    }
    int cur = 0;
    HSES_CHECK_HIP(hipGetDevice(&cur));
    if (cur != dev) HSES_CHECK_HIP(hipSetDevice(dev));
    DeviceState* st = new DeviceState();
    st->device = dev;
    hipDeviceProp_t prop;
    HSES_CHECK_HIP(hipGetDeviceProperties(&prop, dev));
    st->num_cus = prop.multiProcessorCount;
    st->max_lds = prop.sharedMemPerBlock;
    HSES_CHECK_HIP(hipMalloc(&st->d_tables, sizeof(BmTables)));
    HSES_CHECK_HIP(hipMalloc(&st->d_log_exc, sizeof(uint32_t) * kBitmapAlloc));
    HSES_CHECK_HIP(hipMalloc(&st->d_cos_exc, sizeof(uint32_t) * kBitmapAlloc));
    HSES_CHECK_HIP(hipMemcpy(st->d_tables, &g_host_tables->small, sizeof(BmTables),
                             hipMemcpyHostToDevice));
    HSES_CHECK_HIP(hipMemcpy(st->d_log_exc, g_host_tables->log_exc.data(),
                             sizeof(uint32_t) * kBitmapAlloc, hipMemcpyHostToDevice));
    HSES_CHECK_HIP(hipMemcpy(st->d_cos_exc, g_host_tables->cos_exc.data(),
                             sizeof(uint32_t) * kBitmapAlloc, hipMemcpyHostToDevice));
    if (cur != dev) HSES_CHECK_HIP(hipSetDevice(cur));
    g_states[dev] = st;
    *out = st;
    return HSES_OK;
}

int get_state(DeviceState** out) {
    int dev = 0;
    HSES_CHECK_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_mu);
    return init_device_locked(dev, out);
}

int get_jump_table(DeviceState* st, int64_t row_len, int64_t rows, const uint64_t** out) {
    std::lock_guard<std::mutex> lk(g_mu);
    const int64_t need_n1 = (rows + kJumpG - 1) / kJumpG;
    for (auto& j : st->jumps) {
        if (j.row_len == row_len && j.n1 >= need_n1) {
            *out = j.d_cols;
            return HSES_OK;
        }
    }
    // Build (or rebuild larger) the table for this row length.
    int32_t n1 = (int32_t)std::max<int64_t>(need_n1, 64);
    std::vector<uint64_t> host((size_t)(kJumpG + n1) * kJumpNib);
    // Matrix J in nibble form: entry 16 i + v = J (v << 4i) = XOR of the
    // columns 4i + bit over the set bits of v.
    auto put = [&](size_t m, const Gf2& J) {
        uint64_t* e = &host[m * kJumpNib];
        for (int i = 0; i < 16; ++i)
            for (int v = 0; v < 16; ++v) {
                uint64_t y = 0;
                for (int bit = 0; bit < 4; ++bit)
                    if ((v >> bit) & 1) y ^= J.c[4 * i + bit];
                e[16 * i + v] = y;
            }
    };
    const Gf2 M = gf2_step();
    const Gf2 row = gf2_pow(M, 2ull * (uint64_t)row_len);  // one factor row = 2L steps
    Gf2 acc = gf2_identity();
    for (int j0 = 0; j0 < kJumpG; ++j0) {
        put((size_t)j0, acc);
        acc = gf2_mul(row, acc);
    }
    const Gf2 grp = acc;  // row^16
    Gf2 g = gf2_identity();
    for (int j1 = 0; j1 < n1; ++j1) {
        put((size_t)(kJumpG + j1), g);
        g = gf2_mul(grp, g);
    }
    uint64_t* d = nullptr;
    HSES_CHECK_HIP(hipMalloc(&d, host.size() * sizeof(uint64_t)));
    HSES_CHECK_HIP(hipMemcpy(d, host.data(), host.size() * sizeof(uint64_t), hipMemcpyHostToDevice));
    bool replaced = false;
    for (auto& j : st->jumps) {
        if (j.row_len == row_len) {
            // The old table may still be read by in-flight kernels; keep it alive.
            j.n1 = n1;
            j.d_cols = d;
            replaced = true;
            break;
        }
    }
    if (!replaced) st->jumps.push_back({row_len, n1, d});
    *out = d;
    return HSES_OK;
}

}  // namespace hses

using namespace hses;

extern "C" int hses_init(int device) {
    std::lock_guard<std::mutex> lk(g_mu);
    DeviceState* st = nullptr;
    return init_device_locked(device, &st);
}

extern "C" int hses_last_error(char* buf, size_t len) {
    if (!buf || len == 0) return HSES_ERR_INVALID_ARG;
    size_t n = std::min(len - 1, g_err.size());
    memcpy(buf, g_err.data(), n);
    buf[n] = 0;
    return HSES_OK;
}

extern "C" const char* hses_version(void) { return "hses 0.1 (gfx950)"; }

extern "C" int hses_bm_stats(uint32_t out[2]) {
    if (!out) return set_error(HSES_ERR_INVALID_ARG, "out is NULL");
    DeviceState* st;
    int rc = get_state(&st);
    if (rc) return rc;
    out[0] = g_host_tables->n_log_exc;
    out[1] = g_host_tables->n_cos_exc;
    return HSES_OK;
}

extern "C" uint64_t hses_noise_seed(uint64_t key, int32_t te, int32_t tt) {
    return noise_seed(key, te, tt);
}
