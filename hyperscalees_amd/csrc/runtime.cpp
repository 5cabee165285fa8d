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
std::vector<uint64_t>* g_host_jump = nullptr;
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
    if (!g_host_jump) {
        unsigned hc = std::thread::hardware_concurrency();
        auto* j = new std::vector<uint64_t>();
        build_jump_tables(j, (int)std::min<unsigned>(hc ? hc : 1, 16u));
        g_host_jump = j;
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
    HSES_CHECK_HIP(hipMalloc(&st->d_jump, sizeof(uint64_t) * g_host_jump->size()));
    HSES_CHECK_HIP(hipMemcpy(st->d_jump, g_host_jump->data(), sizeof(uint64_t) * g_host_jump->size(),
                             hipMemcpyHostToDevice));
    {
        const int src = es_scratch_setup(st);  // with `dev` current
        if (src) return src;
    }
    if (cur != dev) HSES_CHECK_HIP(hipSetDevice(cur));
    g_states[dev] = st;
    *out = st;
    return HSES_OK;
}

int get_state(DeviceState** out) {
    int dev = 0;
    HSES_CHECK_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_mu);
    if (dev < 0 || dev >= (int)g_states.size() || !g_states[dev]) {
        char buf[96];
        snprintf(buf, sizeof buf, "hses_init(%d) has not been called for the current device", dev);
        return set_error(HSES_ERR_INVALID_ARG, buf);
    }
    *out = g_states[dev];
    return HSES_OK;
}

int get_jump_table(DeviceState* st, int64_t row_len, int64_t rows, const uint64_t** out) {
    if (row_len < 1 || row_len > kJumpMaxL || rows > kJumpMaxRows) {
        char buf[160];
        snprintf(buf, sizeof buf,
                 "noise stream rows of %lld normals x %lld rows exceed the jump tables "
                 "(row length <= %d, rows <= %lld)",
                 (long long)row_len, (long long)rows, kJumpMaxL, (long long)kJumpMaxRows);
        return set_error(HSES_ERR_UNSUPPORTED, buf);
    }
    *out = st->d_jump + (size_t)(row_len - 1) * kJumpPerL * kJumpNib;
    return HSES_OK;
}

// Nibble form of J: entry 16 i + v = J (v << 4i), the XOR of the columns
// 4i + bit over the set bits of v.
static void put_nibbles(uint64_t* e, const Gf2& J) {
    for (int i = 0; i < 16; ++i)
        for (int v = 0; v < 16; ++v) {
            uint64_t y = 0;
            for (int bit = 0; bit < 4; ++bit)
                if ((v >> bit) & 1) y ^= J.c[4 * i + bit];
            e[16 * i + v] = y;
        }
}

void build_jump_tables(std::vector<uint64_t>* out, int nthreads) {
    out->assign((size_t)kJumpMaxL * kJumpPerL * kJumpNib, 0);
    const Gf2 M = gf2_step();
    auto one_length = [&](int L) {
        uint64_t* blk = out->data() + (size_t)(L - 1) * kJumpPerL * kJumpNib;
        const Gf2 R = gf2_pow(M, 2ull * (uint64_t)L);  // one stream row = 2L steps
        Gf2 acc = gf2_identity();
        for (int j0 = 0; j0 < 16; ++j0) {
            put_nibbles(blk + (size_t)j0 * kJumpNib, acc);
            acc = gf2_mul(R, acc);
        }
        const Gf2 R16 = acc;
        acc = gf2_identity();
        for (int j1 = 0; j1 < 16; ++j1) {
            put_nibbles(blk + (size_t)(16 + j1) * kJumpNib, acc);
            acc = gf2_mul(R16, acc);
        }
        const Gf2 R256 = acc;
        acc = gf2_identity();
        for (int j2 = 0; j2 < kJumpN2; ++j2) {
            put_nibbles(blk + (size_t)(32 + j2) * kJumpNib, acc);
            acc = gf2_mul(R256, acc);
        }
    };
    const int nt = std::max(1, nthreads);
    std::vector<std::thread> pool;
    for (int t = 0; t < nt; ++t)
        pool.emplace_back([&, t] {
            for (int L = 1 + t; L <= kJumpMaxL; L += nt) one_length(L);
        });
    for (auto& th : pool) th.join();
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
