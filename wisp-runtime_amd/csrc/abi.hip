// C-ABI glue: version, error strings, expert size, tuning state.
#include <cstring>

#include "wisp_internal.hpp"

namespace wisp {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

void clear_error() { g_err[0] = 0; }

Tuning& tuning() {
    static Tuning t{2, 4, 4};
    return t;
}

}  // namespace wisp

extern "C" int wisp_abi_version(void) { return WISP_ABI_VERSION; }

extern "C" const char* wisp_last_error(void) { return wisp::g_err; }

// quant.py:17-22 (bits == 16 is raw bf16)
extern "C" int64_t wisp_expert_nbytes(int64_t n, int bits, int64_t group) {
    if (n <= 0) return -1;
    if (bits == 16) return 3 * n * 2;
    if (!(bits == 8 || bits == 4 || bits == 3 || bits == 2)) return -1;
    if (group <= 0 || (3 * n) % group != 0 || (3 * n * bits) % 8 != 0) return -1;
    return (3 * n * bits) / 8 + 4 * (3 * n / group);
}

extern "C" int wisp_set_tuning(int gu_rows, int gu_waves, int dn_iters) {
    wisp::clear_error();
    wisp::Tuning& t = wisp::tuning();
    if (gu_rows && !(gu_rows == 1 || gu_rows == 2 || gu_rows == 4 || gu_rows == 8))
        return wisp::fail_inval("gu_rows must be 1, 2, 4 or 8");
    if (gu_waves && !(gu_waves == 1 || gu_waves == 2 || gu_waves == 4 || gu_waves == 8))
        return wisp::fail_inval("gu_waves must be 1, 2, 4 or 8");
    if (dn_iters && !(dn_iters == 1 || dn_iters == 2 || dn_iters == 4 || dn_iters == 8))
        return wisp::fail_inval("dn_iters must be 1, 2, 4 or 8");
    if (gu_rows) t.gu_rows = gu_rows;
    if (gu_waves) t.gu_waves = gu_waves;
    if (dn_iters) t.dn_iters = dn_iters;
    return WISP_OK;
}
