// Host-side runtime of libie_attn: error reporting, cache-descriptor checks, per-device CU count.
#include <string.h>

#include <mutex>

#include "ie_common.h"

namespace ie {

static thread_local char g_last_error[256] = "";

void set_error(const char* msg) {
    strncpy(g_last_error, msg, sizeof(g_last_error) - 1);
    g_last_error[sizeof(g_last_error) - 1] = 0;
}

hipError_t check_cache(const ie_kv_cache* c) {
    IE_REQUIRE(c != nullptr, "cache descriptor is null");
    IE_REQUIRE(c->k && c->v && c->k_scale && c->v_scale && c->k_calibration,
               "cache descriptor has a null tensor");
    IE_REQUIRE(c->head_dim == 128, "head_dim must be 128");
    IE_REQUIRE(c->pool > 0 && c->num_kv_heads > 0 && c->max_len > 0, "empty cache");
    IE_REQUIRE(c->stride_tok == c->head_dim, "cache token stride must equal head_dim");
    IE_REQUIRE(c->stride_head % 16 == 0 && c->stride_slot % 16 == 0,
               "cache head/slot strides must be multiples of 16 elements");
    IE_REQUIRE((reinterpret_cast<uintptr_t>(c->k) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(c->v) & 15) == 0,
               "cache k/v must be 16-byte aligned");
    IE_REQUIRE((reinterpret_cast<uintptr_t>(c->k_scale) & 3) == 0 &&
                   (reinterpret_cast<uintptr_t>(c->v_scale) & 3) == 0,
               "cache scales must be 4-byte aligned");
    return hipSuccess;
}

// CU count of the current device, cached per device (kernels.py:267-269 caches SM count).
int device_cu_count() {
    static int counts[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (counts[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        counts[dev] = n;
    }
    return counts[dev];
}

}  // namespace ie

extern "C" int32_t ie_attn_version(void) { return (1 << 16) | 0; }

extern "C" const char* ie_attn_last_error(void) { return ie::g_last_error; }
