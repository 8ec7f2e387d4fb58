// FLASH_ATTN_EXT on the device (attention.cc): placeholder until the kernel lands.
#include "host.h"

using namespace sdhip;

extern "C" {

int sdhip_attention_supported(const sdhip_tensor *, const sdhip_tensor *, const sdhip_tensor *, const sdhip_tensor *,
                              float, float) {
    return 0;
}

size_t sdhip_attention_work_size(const sdhip_tensor *, const sdhip_tensor *, const sdhip_tensor *,
                                 const sdhip_tensor *) {
    return 0;
}

sdhip_status sdhip_attention(const sdhip_tensor *, const sdhip_tensor *, const sdhip_tensor *, const sdhip_tensor *,
                             float, float, float, void *, size_t, void *) {
    return fail(SDHIP_UNSUPPORTED, "attention: not built yet");
}

}  // extern "C"
