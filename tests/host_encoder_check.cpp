// Host build of the kernels' shared HiF8 arithmetic (osp-next_amd/csrc/hif8_common.h)
// so the CPU test suite can compare it with the oracle without a GPU.
#include <stdint.h>

#include "../osp-next_amd/csrc/hif8_common.h"

extern "C" {

void chk_encode_bits(const uint32_t *x, uint8_t *c, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) c[i] = uint8_t(hif8::encode_npu_bits(x[i]));
}

void chk_decode_bits(uint32_t *y)
{
    for (uint32_t c = 0; c < 256; ++c) y[c] = hif8::decode_bits(c);
}

// The encode table the kernels copy to LDS (computed at compile time).
static constexpr hif8::EncTable kTab = hif8::make_enc_table();

int64_t chk_table(uint8_t *out, uint32_t *lo, uint32_t *hi)
{
    for (uint32_t i = 0; i < sizeof(kTab.v); ++i) out[i] = kTab.v[i];
    *lo = hif8::kTabLo;
    *hi = hif8::kTabHi;
    return int64_t(sizeof(kTab.v));
}
}
