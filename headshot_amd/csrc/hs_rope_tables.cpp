// Host-side axial 2D RoPE tables (rope::periods / rope::tables,
// crates/headshot-server/src/engine/rope.rs:5-43). Like the reference these
// are computed once per session on the CPU in f32 and uploaded; the kernels
// only read them.
//
// Bit-exactness with the reference: every step is a single IEEE f32
// operation in the reference's operand order, and sin/cos/pow are the
// platform libm's sinf/cosf/powf (what Rust's f32::sin/cos/powf call). This
// file is compiled with -ffp-contract=off so that 2*q - 1 is never fused.
#include <math.h>
#include <stdint.h>

#include "headshot_hip.h"

namespace hs {
hs_status fail(hs_status code, const char* fmt, ...);
}

extern "C" {

void hs_rope_periods(float* out16) {
    if (!out16) return;
    for (int i = 0; i < 16; i++) {
        // 100.0f32.powf(2.0 * i as f32 / 32.0)
        volatile float e = 2.0f * static_cast<float>(i);
        e = e / 32.0f;
        out16[i] = powf(100.0f, e);
    }
}

hs_status hs_rope_tables(const float* periods16, int32_t h_p, int32_t w_p, float* sin_out,
                         float* cos_out) {
    if (h_p < 0 || w_p < 0) return hs::fail(HS_EINVAL, "rope_tables: negative grid %dx%d", h_p, w_p);
    if (h_p == 0 || w_p == 0) return HS_OK;
    if (!periods16 || !sin_out || !cos_out) return hs::fail(HS_EINVAL, "rope_tables: null buffer");
    const float side = static_cast<float>(h_p > w_p ? h_p : w_p);
    const float tau = 6.28318530717958647692f;  // std::f32::consts::TAU
    // coord(i) = 2.0 * ((i as f32 + 0.5) / side) - 1.0
    auto coord = [side](int32_t i) {
        volatile float q = (static_cast<float>(i) + 0.5f) / side;
        volatile float twice = 2.0f * q;
        return twice - 1.0f;
    };
    for (int32_t row = 0; row < h_p; row++) {
        const float ch = coord(row);
        for (int32_t col = 0; col < w_p; col++) {
            const float cw = coord(col);
            const int64_t idx = (static_cast<int64_t>(row) * w_p + col) * 64;
            for (int i = 0; i < 16; i++) {
                // angle = tau * coord / period, left to right
                volatile float th = tau * ch;
                volatile float tw = tau * cw;
                const float ah = th / periods16[i];
                const float aw = tw / periods16[i];
                const float sh = sinf(ah), chh = cosf(ah);
                const float sw = sinf(aw), cww = cosf(aw);
                for (int half = 0; half <= 32; half += 32) {
                    sin_out[idx + half + i] = sh;
                    cos_out[idx + half + i] = chh;
                    sin_out[idx + half + 16 + i] = sw;
                    cos_out[idx + half + 16 + i] = cww;
                }
            }
        }
    }
    return HS_OK;
}

}  // extern "C"
