/* Exhaustive check of the Q8 rounding identity used by the device kernels
 * (pi_gemv.h, q8_round_clamp): for every float y with |y| < 2^22,
 *     truncf(y + copysignf(0.5f - 2^-25, y)) == roundf(y)
 * (roundf: half away from zero, as Rust's f32::round in quant_int.rs:49).
 * IEEE single precision, round to nearest even.  Exit status 0 when no value
 * differs; prints the count checked. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
    const float h = 0.49999997f; /* 0.5 - 2^-25, the largest float below 0.5 */
    uint32_t hb;
    memcpy(&hb, &h, 4);
    if (hb != 0x3effffffu) { printf("unexpected h bits 0x%08x\n", hb); return 2; }
    uint64_t n = 0, bad = 0;
    for (uint32_t s = 0; s < 2; s++)
        for (uint32_t m = 0; m < 0x4A800000u; m++) { /* 0 <= |y| < 2^22 */
            const uint32_t b = m | (s << 31);
            float y;
            memcpy(&y, &b, 4);
            volatile float r = y + copysignf(h, y);
            if (truncf(r) != roundf(y)) {
                if (bad < 4) printf("differs at y = %a\n", (double)y);
                bad++;
            }
            n++;
        }
    printf("checked %llu floats, %llu differ\n", (unsigned long long)n, (unsigned long long)bad);
    return bad != 0;
}
