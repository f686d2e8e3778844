/* Every float y with |y| <= 128: (int)(y + copysignf(0.5 - 2^-25, y)) equals (int)roundf(y). The GEMV activation
 * quantizer rounds y = x / d (|y| <= 127 (1 + 2^-22)) this way instead of with roundf. Prints the mismatch count. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
    const float h = 0.49999997f;
    unsigned long long bad = 0, n = 0;
    for (uint64_t u = 0; u <= 0xffffffffull; ++u) {
        const uint32_t b = (uint32_t)u;
        float y;
        memcpy(&y, &b, 4);
        if (!(fabsf(y) <= 128.0f)) continue;
        ++n;
        volatile float s = y + copysignf(h, y);
        if ((int)s != (int)roundf(y)) ++bad;
    }
    printf("%llu %llu\n", n, bad);
    return 0;
}
