/* Scalar C restatement of the bit-level parts of Vaayu's packed-expert arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: a second, independently written oracle that the numpy one
 * (oracle/oracle.py) is cross-checked against. Rounding here is done by scaling to the
 * target format's quantum and rounding with nearbyint() (IEEE nearest-even), not by the
 * bit tricks the numpy oracle uses, so a mistake in either shows up as a disagreement.
 *
 * Reference arithmetic restated:
 *   - round to the activation dtype: vaayu/packed_expert_kernels.py:75-88
 *   - code extraction and dequant:   vaayu/moe_patch.py:750-769, vaayu/packed_expert_kernels.py:100-106
 *   - one expert's stock stages:     vaayu/packed_expert_kernels.py:399-410
 *   - e4m3 block dequant:            vaayu/model_code/deepseek_v4/modeling_deepseek_v4.py:228-240
 *   - e2m1 values:                   vendor .../numerics_details/mxfp.py:238-253
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* act codes as the reference's _DTYPE_CODE: 0 bf16, 1 fp16, 2 fp32 */
static double round_fmt(double v, int p, int emin, double maxv) {
    if (isnan(v) || isinf(v) || v == 0.0) return v;
    int e;
    frexp(v, &e);
    int lead = e - 1;                 /* exponent of the leading bit */
    if (lead < emin) lead = emin;     /* subnormal: fixed quantum */
    double q = ldexp(1.0, lead - (p - 1));
    double r = nearbyint(v / q) * q;  /* v / q is exact: q is a power of two */
    if (fabs(r) > maxv) return copysign(INFINITY, v);
    return r;
}

double cref_round(double v, int act) {
    switch (act) {
    case 0: return round_fmt(v, 8, -126, 3.3895313892515355e38);
    case 1: return round_fmt(v, 11, -14, 65504.0);
    default: return round_fmt(v, 24, -126, 3.4028234663852886e38);
    }
}

uint16_t cref_bf16_bits(float f) {
    if (isnan(f)) return 0x7FC0;
    float r = (float)cref_round((double)f, 0);
    uint32_t u;
    memcpy(&u, &r, 4);
    return (uint16_t)(u >> 16);
}

/* Whole-blob dequant: n_words int32 words, codes (w >> j*bits) & mask, minus 2^(bits-1),
 * times the group scale (scale[] already holds float values of its own dtype), each
 * converted to `act` and the product rounded to `act`. Writes n_words*32/bits floats. */
void cref_dequant(const int32_t *packed, long n_words, const float *scale, int bits, int gs,
                  int act, float *out) {
    int per = 32 / bits;
    uint32_t mask = (1u << bits) - 1u;
    for (long w = 0; w < n_words; ++w) {
        uint32_t word = (uint32_t)packed[w];
        for (int j = 0; j < per; ++j) {
            long i = w * per + j;
            double code = (double)((word >> (j * bits)) & mask) - (double)(1 << (bits - 1));
            double s = cref_round((double)scale[i / gs], act);
            out[i] = (float)cref_round(code * s, act);
        }
    }
}

static double silu_f32(double g) {
    float gf = (float)g;
    return (double)(gf / (1.0f + expf(-gf)));
}

/* One expert's stock stages for one token: g = x.Wg, u = x.Wu (double sums, rounded
 * once), a = SiLU(g) rounded, h = a*u rounded, y = h.Wd rounded.
 * wg, wu: [inter, hidden]; wd: [hidden, inter]; h: [inter]; y: [hidden]. */
void cref_expert(const float *x, const float *wg, const float *wd, const float *wu, int hidden,
                 int inter, int act, float *h, float *y) {
    for (int i = 0; i < inter; ++i) {
        double g = 0.0, u = 0.0;
        for (int k = 0; k < hidden; ++k) {
            g += (double)x[k] * (double)wg[(long)i * hidden + k];
            u += (double)x[k] * (double)wu[(long)i * hidden + k];
        }
        double gr = cref_round(g, act), ur = cref_round(u, act);
        double a = cref_round(silu_f32(gr), act);
        h[i] = (float)cref_round(a * ur, act);
    }
    for (int r = 0; r < hidden; ++r) {
        double acc = 0.0;
        for (int i = 0; i < inter; ++i) acc += (double)h[i] * (double)wd[(long)r * inter + i];
        y[r] = (float)cref_round(acc, act);
    }
}

float cref_e4m3(uint8_t b) {
    int s = b >> 7, e = (b >> 3) & 0xF, m = b & 7;
    if (e == 0xF && m == 7) return NAN;
    double v = e == 0 ? ldexp((double)m, -9) : ldexp(8.0 + m, e - 10);
    return (float)(s ? -v : v);
}

float cref_e2m1(uint8_t nibble) {
    int s = (nibble >> 3) & 1, e = (nibble >> 1) & 3, m = nibble & 1;
    double v = e == 0 ? 0.5 * m : ldexp(1.0 + 0.5 * m, e - 1);
    return (float)(s ? -v : v);
}
