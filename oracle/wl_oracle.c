/*
 * wl_oracle.c - CPU restatement of Windlass's quantized-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE (the oracle). Loaded only by the tests, the smoke check and the
 * benchmark's CPU-baseline leg; the product library never links or calls it.
 *
 * Build (oracle/Makefile): gcc -O2 -fno-tree-vectorize -ffp-contract=off -fopenmp.
 * No fast-math and no contraction: every float operation below rounds on its own and in
 * the order the reference writes it, which is what "bit-exact decode" is measured against.
 * Each function cites the reference lines it restates.
 */
#include "wl_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ fp16 (src/Half.cs) */

static float bits_to_float(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t float_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* src/Half.cs:59-90: sign, 5-bit exponent, 10-bit mantissa; subnormals renormalised. */
float wlo_half_to_float(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    int exp = (h >> 10) & 0x1F;
    uint32_t mant = h & 0x3FFu;
    if (exp == 0) {
        if (mant == 0) return bits_to_float(sign);
        int shift = 0;
        while ((mant & 0x400u) == 0) { mant <<= 1; shift++; }
        /* value = 1.m * 2^(-14 - (shift - 1)) */
        return bits_to_float(sign | (uint32_t)(127 - 15 - (shift - 1)) << 23 | (mant & 0x3FFu) << 13);
    }
    if (exp == 31) return bits_to_float(sign | 0x7F800000u | mant << 13);
    return bits_to_float(sign | (uint32_t)(exp - 15 + 127) << 23 | mant << 13);
}

/* src/Half.cs:29-57: NaN keeps a quiet payload bit, overflow -> Inf, RNE everywhere. */
uint16_t wlo_half_from_float(float value)
{
    uint32_t f = float_to_bits(value);
    uint32_t sign = (f >> 16) & 0x8000u;
    int e = (int)((f >> 23) & 0xFF);
    uint32_t m = f & 0x7FFFFFu;
    if (e == 255) return (uint16_t)(sign | 0x7C00u | (m ? 0x200u : 0u));
    int ne = e - 127 + 15;
    if (ne >= 31) return (uint16_t)(sign | 0x7C00u);
    if (ne <= 0) {
        if (ne < -10) return (uint16_t)sign;
        m |= 0x800000u;
        int shift = 14 - ne;
        uint32_t hm = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)ne << 10) | (m >> 13);
    uint32_t r = m & 0x1FFFu;
    if (r > 0x1000u || (r == 0x1000u && (h & 1u))) h++;   /* a carry into the exponent is right */
    return (uint16_t)h;
}

float wlo_half_round(float f) { return wlo_half_to_float(wlo_half_from_float(f)); }

void wlo_half_to_float_n(const uint16_t *h, int64_t n, float *out)
{
    for (int64_t i = 0; i < n; i++) out[i] = wlo_half_to_float(h[i]);
}

void wlo_half_from_float_n(const float *f, int64_t n, uint16_t *out)
{
    for (int64_t i = 0; i < n; i++) out[i] = wlo_half_from_float(f[i]);
}

static float H(const uint8_t *p) { return wlo_half_to_float((uint16_t)(p[0] | (p[1] << 8))); }
static uint32_t U32(const uint8_t *p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }

/* ------------------------------------------------------- Rng (tests/TinyModels.cs:89-97) */

void wlo_rng_init(uint64_t *s, uint64_t seed) { *s = seed * 0x9E3779B97F4A7C15ull + 1; }

uint64_t wlo_rng_next(uint64_t *s)
{
    uint64_t v = *s;
    v ^= v >> 12; v ^= v << 25; v ^= v >> 27;
    *s = v;
    return v * 2685821657736338717ull;
}

static uint8_t rng_byte(uint64_t *s) { return (uint8_t)(wlo_rng_next(s) >> 56); }
static double rng_uniform(uint64_t *s) { return (double)(wlo_rng_next(s) >> 11) * (1.0 / 9007199254740992.0); }
static float rng_normal(uint64_t *s)
{
    double u = rng_uniform(s), v = rng_uniform(s);
    if (u < 1e-12) u = 1e-12;
    return (float)(sqrt(-2 * log(u)) * cos(2 * M_PI * v));
}

void wlo_rng_bytes(uint64_t *s, int64_t n, uint8_t *out) { for (int64_t i = 0; i < n; i++) out[i] = rng_byte(s); }
void wlo_rng_uniforms(uint64_t *s, int64_t n, double *out) { for (int64_t i = 0; i < n; i++) out[i] = rng_uniform(s); }
void wlo_rng_normals(uint64_t *s, int64_t n, float *out) { for (int64_t i = 0; i < n; i++) out[i] = rng_normal(s); }

/* --------------------------------------------------------- layouts (src/Gguf.cs:30-66) */

int wlo_layout(int t, int *be, int *bb)
{
    switch (t) {
    case WLO_F32: *be = 1; *bb = 4; return 1;
    case WLO_F16: case WLO_BF16: *be = 1; *bb = 2; return 1;
    case WLO_Q4_0: *be = 32; *bb = 18; return 1;
    case WLO_Q4_1: *be = 32; *bb = 20; return 1;
    case WLO_Q5_0: *be = 32; *bb = 22; return 1;
    case WLO_Q5_1: *be = 32; *bb = 24; return 1;
    case WLO_Q8_0: *be = 32; *bb = 34; return 1;
    case WLO_Q2_K: *be = 256; *bb = 84; return 1;
    case WLO_Q3_K: *be = 256; *bb = 110; return 1;
    case WLO_Q4_K: *be = 256; *bb = 144; return 1;
    case WLO_Q5_K: *be = 256; *bb = 176; return 1;
    case WLO_Q6_K: *be = 256; *bb = 210; return 1;
    case WLO_IQ2_XXS: *be = 256; *bb = 66; return 1;
    case WLO_IQ3_S: *be = 256; *bb = 110; return 1;
    case WLO_IQ2_S: *be = 256; *bb = 82; return 1;
    case WLO_IQ4_NL: *be = 32; *bb = 18; return 1;
    case WLO_IQ4_XS: *be = 256; *bb = 136; return 1;
    }
    *be = 0; *bb = 0;
    return 0;
}

int wlo_can_decode(int t)
{
    int be, bb;
    return wlo_layout(t, &be, &bb);
}

int wlo_can_dot(int t)
{
    return t == WLO_F32 || t == WLO_F16 || t == WLO_BF16 || t == WLO_Q4_0 || t == WLO_Q8_0 || t == WLO_Q4_K ||
           t == WLO_Q5_K || t == WLO_Q6_K;
}

/* ------------------------------------------------------ I-quant tables (src/IqTables.cs) */

/* kvalues_iq4nl (src/IqTables.cs:22). */
static const int8_t KVALUES[16] = { -127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113 };

/* iq2xxs_grid (src/IqTables.cs:23-57), stored as 2-bit codes per byte: 0 -> 0x08, 1 -> 0x19,
 * 2 -> 0x2b (the only byte values the grid holds); byte j of entry i is code bits 2j..2j+1. */
static const uint16_t IQ2XXS_CODES[256] = {
    0x0000, 0x0002, 0x0005, 0x0008, 0x000a, 0x0011, 0x0014, 0x0020, 0x0022, 0x0028, 0x002a, 0x0041, 0x0044, 0x0050, 0x0058, 0x0061,
    0x0064, 0x0080, 0x0082, 0x008a, 0x00a2, 0x0101, 0x0104, 0x0110, 0x0115, 0x0140, 0x0184, 0x0198, 0x0200, 0x0202, 0x0222, 0x0282,
    0x0401, 0x0404, 0x0410, 0x0421, 0x0424, 0x0440, 0x0442, 0x0448, 0x0460, 0x0481, 0x0484, 0x0490, 0x04a4, 0x0500, 0x0502, 0x0508,
    0x0520, 0x0546, 0x0569, 0x0580, 0x0591, 0x0609, 0x0610, 0x0640, 0x0684, 0x06a4, 0x0800, 0x0805, 0x0808, 0x0814, 0x0828, 0x0841,
    0x0844, 0x0850, 0x0852, 0x0888, 0x0904, 0x0940, 0x0a02, 0x0a14, 0x1001, 0x1004, 0x1010, 0x1021, 0x1040, 0x1060, 0x1084, 0x1090,
    0x1095, 0x1100, 0x1108, 0x1120, 0x1150, 0x115a, 0x1180, 0x1224, 0x1245, 0x1400, 0x1408, 0x1420, 0x1425, 0x1449, 0x1480, 0x1518,
    0x1562, 0x1600, 0x1616, 0x1801, 0x1804, 0x1810, 0x1840, 0x1881, 0x1900, 0x1905, 0x19a0, 0x1a51, 0x2000, 0x2002, 0x200a, 0x2044,
    0x2061, 0x2080, 0x2082, 0x2129, 0x2148, 0x2200, 0x2202, 0x2401, 0x2404, 0x2410, 0x2440, 0x2456, 0x2500, 0x2541, 0x2564, 0x2690,
    0x2808, 0x2820, 0x2894, 0x2a44, 0x4001, 0x4004, 0x4010, 0x4018, 0x4021, 0x4024, 0x4040, 0x4048, 0x4056, 0x4060, 0x4081, 0x4084,
    0x4090, 0x4100, 0x4120, 0x4161, 0x4180, 0x4185, 0x4201, 0x4210, 0x4248, 0x4256, 0x4268, 0x4400, 0x4408, 0x4420, 0x4480, 0x4499,
    0x4512, 0x4524, 0x4600, 0x4801, 0x4804, 0x4810, 0x4840, 0x4845, 0x4900, 0x4958, 0x4961, 0x4982, 0x4a45, 0x4a90, 0x5000, 0x5008,
    0x5011, 0x5019, 0x5020, 0x5080, 0x5088, 0x5104, 0x5142, 0x51a4, 0x5291, 0x5490, 0x5492, 0x550a, 0x5601, 0x5654, 0x5800, 0x5811,
    0x5819, 0x5864, 0x5940, 0x5a08, 0x6004, 0x6010, 0x6040, 0x6068, 0x6100, 0x6155, 0x6218, 0x6260, 0x6400, 0x6405, 0x6510, 0x6512,
    0x6584, 0x6842, 0x8000, 0x8002, 0x800a, 0x8041, 0x8082, 0x8104, 0x8118, 0x8140, 0x8211, 0x8401, 0x8404, 0x8410, 0x8415, 0x8440,
    0x8460, 0x8500, 0x8546, 0x8594, 0x8609, 0x8640, 0x8660, 0x8802, 0x8904, 0x8a11, 0x9004, 0x9010, 0x9024, 0x9040, 0x90a1, 0x9116,
    0x9180, 0x9245, 0x9400, 0x9422, 0x9444, 0x9551, 0x9881, 0x9920, 0xa002, 0xa050, 0xa085, 0xa109, 0xa200, 0xa418, 0xa850, 0xa904,
};

/* iq2s_grid (src/IqTables.cs:125-255), 2-bit codes per byte as above; iq3s_grid
 * (src/IqTables.cs:291-357), 3-bit codes per byte: code c -> 2c + 1 (the grid holds the odd
 * bytes 1..15); byte j of entry i is code bits 3j..3j+2. */
static const uint16_t IQ2S_CODES[1024] = {
    0x0000, 0x0002, 0x0005, 0x0008, 0x000a, 0x0011, 0x0014, 0x0016, 0x0019, 0x0020, 0x0022, 0x0025, 0x0028, 0x0041, 0x0044, 0x0046,
    0x0049, 0x0050, 0x0052, 0x0055, 0x0058, 0x0061, 0x0064, 0x0066, 0x0069, 0x0080, 0x0082, 0x0085, 0x0088, 0x0091, 0x0094, 0x00a0,
    0x00a5, 0x00aa, 0x0101, 0x0104, 0x0106, 0x0109, 0x0110, 0x0112, 0x0115, 0x0118, 0x0121, 0x0124, 0x0140, 0x0142, 0x0145, 0x0148,
    0x0151, 0x0154, 0x0156, 0x0159, 0x0160, 0x0165, 0x0168, 0x0181, 0x0184, 0x0190, 0x0192, 0x0195, 0x01a1, 0x01a4, 0x0200, 0x0202,
    0x0205, 0x0208, 0x0211, 0x0214, 0x0220, 0x022a, 0x0241, 0x0244, 0x0246, 0x0249, 0x0250, 0x0255, 0x0280, 0x0285, 0x028a, 0x0294,
    0x02a2, 0x0401, 0x0404, 0x0406, 0x0409, 0x0410, 0x0412, 0x0415, 0x0418, 0x0421, 0x0424, 0x0426, 0x0429, 0x0440, 0x0442, 0x0445,
    0x0448, 0x044a, 0x0451, 0x0454, 0x0456, 0x0459, 0x0460, 0x0462, 0x0465, 0x0481, 0x0484, 0x0486, 0x0489, 0x0490, 0x0495, 0x0498,
    0x04a1, 0x04a4, 0x0500, 0x0502, 0x0505, 0x0508, 0x050a, 0x0511, 0x0514, 0x0516, 0x0519, 0x0520, 0x0525, 0x0528, 0x0541, 0x0544,
    0x0546, 0x0549, 0x0550, 0x0552, 0x0555, 0x0558, 0x0561, 0x0564, 0x0580, 0x0582, 0x0585, 0x0588, 0x0591, 0x0594, 0x05a0, 0x0601,
    0x0604, 0x0606, 0x0609, 0x0610, 0x0615, 0x0640, 0x0645, 0x0648, 0x0651, 0x0654, 0x0660, 0x0681, 0x0684, 0x0690, 0x0800, 0x0802,
    0x0805, 0x0808, 0x0811, 0x0814, 0x0816, 0x0819, 0x0820, 0x0825, 0x082a, 0x0841, 0x0844, 0x0846, 0x0849, 0x0850, 0x0852, 0x0855,
    0x0858, 0x0861, 0x0864, 0x0880, 0x0885, 0x0894, 0x08aa, 0x0901, 0x0904, 0x0910, 0x0912, 0x0915, 0x0918, 0x0921, 0x0940, 0x0945,
    0x0948, 0x0951, 0x0954, 0x0960, 0x0981, 0x0990, 0x0a00, 0x0a11, 0x0a14, 0x0a22, 0x0a28, 0x0a2a, 0x0a50, 0x0a99, 0x1001, 0x1004,
    0x1006, 0x1009, 0x1010, 0x1012, 0x1015, 0x1018, 0x1021, 0x1024, 0x1026, 0x1040, 0x1042, 0x1045, 0x1048, 0x1051, 0x1054, 0x1056,
    0x1059, 0x1060, 0x1062, 0x1065, 0x1068, 0x1081, 0x1084, 0x1086, 0x1090, 0x1095, 0x1098, 0x10a1, 0x10a4, 0x1100, 0x1102, 0x1105,
    0x1108, 0x110a, 0x1111, 0x1114, 0x1116, 0x1119, 0x1120, 0x1122, 0x1125, 0x1128, 0x1141, 0x1144, 0x1146, 0x1149, 0x1150, 0x1152,
    0x1155, 0x1158, 0x1161, 0x1164, 0x1180, 0x1182, 0x1185, 0x1188, 0x1191, 0x1194, 0x1201, 0x1204, 0x1209, 0x1210, 0x1215, 0x1221,
    0x1224, 0x1240, 0x1245, 0x1251, 0x1254, 0x1281, 0x1284, 0x1290, 0x1400, 0x1402, 0x1405, 0x1408, 0x1411, 0x1414, 0x1416, 0x1419,
    0x1420, 0x1425, 0x1428, 0x1441, 0x1444, 0x1446, 0x1449, 0x1450, 0x1452, 0x1455, 0x1458, 0x1461, 0x1464, 0x1480, 0x1482, 0x1485,
    0x1488, 0x1491, 0x1494, 0x14a0, 0x1501, 0x1504, 0x1506, 0x1509, 0x1510, 0x1512, 0x1515, 0x1518, 0x1521, 0x1524, 0x1540, 0x1542,
    0x1545, 0x1548, 0x1551, 0x1554, 0x1560, 0x1581, 0x1584, 0x1590, 0x1600, 0x1605, 0x1608, 0x1611, 0x1614, 0x1620, 0x1641, 0x1644,
    0x1650, 0x1680, 0x16aa, 0x1801, 0x1804, 0x1806, 0x1809, 0x1810, 0x1815, 0x1818, 0x1821, 0x1840, 0x1842, 0x1845, 0x1848, 0x1851,
    0x1854, 0x1860, 0x1881, 0x1884, 0x1900, 0x1902, 0x1905, 0x1908, 0x1911, 0x1914, 0x1920, 0x1941, 0x1944, 0x1950, 0x1969, 0x19a2,
    0x1a04, 0x1a10, 0x1a40, 0x1a56, 0x2000, 0x2002, 0x2005, 0x2008, 0x2011, 0x2014, 0x2016, 0x2019, 0x2020, 0x2025, 0x202a, 0x2041,
    0x2044, 0x2050, 0x2052, 0x2055, 0x2064, 0x2080, 0x208a, 0x2094, 0x20aa, 0x2101, 0x2104, 0x2110, 0x2112, 0x2115, 0x2121, 0x2140,
    0x2142, 0x2145, 0x2151, 0x2154, 0x2160, 0x2181, 0x2184, 0x2190, 0x2200, 0x220a, 0x2222, 0x2228, 0x222a, 0x2244, 0x2250, 0x2288,
    0x228a, 0x22a8, 0x2401, 0x2404, 0x2406, 0x2409, 0x2410, 0x2415, 0x2418, 0x2421, 0x2424, 0x2440, 0x2442, 0x2445, 0x2448, 0x2451,
    0x2454, 0x2460, 0x2481, 0x2484, 0x2490, 0x2500, 0x2505, 0x2508, 0x2511, 0x2514, 0x2520, 0x2541, 0x2544, 0x2550, 0x2566, 0x2580,
    0x2601, 0x2604, 0x2610, 0x2640, 0x2659, 0x2800, 0x2805, 0x2811, 0x2814, 0x2841, 0x2844, 0x2850, 0x288a, 0x28aa, 0x2901, 0x2904,
    0x2910, 0x2995, 0x2a0a, 0x2a22, 0x2a64, 0x2a88, 0x2a8a, 0x4001, 0x4004, 0x4006, 0x4009, 0x4010, 0x4012, 0x4015, 0x4018, 0x401a,
    0x4021, 0x4024, 0x4026, 0x4040, 0x4042, 0x4045, 0x4048, 0x404a, 0x4051, 0x4054, 0x4056, 0x4059, 0x4060, 0x4062, 0x4065, 0x4081,
    0x4084, 0x4090, 0x4095, 0x4098, 0x40a1, 0x40a4, 0x4100, 0x4102, 0x4105, 0x4108, 0x4111, 0x4114, 0x4116, 0x4119, 0x4120, 0x4122,
    0x4125, 0x4141, 0x4144, 0x4146, 0x4149, 0x4150, 0x4152, 0x4155, 0x4158, 0x4161, 0x4164, 0x4180, 0x4182, 0x4185, 0x4188, 0x4191,
    0x4194, 0x41a0, 0x4201, 0x4204, 0x4210, 0x4212, 0x4215, 0x4218, 0x4224, 0x4240, 0x4245, 0x4248, 0x4251, 0x4254, 0x4260, 0x4281,
    0x4284, 0x4400, 0x4402, 0x4405, 0x4408, 0x440a, 0x4411, 0x4414, 0x4416, 0x4419, 0x4420, 0x4422, 0x4425, 0x4428, 0x4441, 0x4444,
    0x4446, 0x4449, 0x4450, 0x4452, 0x4455, 0x4458, 0x4461, 0x4464, 0x4480, 0x4482, 0x4485, 0x4488, 0x4491, 0x4494, 0x44a0, 0x4501,
    0x4504, 0x4506, 0x4509, 0x4510, 0x4512, 0x4515, 0x4518, 0x4521, 0x4524, 0x4540, 0x4542, 0x4545, 0x4548, 0x4551, 0x4554, 0x4560,
    0x456a, 0x4581, 0x4584, 0x4590, 0x4600, 0x4602, 0x4605, 0x4608, 0x4611, 0x4614, 0x4620, 0x4641, 0x4644, 0x4650, 0x4680, 0x46a5,
    0x4801, 0x4804, 0x4809, 0x4810, 0x4812, 0x4815, 0x4818, 0x4821, 0x4824, 0x4840, 0x4842, 0x4845, 0x4848, 0x4851, 0x4854, 0x4860,
    0x4884, 0x4890, 0x4900, 0x4902, 0x4905, 0x4908, 0x4911, 0x4914, 0x4920, 0x4941, 0x4944, 0x4950, 0x4980, 0x4996, 0x4a01, 0x4a04,
    0x4a10, 0x4a40, 0x5000, 0x5002, 0x5005, 0x5008, 0x5011, 0x5014, 0x5016, 0x5019, 0x5020, 0x5022, 0x5025, 0x5028, 0x5041, 0x5044,
    0x5046, 0x5049, 0x5050, 0x5052, 0x5055, 0x5058, 0x5061, 0x5064, 0x5080, 0x5082, 0x5085, 0x5088, 0x5091, 0x5094, 0x5101, 0x5104,
    0x5106, 0x5109, 0x5110, 0x5112, 0x5115, 0x5118, 0x5121, 0x5124, 0x5140, 0x5142, 0x5145, 0x5148, 0x5151, 0x5154, 0x5160, 0x5181,
    0x5184, 0x5190, 0x5200, 0x5205, 0x5208, 0x5211, 0x5214, 0x5220, 0x5241, 0x5244, 0x5250, 0x5269, 0x5280, 0x5401, 0x5404, 0x5406,
    0x5409, 0x5410, 0x5412, 0x5415, 0x5418, 0x5421, 0x5424, 0x5440, 0x5442, 0x5445, 0x5448, 0x5451, 0x5454, 0x5460, 0x5481, 0x5484,
    0x5490, 0x5500, 0x5502, 0x5505, 0x5508, 0x5511, 0x5514, 0x5520, 0x5541, 0x5544, 0x5550, 0x5580, 0x5601, 0x5604, 0x5610, 0x5626,
    0x5640, 0x5800, 0x5802, 0x5805, 0x5808, 0x5811, 0x5814, 0x5820, 0x5841, 0x5844, 0x5850, 0x585a, 0x5880, 0x5901, 0x5904, 0x5910,
    0x5940, 0x5a00, 0x5a19, 0x5a85, 0x5aa8, 0x6001, 0x6004, 0x6006, 0x6010, 0x6012, 0x6015, 0x6018, 0x6021, 0x6024, 0x6040, 0x6045,
    0x6048, 0x6051, 0x6054, 0x6060, 0x6084, 0x6090, 0x6100, 0x6102, 0x6105, 0x6108, 0x6111, 0x6114, 0x6120, 0x6141, 0x6144, 0x6150,
    0x6180, 0x6199, 0x6204, 0x6210, 0x6240, 0x6256, 0x62a1, 0x6400, 0x6405, 0x6408, 0x6411, 0x6414, 0x6420, 0x6441, 0x6444, 0x6450,
    0x6480, 0x6501, 0x6504, 0x6510, 0x6540, 0x654a, 0x6568, 0x6592, 0x6600, 0x6694, 0x6801, 0x6804, 0x6810, 0x6865, 0x6898, 0x6900,
    0x692a, 0x6a42, 0x6aa1, 0x8000, 0x8002, 0x8005, 0x8008, 0x8011, 0x8014, 0x8019, 0x8020, 0x8025, 0x8041, 0x8044, 0x8050, 0x8052,
    0x8055, 0x8058, 0x8061, 0x8080, 0x8085, 0x8091, 0x8094, 0x8101, 0x8104, 0x8109, 0x8110, 0x8112, 0x8115, 0x8118, 0x8121, 0x8124,
    0x8140, 0x8142, 0x8145, 0x8148, 0x8151, 0x8154, 0x8181, 0x8184, 0x8190, 0x81a9, 0x8200, 0x8205, 0x820a, 0x8211, 0x8214, 0x8241,
    0x8244, 0x8250, 0x8401, 0x8404, 0x8406, 0x8409, 0x8410, 0x8412, 0x8415, 0x8418, 0x8421, 0x8440, 0x8442, 0x8445, 0x8448, 0x8451,
    0x8454, 0x8460, 0x8481, 0x8484, 0x8490, 0x8500, 0x8502, 0x8505, 0x8508, 0x8511, 0x8514, 0x8520, 0x8541, 0x8544, 0x8550, 0x8580,
    0x858a, 0x8601, 0x8604, 0x8610, 0x8629, 0x8640, 0x8800, 0x8805, 0x8811, 0x8814, 0x8841, 0x8844, 0x8850, 0x88a2, 0x8901, 0x8904,
    0x8940, 0x8965, 0x8a22, 0x8a58, 0x8a5a, 0x8a82, 0x8aa2, 0x9001, 0x9004, 0x9009, 0x9010, 0x9012, 0x9015, 0x9018, 0x9024, 0x9040,
    0x9042, 0x9045, 0x9048, 0x9051, 0x9054, 0x9060, 0x9081, 0x9084, 0x9090, 0x9100, 0x9105, 0x9111, 0x9114, 0x9141, 0x9144, 0x9150,
    0x915a, 0x9201, 0x9204, 0x9210, 0x9240, 0x92a6, 0x9400, 0x9402, 0x9405, 0x9408, 0x9411, 0x9414, 0x9420, 0x9441, 0x9444, 0x9450,
    0x9480, 0x9496, 0x9501, 0x9504, 0x9510, 0x9540, 0x9598, 0x95a1, 0x9600, 0x9646, 0x9664, 0x9801, 0x9804, 0x9810, 0x9826, 0x9840,
    0x98a9, 0x9900, 0x9949, 0x9952, 0x9a90, 0xa000, 0xa005, 0xa00a, 0xa014, 0xa022, 0xa02a, 0xa041, 0xa044, 0xa050, 0xa0a2, 0xa0aa,
    0xa140, 0xa165, 0xa202, 0xa20a, 0xa222, 0xa228, 0xa22a, 0xa282, 0xa288, 0xa28a, 0xa2a8, 0xa401, 0xa404, 0xa410, 0xa440, 0xa489,
    0xa4a4, 0xa500, 0xa519, 0xa651, 0xa80a, 0xa828, 0xa8a2, 0xa954, 0xa986, 0xaa08, 0xaa0a, 0xaa20, 0xaa22, 0xaa28, 0xaa88, 0xaaaa,
};

static const uint16_t IQ3S_CODES[512] = {
    0x0000, 0x0001, 0x0002, 0x0005, 0x0007, 0x0008, 0x0009, 0x000a, 0x000c, 0x000e, 0x0010, 0x0011, 0x0015, 0x001b, 0x0020, 0x0022,
    0x0025, 0x0027, 0x0029, 0x002b, 0x0030, 0x0032, 0x0039, 0x003c, 0x003f, 0x0040, 0x0041, 0x0042, 0x0044, 0x0048, 0x0049, 0x004d,
    0x0050, 0x0053, 0x0057, 0x0059, 0x005d, 0x0064, 0x0071, 0x0075, 0x007a, 0x0080, 0x0081, 0x0085, 0x0087, 0x0088, 0x008b, 0x008e,
    0x0091, 0x0095, 0x0098, 0x009c, 0x00a2, 0x00a5, 0x00a7, 0x00a9, 0x00ab, 0x00b8, 0x00bb, 0x00c3, 0x00c9, 0x00cd, 0x00d0, 0x00d2,
    0x00d9, 0x00db, 0x00de, 0x00e4, 0x00e8, 0x00ea, 0x00f7, 0x00f9, 0x00fd, 0x0100, 0x010b, 0x010f, 0x0111, 0x0114, 0x011a, 0x0120,
    0x0123, 0x0129, 0x0138, 0x0142, 0x0144, 0x0150, 0x0152, 0x0156, 0x015b, 0x0161, 0x0165, 0x0167, 0x0176, 0x017b, 0x0186, 0x0189,
    0x018b, 0x0199, 0x01aa, 0x01b9, 0x01c0, 0x01c2, 0x01c4, 0x01d0, 0x01d2, 0x01d6, 0x01db, 0x01e8, 0x01ec, 0x0200, 0x0201, 0x0202,
    0x0204, 0x0208, 0x0209, 0x020b, 0x020d, 0x020f, 0x0210, 0x0212, 0x0219, 0x021c, 0x021e, 0x022c, 0x022e, 0x0231, 0x023a, 0x0240,
    0x0241, 0x0243, 0x0246, 0x0248, 0x024c, 0x0251, 0x0258, 0x025b, 0x0261, 0x0268, 0x026a, 0x0278, 0x027e, 0x0280, 0x028a, 0x028d,
    0x028f, 0x0290, 0x0294, 0x029a, 0x02a0, 0x02a3, 0x02ad, 0x02b0, 0x02ba, 0x02c1, 0x02c4, 0x02c7, 0x02c8, 0x02cb, 0x02d1, 0x02d7,
    0x02d8, 0x02dc, 0x02e1, 0x02f2, 0x02f8, 0x0303, 0x0305, 0x030a, 0x030c, 0x0319, 0x031b, 0x0322, 0x0326, 0x0328, 0x032c, 0x0341,
    0x0348, 0x034b, 0x0351, 0x0358, 0x035a, 0x0369, 0x0390, 0x0394, 0x0397, 0x03a4, 0x03a6, 0x03c1, 0x03c3, 0x03c8, 0x03ca, 0x03d1,
    0x03dd, 0x03e1, 0x03f2, 0x03f8, 0x0400, 0x0401, 0x0403, 0x0405, 0x0407, 0x0408, 0x040a, 0x040c, 0x040e, 0x0411, 0x0413, 0x0417,
    0x0418, 0x041a, 0x0421, 0x0423, 0x0425, 0x0428, 0x042a, 0x0437, 0x0438, 0x043b, 0x043d, 0x0440, 0x0442, 0x0448, 0x044b, 0x044f,
    0x0452, 0x0455, 0x0459, 0x045c, 0x0462, 0x0469, 0x0481, 0x0484, 0x0487, 0x0491, 0x0493, 0x0498, 0x049f, 0x04a1, 0x04ab, 0x04af,
    0x04b9, 0x04bc, 0x04c0, 0x04c2, 0x04c5, 0x04c9, 0x04d2, 0x04d4, 0x04d9, 0x04db, 0x04e2, 0x04e8, 0x04f6, 0x0501, 0x0507, 0x0510,
    0x0513, 0x051a, 0x051d, 0x0521, 0x053a, 0x053d, 0x0544, 0x0549, 0x0552, 0x055f, 0x0560, 0x056b, 0x0578, 0x0580, 0x0582, 0x0587,
    0x0591, 0x05ad, 0x05b1, 0x05c5, 0x05c9, 0x05d6, 0x05d8, 0x05e3, 0x05e8, 0x0602, 0x0609, 0x060b, 0x060d, 0x060f, 0x0612, 0x0619,
    0x061b, 0x061d, 0x0622, 0x0624, 0x0627, 0x0629, 0x0633, 0x0639, 0x0641, 0x0643, 0x0645, 0x064c, 0x0651, 0x0653, 0x0660, 0x0670,
    0x067a, 0x067e, 0x0680, 0x068a, 0x0690, 0x069a, 0x069c, 0x06a8, 0x06c1, 0x06c8, 0x06cc, 0x06d1, 0x06d3, 0x06d7, 0x06d8, 0x06e1,
    0x06e3, 0x06e7, 0x06ed, 0x06fb, 0x0703, 0x0709, 0x070e, 0x0712, 0x0719, 0x072a, 0x0730, 0x0734, 0x0741, 0x0748, 0x074a, 0x0755,
    0x075a, 0x0764, 0x076e, 0x077b, 0x078e, 0x07a1, 0x07c1, 0x07c3, 0x07d0, 0x07d2, 0x07dd, 0x0800, 0x0804, 0x080a, 0x0810, 0x0814,
    0x0817, 0x081a, 0x0821, 0x0828, 0x0838, 0x0842, 0x0847, 0x0849, 0x084b, 0x0852, 0x0858, 0x085d, 0x0863, 0x0869, 0x086d, 0x0881,
    0x0883, 0x0888, 0x088d, 0x0891, 0x089b, 0x08a0, 0x08af, 0x08b2, 0x08b8, 0x08c4, 0x08c9, 0x08cb, 0x08d0, 0x08d2, 0x08d9, 0x08dd,
    0x0900, 0x0902, 0x0914, 0x091f, 0x0920, 0x0939, 0x0945, 0x0947, 0x0951, 0x0972, 0x098b, 0x099c, 0x09b0, 0x09c8, 0x09cd, 0x09d8,
    0x09e3, 0x09e9, 0x0a02, 0x0a08, 0x0a0c, 0x0a12, 0x0a20, 0x0a24, 0x0a27, 0x0a2a, 0x0a36, 0x0a3c, 0x0a41, 0x0a43, 0x0a45, 0x0a4a,
    0x0a51, 0x0a5a, 0x0a7a, 0x0a80, 0x0a89, 0x0a93, 0x0a98, 0x0a9e, 0x0aab, 0x0ac2, 0x0ac7, 0x0ac8, 0x0ad7, 0x0ae4, 0x0ae9, 0x0af5,
    0x0afb, 0x0b01, 0x0b04, 0x0b10, 0x0b1a, 0x0b26, 0x0b4a, 0x0b56, 0x0b69, 0x0b6b, 0x0ba2, 0x0bc2, 0x0bc4, 0x0bd2, 0x0c09, 0x0c0b,
    0x0c0d, 0x0c19, 0x0c1b, 0x0c30, 0x0c40, 0x0c50, 0x0c57, 0x0c74, 0x0c8a, 0x0c9c, 0x0ca2, 0x0cad, 0x0cb2, 0x0cb8, 0x0cc0, 0x0ccc,
    0x0cd1, 0x0ce0, 0x0d15, 0x0d23, 0x0d32, 0x0d40, 0x0d43, 0x0d5c, 0x0d70, 0x0d85, 0x0da0, 0x0dc9, 0x0dcb, 0x0e00, 0x0e04, 0x0e07,
    0x0e10, 0x0e12, 0x0e1e, 0x0e20, 0x0e2c, 0x0e32, 0x0e42, 0x0e49, 0x0e54, 0x0e63, 0x0e65, 0x0e81, 0x0e84, 0x0e88, 0x0e8e, 0x0e91,
    0x0e98, 0x0ea9, 0x0ec2, 0x0eda, 0x0edd, 0x0eeb, 0x0f01, 0x0f05, 0x0f0b, 0x0f10, 0x0f28, 0x0f52, 0x0f62, 0x0f82, 0x0f99, 0x0fc0,
};

static uint64_t IQ2XXS_GRID[256];
static uint64_t IQ2S_GRID[1024];
static uint32_t IQ3S_GRID[512];
static uint8_t KSIGNS[128];

static void tables_init(void)
{
    static const uint8_t vals[3] = { 0x08, 0x19, 0x2b };
    if (IQ2XXS_GRID[0]) return;
    for (int i = 0; i < 128; i++) {
        /* ksigns_iq2xs[i]: i plus an eighth bit that makes the bit count even (src/IqTables.cs:10-21). */
        KSIGNS[i] = (uint8_t)(i | ((__builtin_popcount(i) & 1) << 7));
    }
    for (int i = 0; i < 256; i++) {
        uint64_t g = 0;
        for (int j = 0; j < 8; j++) g |= (uint64_t)vals[(IQ2XXS_CODES[i] >> (2 * j)) & 3] << (8 * j);
        IQ2XXS_GRID[i] = g;
    }
    for (int i = 0; i < 1024; i++) {
        uint64_t g = 0;
        for (int j = 0; j < 8; j++) g |= (uint64_t)vals[(IQ2S_CODES[i] >> (2 * j)) & 3] << (8 * j);
        IQ2S_GRID[i] = g;
    }
    for (int i = 0; i < 512; i++) {
        uint32_t g = 0;
        for (int j = 0; j < 4; j++) g |= (uint32_t)(2 * ((IQ3S_CODES[i] >> (3 * j)) & 7) + 1) << (8 * j);
        IQ3S_GRID[i] = g;
    }
}

const uint64_t *wlo_iq2xxs_grid(void) { tables_init(); return IQ2XXS_GRID; }
const uint64_t *wlo_iq2s_grid(void) { tables_init(); return IQ2S_GRID; }
const uint32_t *wlo_iq3s_grid(void) { tables_init(); return IQ3S_GRID; }
const uint8_t *wlo_ksigns_iq2xs(void) { tables_init(); return KSIGNS; }
const int8_t *wlo_kvalues_iq4nl(void) { return KVALUES; }

/* ------------------------------------------------------------ decoders (src/Quants.cs) */

/* get_scale_min_k4 (src/Quants.cs:321-330). */
static void scale_min_k4(int j, const uint8_t *q, int *sc, int *m)
{
    if (j < 4) { *sc = q[j] & 63; *m = q[j + 4] & 63; }
    else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* src/Quants.cs:251-259: y = q * d. */
static void dec_q8_0(const uint8_t *b, int64_t n, float *y)
{
    for (int64_t i = 0; i < n / 32; i++, b += 34, y += 32) {
        float d = H(b);
        const int8_t *q = (const int8_t *)(b + 2);
        for (int j = 0; j < 32; j++) y[j] = (float)q[j] * d;
    }
}

/* src/Quants.cs:332-350: d1 = d*s, m1 = dmin*m, y = d1*nibble - m1. */
static void dec_q4_k(const uint8_t *b, int64_t n, float *y)
{
    for (int64_t i = 0; i < n / 256; i++, b += 144) {
        float d = H(b), min = H(b + 2);
        const uint8_t *sc = b + 4, *q = b + 16;
        for (int j = 0, idx = 0; j < 256; j += 64, q += 32, idx += 2) {
            int s, m;
            scale_min_k4(idx, sc, &s, &m);
            float d1 = d * (float)s, m1 = min * (float)m;
            scale_min_k4(idx + 1, sc, &s, &m);
            float d2 = d * (float)s, m2 = min * (float)m;
            for (int l = 0; l < 32; l++) *y++ = d1 * (float)(q[l] & 0xF) - m1;
            for (int l = 0; l < 32; l++) *y++ = d2 * (float)(q[l] >> 4) - m2;
        }
    }
}

/* src/Quants.cs:189-200: y = (nibble - 8) * d; low nibbles give values 0-15, high 16-31. */
static void dec_q4_0(const uint8_t *b, int64_t n, float *y)
{
    for (int64_t i = 0; i < n / 32; i++, b += 18, y += 32) {
        float d = H(b);
        const uint8_t *q = b + 2;
        for (int j = 0; j < 16; j++) {
            y[j] = (float)((q[j] & 0xF) - 8) * d;
            y[j + 16] = (float)((q[j] >> 4) - 8) * d;
        }
    }
}

/* src/Quants.cs:202-214: y = nibble * d + m. */
static void dec_q4_1(const uint8_t *b, int64_t n, float *y)
{
    for (int64_t i = 0; i < n / 32; i++, b += 20, y += 32) {
        float d = H(b), m = H(b + 2);
        const uint8_t *q = b + 4;
        for (int j = 0; j < 16; j++) {
            y[j] = (float)(q[j] & 0xF) * d + m;
            y[j + 16] = (float)(q[j] >> 4) * d + m;
        }
    }
}

/* src/Quants.cs:216-231: the fifth bit of value j is bit j of qh (value j + 16: bit j + 16);
 * y = (q5 - 16) * d. */
static void dec_q5_0(const uint8_t *b, int64_t n, float *y)
{
    for (int64_t i = 0; i < n / 32; i++, b += 22, y += 32) {
        float d = H(b);
        uint32_t qh = U32(b + 2);
        const uint8_t *q = b + 6;
        for (int j = 0; j < 16; j++) {
            int h0 = (int)(((qh >> j) << 4) & 0x10), h1 = (int)((qh >> (j + 12)) & 0x10);
            y[j] = (float)(((q[j] & 0xF) | h0) - 16) * d;
            y[j + 16] = (float)(((q[j] >> 4) | h1) - 16) * d;
        }
    }
}

/* src/Quants.cs:233-249: y = q5 * d + m. */
static void dec_q5_1(const uint8_t *b, int64_t n, float *y)
{
    for (int64_t i = 0; i < n / 32; i++, b += 24, y += 32) {
        float d = H(b), m = H(b + 2);
        uint32_t qh = U32(b + 4);
        const uint8_t *q = b + 8;
        for (int j = 0; j < 16; j++) {
            int h0 = (int)(((qh >> j) << 4) & 0x10), h1 = (int)((qh >> (j + 12)) & 0x10);
            y[j] = (float)((q[j] & 0xF) | h0) * d + m;
            y[j + 16] = (float)((q[j] >> 4) | h1) * d + m;
        }
    }
}

/* src/Quants.cs:261-285: block = scales[16] | qs[64] | d | dmin. Each 128-value half reads
 * 32 qs bytes four times (2-bit fields at shifts 0, 2, 4, 6); each run of 16 values takes
 * one scale byte: dl = d * (s & 15), ml = dmin * (s >> 4), y = dl * q2 - ml. */
static void dec_q2_k(const uint8_t *b, int64_t n, float *y)
{
    for (int64_t i = 0; i < n / 256; i++, b += 84) {
        const uint8_t *sc = b, *q = b + 16;
        float d = H(b + 80), min = H(b + 82);
        int idx = 0;
        for (int k = 0; k < 256; k += 128, q += 32) {
            for (int j = 0, shift = 0; j < 4; j++, shift += 2) {
                for (int half = 0; half < 2; half++) {
                    int s = sc[idx++];
                    float dl = d * (float)(s & 0xF), ml = min * (float)(s >> 4);
                    for (int l = 0; l < 16; l++) *y++ = dl * (float)((q[l + 16 * half] >> shift) & 3) - ml;
                }
            }
        }
    }
}

/* The sixteen 6-bit Q3_K scales from their 12 packed bytes, by the reference's kmask shuffle
 * (src/Quants.cs:295-301): the low four bits of scale i are the low nibble of byte i (i < 8)
 * or the high nibble of byte i - 8; the top two bits are bits 2*(i/4)..+1 of byte 8 + i%4. */
static void q3k_scales(const uint8_t *s12, int *scales)
{
    uint32_t a0 = U32(s12), a1 = U32(s12 + 4), tmp = U32(s12 + 8);
    uint32_t aux[4];
    const uint32_t kmask1 = 0x03030303u, kmask2 = 0x0f0f0f0fu;
    aux[2] = ((a0 >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
    aux[3] = ((a1 >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
    aux[0] = (a0 & kmask2) | (((tmp >> 0) & kmask1) << 4);
    aux[1] = (a1 & kmask2) | (((tmp >> 2) & kmask1) << 4);
    for (int i = 0; i < 16; i++) scales[i] = (int)(int8_t)(uint8_t)(aux[i / 4] >> (8 * (i % 4)));
}

/* src/Quants.cs:287-319: block = hmask[32] | qs[64] | scales[12] | d. Runs of 16 values as in
 * Q2_K; the high bit of value l of run (k, j) is bit 4*(k/128) + j of hmask[l], and a clear
 * bit subtracts 4: y = (d * (sc - 32)) * (q2 - (h ? 0 : 4)). */
static void dec_q3_k(const uint8_t *b, int64_t n, float *y)
{
    for (int64_t i = 0; i < n / 256; i++, b += 110) {
        const uint8_t *hm = b, *q = b + 32;
        float dall = H(b + 108);
        int scales[16];
        q3k_scales(b + 96, scales);
        int idx = 0, m = 1;
        for (int k = 0; k < 256; k += 128, q += 32) {
            for (int j = 0, shift = 0; j < 4; j++, shift += 2, m <<= 1) {
                for (int half = 0; half < 2; half++) {
                    float dl = dall * (float)(scales[idx++] - 32);
                    for (int l = 16 * half; l < 16 * half + 16; l++)
                        *y++ = dl * (float)(((q[l] >> shift) & 3) - ((hm[l] & m) ? 0 : 4));
                }
            }
        }
    }
}

/* src/Quants.cs:352-370: as Q4_K with a fifth bit per value from qh[l] (bit 2j for the low
 * nibbles of group j, bit 2j+1 for the high ones): y = d1 * q5 - m1. */
static void dec_q5_k(const uint8_t *b, int64_t n, float *y)
{
    for (int64_t i = 0; i < n / 256; i++, b += 176) {
        float d = H(b), min = H(b + 2);
        const uint8_t *sc = b + 4, *qh = b + 16, *ql = b + 48;
        int idx = 0, u1 = 1, u2 = 2;
        for (int j = 0; j < 256; j += 64, ql += 32, idx += 2, u1 <<= 2, u2 <<= 2) {
            int s, m;
            scale_min_k4(idx, sc, &s, &m);
            float d1 = d * (float)s, m1 = min * (float)m;
            scale_min_k4(idx + 1, sc, &s, &m);
            float d2 = d * (float)s, m2 = min * (float)m;
            for (int l = 0; l < 32; l++) *y++ = d1 * (float)((ql[l] & 0xF) + ((qh[l] & u1) ? 16 : 0)) - m1;
            for (int l = 0; l < 32; l++) *y++ = d2 * (float)((ql[l] >> 4) + ((qh[l] & u2) ? 16 : 0)) - m2;
        }
    }
}

/* src/IQuants.cs:45-58: y = d * kvalues[nibble]; low nibbles give values 0-15, high 16-31. */
static void dec_iq4_nl(const uint8_t *b, int64_t n, float *y)
{
    for (int64_t i = 0; i < n / 32; i++, b += 18, y += 32) {
        float d = H(b);
        const uint8_t *q = b + 2;
        for (int j = 0; j < 16; j++) {
            y[j] = d * (float)KVALUES[q[j] & 0xF];
            y[j + 16] = d * (float)KVALUES[q[j] >> 4];
        }
    }
}

/* src/Quants.cs:372-396: y = (d * sc) * (q6 - 32). */
static void dec_q6_k(const uint8_t *b, int64_t n, float *y)
{
    for (int64_t i = 0; i < n / 256; i++, b += 210) {
        float d = H(b + 208);
        const uint8_t *ql = b, *qh = b + 128;
        const int8_t *sc = (const int8_t *)(b + 192);
        for (int k = 0; k < 256; k += 128, y += 128, ql += 64, qh += 32, sc += 8) {
            for (int l = 0; l < 32; l++) {
                int s = l / 16;
                int q1 = ((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                int q2 = ((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                y[l] = d * (float)sc[s] * (float)q1;
                y[l + 32] = d * (float)sc[s + 2] * (float)q2;
                y[l + 64] = d * (float)sc[s + 4] * (float)q3;
                y[l + 96] = d * (float)sc[s + 6] * (float)q4;
            }
        }
    }
}

/* src/IQuants.cs:60-80: ls = low4 | high2 << 4, dl = d * (ls - 32), y = dl * kvalues[nibble]. */
static void dec_iq4_xs(const uint8_t *b, int64_t n, float *y)
{
    for (int64_t i = 0; i < n / 256; i++, b += 136) {
        float d = H(b);
        int scales_h = b[2] | (b[3] << 8);
        const uint8_t *scales_l = b + 4, *q = b + 8;
        for (int ib = 0; ib < 8; ib++, q += 16, y += 32) {
            int ls = ((scales_l[ib / 2] >> (4 * (ib % 2))) & 0xF) | (((scales_h >> (2 * ib)) & 3) << 4);
            float dl = d * (float)(ls - 32);
            for (int j = 0; j < 16; j++) {
                y[j] = dl * (float)KVALUES[q[j] & 0xF];
                y[j + 16] = dl * (float)KVALUES[q[j] >> 4];
            }
        }
    }
}

/* src/IQuants.cs:147-170: db = d * (0.5 + scale4) * 0.25, y = db * gridbyte * sign. */
static void dec_iq2_xxs(const uint8_t *b, int64_t n, float *y)
{
    tables_init();
    for (int64_t i = 0; i < n / 256; i++, b += 66) {
        float d = H(b);
        const uint8_t *qs = b + 2;
        for (int ib32 = 0; ib32 < 8; ib32++) {
            uint32_t aux0 = U32(qs + 8 * ib32), aux1 = U32(qs + 8 * ib32 + 4);
            float db = d * (0.5f + (float)(aux1 >> 28)) * 0.25f;
            for (int l = 0; l < 4; l++) {
                uint64_t g = IQ2XXS_GRID[(aux0 >> (8 * l)) & 0xFF];
                int signs = KSIGNS[(aux1 >> (7 * l)) & 127];
                for (int j = 0; j < 8; j++)
                    y[j] = db * (float)(uint8_t)(g >> (8 * j)) * ((signs & (1 << j)) ? -1.0f : 1.0f);
                y += 8;
            }
        }
    }
}

/* IQ3_S (src/IQuants.cs:112-143): block = d, qs[64], qh[8], signs[32], scales[4] (110 bytes).
 * Per 32 values: db = d * (1 + 2 * scale nibble); grid index = qs byte plus one qh bit; each
 * grid entry gives 4 values, each sign byte 8. */
static void dec_iq3_s(const uint8_t *b, int64_t n, float *y)
{
    tables_init();
    for (int64_t i = 0; i < n / 256; i++, b += 110) {
        float d = H(b);
        const uint8_t *qs = b + 2, *qh = b + 66, *signs = b + 74, *scales = b + 106;
        for (int ib32 = 0; ib32 < 8; ib32 += 2) {
            float db1 = d * (float)(1 + 2 * (scales[ib32 / 2] & 0xF));
            float db2 = d * (float)(1 + 2 * (scales[ib32 / 2] >> 4));
            for (int half = 0; half < 2; half++) {
                float db = half == 0 ? db1 : db2;
                int h = qh[half];
                for (int l = 0; l < 4; l++) {
                    uint32_t g1 = IQ3S_GRID[qs[2 * l] | ((h << (8 - 2 * l)) & 256)];
                    uint32_t g2 = IQ3S_GRID[qs[2 * l + 1] | ((h << (7 - 2 * l)) & 256)];
                    for (int j = 0; j < 4; j++) {
                        y[j] = db * (float)(uint8_t)(g1 >> (8 * j)) * ((signs[l] & (1 << j)) ? -1.0f : 1.0f);
                        y[j + 4] = db * (float)(uint8_t)(g2 >> (8 * j)) * ((signs[l] & (1 << (j + 4))) ? -1.0f : 1.0f);
                    }
                    y += 8;
                }
                qs += 8;
                signs += 4;
            }
            qh += 2;
        }
    }
}

/* IQ2_S (src/IQuants.cs:199-222): block = d, qs[32] grid bytes, signs[32], qh[8], scales[8]
 * (82 bytes). Per 32 values two 4-bit scales, db = d * (0.5 + nibble) * 0.25; grid index =
 * qs byte plus two qh bits (10 bits); one sign byte per 8 values. */
static void dec_iq2_s(const uint8_t *b, int64_t n, float *y)
{
    tables_init();
    for (int64_t i = 0; i < n / 256; i++, b += 82) {
        float d = H(b);
        const uint8_t *qs = b + 2, *signs = b + 34, *qh = b + 66, *scales = b + 74;
        for (int ib32 = 0; ib32 < 8; ib32++) {
            float db0 = d * (0.5f + (float)(scales[ib32] & 0xF)) * 0.25f;
            float db1 = d * (0.5f + (float)(scales[ib32] >> 4)) * 0.25f;
            for (int l = 0; l < 4; l++) {
                float dl = l < 2 ? db0 : db1;
                uint64_t g = IQ2S_GRID[qs[l] | ((qh[ib32] << (8 - 2 * l)) & 0x300)];
                for (int j = 0; j < 8; j++)
                    y[j] = dl * (float)(uint8_t)(g >> (8 * j)) * ((signs[l] & (1 << j)) ? -1.0f : 1.0f);
                y += 8;
            }
            qs += 4;
            signs += 4;
        }
    }
}

static float bf16_to_float(uint16_t v) { return bits_to_float((uint32_t)v << 16); }

/* Quants.DecodeRow dispatch (src/Quants.cs:32-52; src/IQuants.cs:27-42). */
int wlo_decode_row(int t, const uint8_t *src, int64_t n, float *dst)
{
    switch (t) {
    case WLO_F32: memcpy(dst, src, (size_t)n * 4); return 0;
    case WLO_F16: for (int64_t i = 0; i < n; i++) dst[i] = H(src + 2 * i); return 0;
    case WLO_BF16: for (int64_t i = 0; i < n; i++) dst[i] = bf16_to_float((uint16_t)(src[2 * i] | src[2 * i + 1] << 8)); return 0;
    case WLO_Q4_0: dec_q4_0(src, n, dst); return 0;
    case WLO_Q4_1: dec_q4_1(src, n, dst); return 0;
    case WLO_Q5_0: dec_q5_0(src, n, dst); return 0;
    case WLO_Q5_1: dec_q5_1(src, n, dst); return 0;
    case WLO_Q8_0: dec_q8_0(src, n, dst); return 0;
    case WLO_Q2_K: dec_q2_k(src, n, dst); return 0;
    case WLO_Q3_K: dec_q3_k(src, n, dst); return 0;
    case WLO_Q4_K: dec_q4_k(src, n, dst); return 0;
    case WLO_Q5_K: dec_q5_k(src, n, dst); return 0;
    case WLO_Q6_K: dec_q6_k(src, n, dst); return 0;
    case WLO_IQ4_NL: dec_iq4_nl(src, n, dst); return 0;
    case WLO_IQ4_XS: dec_iq4_xs(src, n, dst); return 0;
    case WLO_IQ2_XXS: dec_iq2_xxs(src, n, dst); return 0;
    case WLO_IQ3_S: dec_iq3_s(src, n, dst); return 0;
    case WLO_IQ2_S: dec_iq2_s(src, n, dst); return 0;
    }
    return -1;
}

/* ---------------------------------------------------------- fused dots (src/Quants.cs) */

/* Transformer.Dot (src/Transformer.cs:466-477): four partial chains, then (s0+s1)+(s2+s3). */
static float dot_f32(const float *a, const float *b, int n)
{
    float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
    int i = 0;
    for (; i + 4 <= n; i += 4) {
        s0 += a[i] * b[i]; s1 += a[i + 1] * b[i + 1];
        s2 += a[i + 2] * b[i + 2]; s3 += a[i + 3] * b[i + 3];
    }
    for (; i < n; i++) s0 += a[i] * b[i];
    return (s0 + s1) + (s2 + s3);
}

/* Quants.DotRow (src/Quants.cs:67-187). */
int wlo_dot_row(int t, const uint8_t *b, const float *x, int n, float *out)
{
    switch (t) {
    case WLO_F32:
        /* DotRow hands the row to Transformer.Dot as a float pointer (src/Quants.cs:71). */
        *out = dot_f32((const float *)b, x, n);
        return 0;
    case WLO_F16: case WLO_BF16: {          /* src/Quants.cs:72-85 */
        float s0 = 0, s1 = 0;
        for (int i = 0; i < n; i += 2) {
            uint16_t h0 = (uint16_t)(b[2 * i] | b[2 * i + 1] << 8), h1 = (uint16_t)(b[2 * i + 2] | b[2 * i + 3] << 8);
            float w0 = t == WLO_F16 ? wlo_half_to_float(h0) : bf16_to_float(h0);
            float w1 = t == WLO_F16 ? wlo_half_to_float(h1) : bf16_to_float(h1);
            s0 += w0 * x[i]; s1 += w1 * x[i + 1];
        }
        *out = s0 + s1;
        return 0;
    }
    case WLO_Q8_0: {                          /* src/Quants.cs:86-97 */
        float sum = 0;
        for (int i = 0; i < n / 32; i++, b += 34, x += 32) {
            const int8_t *q = (const int8_t *)(b + 2);
            float s0 = 0, s1 = 0;
            for (int j = 0; j < 32; j += 2) { s0 += (float)q[j] * x[j]; s1 += (float)q[j + 1] * x[j + 1]; }
            sum += H(b) * (s0 + s1);
        }
        *out = sum;
        return 0;
    }
    case WLO_Q4_0: {                          /* src/Quants.cs:98-109 */
        float sum = 0;
        for (int i = 0; i < n / 32; i++, b += 18, x += 32) {
            const uint8_t *q = b + 2;
            float s0 = 0, s1 = 0;
            for (int j = 0; j < 16; j++) { s0 += (float)((q[j] & 0xF) - 8) * x[j]; s1 += (float)((q[j] >> 4) - 8) * x[j + 16]; }
            sum += H(b) * (s0 + s1);
        }
        *out = sum;
        return 0;
    }
    case WLO_Q5_K: {                          /* src/Quants.cs:134-158 */
        float sum = 0;
        for (int i = 0; i < n / 256; i++, b += 176) {
            float d = H(b), min = H(b + 2);
            const uint8_t *sc = b + 4, *qh = b + 16, *ql = b + 48;
            int u1 = 1, u2 = 2;
            for (int j = 0; j < 4; j++, ql += 32, x += 64, u1 <<= 2, u2 <<= 2) {
                int s1, m1, s2, m2;
                scale_min_k4(2 * j, sc, &s1, &m1);
                scale_min_k4(2 * j + 1, sc, &s2, &m2);
                float a1 = 0, a2 = 0, x1 = 0, x2 = 0;
                for (int l = 0; l < 32; l++) {
                    float xl = x[l], xh = x[l + 32];
                    a1 += (float)((ql[l] & 0xF) + ((qh[l] & u1) ? 16 : 0)) * xl; x1 += xl;
                    a2 += (float)((ql[l] >> 4) + ((qh[l] & u2) ? 16 : 0)) * xh; x2 += xh;
                }
                sum += d * ((float)s1 * a1 + (float)s2 * a2) - min * ((float)m1 * x1 + (float)m2 * x2);
            }
        }
        *out = sum;
        return 0;
    }
    case WLO_Q4_K: {                          /* src/Quants.cs:110-133 */
        float sum = 0;
        for (int i = 0; i < n / 256; i++, b += 144) {
            float d = H(b), min = H(b + 2);
            const uint8_t *sc = b + 4, *q = b + 16;
            for (int j = 0; j < 4; j++, q += 32, x += 64) {
                int s1, m1, s2, m2;
                scale_min_k4(2 * j, sc, &s1, &m1);
                scale_min_k4(2 * j + 1, sc, &s2, &m2);
                float a1 = 0, a2 = 0, x1 = 0, x2 = 0;
                for (int l = 0; l < 32; l++) {
                    float xl = x[l], xh = x[l + 32];
                    a1 += (float)(q[l] & 0xF) * xl; x1 += xl;
                    a2 += (float)(q[l] >> 4) * xh; x2 += xh;
                }
                sum += d * ((float)s1 * a1 + (float)s2 * a2) - min * ((float)m1 * x1 + (float)m2 * x2);
            }
        }
        *out = sum;
        return 0;
    }
    case WLO_Q6_K: {                          /* src/Quants.cs:159-184 */
        float sum = 0, acc[8];
        for (int i = 0; i < n / 256; i++, b += 210) {
            float d = H(b + 208);
            const uint8_t *ql = b, *qh = b + 128;
            const int8_t *sc = (const int8_t *)(b + 192);
            for (int k = 0; k < 2; k++, ql += 64, qh += 32, sc += 8, x += 128) {
                for (int g = 0; g < 8; g++) acc[g] = 0;
                for (int l = 0; l < 32; l++) {
                    int s = l >> 4;
                    acc[s] += (float)(((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32) * x[l];
                    acc[s + 2] += (float)(((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32) * x[l + 32];
                    acc[s + 4] += (float)(((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32) * x[l + 64];
                    acc[s + 6] += (float)(((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32) * x[l + 96];
                }
                float part = 0;
                for (int g = 0; g < 8; g++) part += (float)sc[g] * acc[g];
                sum += d * part;
            }
        }
        *out = sum;
        return 0;
    }
    }
    return -1;
}

/* ------------------------------------------------------- FastMath.Block (src/FastMath.cs) */

/* src/FastMath.cs:216-264: one accumulator chain per (row, token), summed in index order;
 * 4 rows x 2 tokens per pass, then the token tail, then the row tail. */
void wlo_block(const float *w, int ws, int nr, const float *x, int xs, int nt, int cols, float *y, int ys)
{
    int r = 0;
    for (; r + 4 <= nr; r += 4) {
        const float *w0 = w + (int64_t)r * ws, *w1 = w0 + ws, *w2 = w1 + ws, *w3 = w2 + ws;
        int t = 0;
        for (; t + 2 <= nt; t += 2) {
            const float *xa = x + (int64_t)t * xs, *xb = xa + xs;
            float a0 = 0, a1 = 0, a2 = 0, a3 = 0, b0 = 0, b1 = 0, b2 = 0, b3 = 0;
            for (int i = 0; i < cols; i++) {
                float va = xa[i], vb = xb[i];
                float u0 = w0[i], u1 = w1[i], u2 = w2[i], u3 = w3[i];
                a0 += u0 * va; a1 += u1 * va; a2 += u2 * va; a3 += u3 * va;
                b0 += u0 * vb; b1 += u1 * vb; b2 += u2 * vb; b3 += u3 * vb;
            }
            float *ya = y + (int64_t)t * ys + r, *yb = ya + ys;
            ya[0] = a0; ya[1] = a1; ya[2] = a2; ya[3] = a3;
            yb[0] = b0; yb[1] = b1; yb[2] = b2; yb[3] = b3;
        }
        for (; t < nt; t++) {
            const float *xa = x + (int64_t)t * xs;
            float a0 = 0, a1 = 0, a2 = 0, a3 = 0;
            for (int i = 0; i < cols; i++) {
                float va = xa[i];
                a0 += w0[i] * va; a1 += w1[i] * va; a2 += w2[i] * va; a3 += w3[i] * va;
            }
            float *ya = y + (int64_t)t * ys + r;
            ya[0] = a0; ya[1] = a1; ya[2] = a2; ya[3] = a3;
        }
    }
    for (; r < nr; r++) {
        const float *wr = w + (int64_t)r * ws;
        for (int t = 0; t < nt; t++) {
            const float *xa = x + (int64_t)t * xs;
            float s = 0;
            for (int i = 0; i < cols; i++) s += wr[i] * xa[i];
            y[(int64_t)t * ys + r] = s;
        }
    }
}

/* ------------------------------------------------- MatMul dispatch (src/Transformer.cs) */

#define ROW_TILE 32   /* src/Transformer.cs:479 */

static int n_threads(int threads)
{
#ifdef _OPENMP
    return threads > 0 ? threads : omp_get_max_threads();
#else
    (void)threads;
    return 1;
#endif
}

/* Transformer.MatMul (src/Transformer.cs:483-537) without --int-dot, plus MatMulEach
 * (src/Transformer.cs:544-561) when each_token is set. Tiles of 32 rows run in parallel. */
int wlo_matmul(int type, const uint8_t *data, int rows, int cols, int64_t row_bytes,
               const float *x, int T, float *y, int each_token, int threads)
{
    if (!wlo_can_decode(type)) return -1;
    int tiles = (rows + ROW_TILE - 1) / ROW_TILE;
    int nth = n_threads(threads);
    if ((T == 1 || each_token) && wlo_can_dot(type)) {
        /* T == 1: DotRow per row (:494-502); each_token: DotRow per (row, token) (:551-560). */
        #pragma omp parallel for schedule(dynamic, 1) num_threads(nth)
        for (int tile = 0; tile < tiles; tile++) {
            int r0 = tile * ROW_TILE, r1 = r0 + ROW_TILE < rows ? r0 + ROW_TILE : rows;
            for (int r = r0; r < r1; r++)
                for (int t = 0; t < T; t++)
                    wlo_dot_row(type, data + (int64_t)r * row_bytes, x + (int64_t)t * cols, cols, y + (int64_t)t * rows + r);
        }
        return 0;
    }
    /* Decode a 32-row tile, then Block (:526-536). */
    #pragma omp parallel num_threads(nth)
    {
        float *scratch = (float *)malloc(sizeof(float) * ROW_TILE * (size_t)cols);
        #pragma omp for schedule(dynamic, 1)
        for (int tile = 0; tile < tiles; tile++) {
            int r0 = tile * ROW_TILE, r1 = r0 + ROW_TILE < rows ? r0 + ROW_TILE : rows;
            for (int r = r0; r < r1; r++)
                wlo_decode_row(type, data + (int64_t)r * row_bytes, cols, scratch + (int64_t)(r - r0) * cols);
            wlo_block(scratch, cols, r1 - r0, x, cols, T, cols, y + r0, rows);
        }
        free(scratch);
    }
    return 0;
}

static int64_t row_bytes_of(int type, int cols)
{
    int be, bb;
    if (!wlo_layout(type, &be, &bb)) return -1;
    return (int64_t)(cols / be) * bb;
}

/* MatMul's dispatch (src/Transformer.cs:483-494) under a mode: the integer branch first when
 * IntDot is on and applies, then MatMulEach or the plain float product. */
static int matmul_mode(int type, const uint8_t *data, int rows, int cols, int64_t row_bytes,
                       const float *x, int T, float *y, int mode, int threads)
{
    if ((mode & WLO_INT_DOT) && wlo_can_int_dot(type) && wlo_int_fits(type, cols))
        return wlo_int_matmul(type, data, rows, cols, row_bytes, x, T, y, threads);
    return wlo_matmul(type, data, rows, cols, row_bytes, x, T, y, mode & WLO_EACH_TOKEN, threads);
}

/* SwiGlu (src/Transformer.cs:241-251). The exponential is .NET Math.Exp on a double, cast
 * to float; libm exp stands in for it. each_token: the WLO_EACH_TOKEN / WLO_INT_DOT mode. */
int wlo_swiglu(int gtype, const uint8_t *gate, int64_t grb, int utype, const uint8_t *up, int64_t urb,
               int dtype, const uint8_t *down, int64_t drb, int ff, int embd,
               const float *x, int T, float *out, int each_token, int threads)
{
    float *g = (float *)malloc(sizeof(float) * (size_t)T * ff);
    float *u = (float *)malloc(sizeof(float) * (size_t)T * ff);
    int rc = matmul_mode(gtype, gate, ff, embd, grb, x, T, g, each_token, threads);
    if (!rc) rc = matmul_mode(utype, up, ff, embd, urb, x, T, u, each_token, threads);
    if (!rc) {
        for (int64_t i = 0; i < (int64_t)T * ff; i++) {
            float a = g[i];
            g[i] = a / (1.0f + (float)exp((double)(-a))) * u[i];
        }
        rc = matmul_mode(dtype, down, embd, ff, drb, g, T, out, each_token, threads);
    }
    free(g); free(u);
    return rc;
}

#define MIN_EXPERT_WEIGHT_SUM 6.103515625e-5f   /* src/Transformer.cs:253 */

/* Route (src/Transformer.cs:315-340): softmax with a double denominator, top-k with ties to
 * the lower id, optional renormalisation clamped at the smallest fp16 normal. */
void wlo_route(const float *logits, int n, int k, int renorm, int *sel, float *wts, int *count)
{
    if (n <= 0 || k <= 0 || k > n) return;
    float max = -INFINITY;
    for (int i = 0; i < n; i++) if (logits[i] > max) max = logits[i];
    float *p = (float *)malloc(sizeof(float) * (size_t)n);
    char *taken = (char *)calloc((size_t)n, 1);
    double sum = 0;
    for (int i = 0; i < n; i++) { p[i] = (float)exp((double)(logits[i] - max)); sum += p[i]; }
    float inv = (float)(1.0 / sum);
    for (int i = 0; i < n; i++) p[i] *= inv;
    float chosen = 0;
    for (int j = 0; j < k; j++) {
        int best = -1;
        for (int i = 0; i < n; i++) if (!taken[i] && (best < 0 || p[i] > p[best])) best = i;
        taken[best] = 1;
        sel[j] = best; wts[j] = p[best];
        chosen += p[best];
        if (count) count[best]++;
    }
    if (renorm) {
        float div = chosen > MIN_EXPERT_WEIGHT_SUM ? chosen : MIN_EXPERT_WEIGHT_SUM;
        for (int j = 0; j < k; j++) wts[j] /= div;
    }
    free(p); free(taken);
}

/* MoeFfn (src/Transformer.cs:259-294) after the router MatMul: route every token, then for
 * each expert in ascending id gather its tokens, run SwiGlu on the expert's slices and
 * scatter-add the weighted rows. */
int wlo_moe_ffn(const float *logits, int ne, int k, int renorm,
                int gtype, const uint8_t *gate, int utype, const uint8_t *up,
                int dtype, const uint8_t *down, int ff, int embd,
                const float *x, int T, float *out, int each_token, int threads, int *expert_runs)
{
    int64_t grb = row_bytes_of(gtype, embd), urb = row_bytes_of(utype, embd), drb = row_bytes_of(dtype, ff);
    if (grb < 0 || urb < 0 || drb < 0) return -1;
    int *sel = (int *)malloc(sizeof(int) * (size_t)T * k);
    float *wts = (float *)malloc(sizeof(float) * (size_t)T * k);
    int *count = (int *)calloc((size_t)ne, sizeof(int));
    for (int t = 0; t < T; t++) wlo_route(logits + (int64_t)t * ne, ne, k, renorm, sel + t * k, wts + t * k, count);
    memset(out, 0, sizeof(float) * (size_t)T * embd);
    int rc = 0, runs = 0;
    for (int e = 0; e < ne && !rc; e++) {
        int n = count[e];
        if (!n) continue;
        int *toks = (int *)malloc(sizeof(int) * (size_t)n);
        float *w = (float *)malloc(sizeof(float) * (size_t)n);
        float *xe = (float *)malloc(sizeof(float) * (size_t)n * embd);
        float *ye = (float *)malloc(sizeof(float) * (size_t)n * embd);
        int at = 0;
        for (int t = 0; t < T; t++)
            for (int j = 0; j < k; j++)
                if (sel[t * k + j] == e) {
                    toks[at] = t; w[at] = wts[t * k + j];
                    memcpy(xe + (int64_t)at * embd, x + (int64_t)t * embd, sizeof(float) * (size_t)embd);
                    at++;
                }
        runs++;
        rc = wlo_swiglu(gtype, gate + (int64_t)e * ff * grb, grb, utype, up + (int64_t)e * ff * urb, urb,
                        dtype, down + (int64_t)e * embd * drb, drb, ff, embd, xe, n, ye, each_token, threads);
        for (int i = 0; i < n && !rc; i++) {
            float *o = out + (int64_t)toks[i] * embd;
            const float *r = ye + (int64_t)i * embd;
            for (int d = 0; d < embd; d++) o[d] += w[i] * r[d];
        }
        free(toks); free(w); free(xe); free(ye);
    }
    if (expert_runs) *expert_runs = runs;
    free(sel); free(wts); free(count);
    return rc;
}

/* ---------------------------------------------- test matrices (tests/TinyModels.cs) */

/* Offsets of the fp16 scale fields per type (tests/TinyModels.cs:314-329). */
static int scale_fields(int t, int *f)
{
    switch (t) {
    case WLO_Q4_0: case WLO_Q5_0: case WLO_Q8_0: case WLO_IQ4_NL: case WLO_IQ4_XS: case WLO_IQ2_XXS:
    case WLO_IQ3_S: case WLO_IQ2_S:
        f[0] = 0; return 1;
    case WLO_Q4_1: case WLO_Q5_1: case WLO_Q4_K: case WLO_Q5_K: f[0] = 0; f[1] = 2; return 2;
    case WLO_Q2_K: f[0] = 80; f[1] = 82; return 2;
    case WLO_Q3_K: f[0] = 108; return 1;
    case WLO_Q6_K: f[0] = 208; return 1;
    }
    return 0;
}

/* TinyModels.Matrix (tests/TinyModels.cs:344-381). */
int wlo_matrix(uint64_t *rng, int t, int rows, int cols, float rms, uint8_t *data)
{
    int be, bb;
    if (!wlo_layout(t, &be, &bb)) return -1;
    int64_t n = (int64_t)rows * cols;
    int64_t nbytes = n / be * bb;
    if (t == WLO_F32 || t == WLO_F16 || t == WLO_BF16) {
        for (int64_t i = 0; i < n; i++) {
            float v = rms * rng_normal(rng);
            if (t == WLO_F32) memcpy(data + 4 * i, &v, 4);
            else {
                uint16_t h = t == WLO_F16 ? wlo_half_from_float(v) : (uint16_t)(float_to_bits(v) >> 16);
                data[2 * i] = (uint8_t)h; data[2 * i + 1] = (uint8_t)(h >> 8);
            }
        }
        return 0;
    }
    for (int64_t i = 0; i < nbytes; i++) data[i] = rng_byte(rng);
    int fields[2];
    int nf = scale_fields(t, fields);
    if (!nf) return -1;
    int64_t blocks = nbytes / bb;
    float tmp[256];
    uint16_t one = wlo_half_from_float(1.0f);
    for (int64_t b = 0; b < blocks; b++) {
        uint8_t *o = data + b * bb;
        for (int i = 0; i < nf; i++) { o[fields[i]] = (uint8_t)one; o[fields[i] + 1] = (uint8_t)(one >> 8); }
        double sum = 0;
        wlo_decode_row(t, o, be, tmp);
        for (int i = 0; i < be; i++) { float v2 = tmp[i] * tmp[i]; sum += v2; }
        double ms = sum / be;
        float scale = (float)(rms / sqrt(ms > 1e-12 ? ms : 1e-12));
        scale *= (float)(0.75 + 0.5 * rng_uniform(rng));
        uint16_t h = wlo_half_from_float(scale);
        for (int i = 0; i < nf; i++) { o[fields[i]] = (uint8_t)h; o[fields[i] + 1] = (uint8_t)(h >> 8); }
    }
    return 0;
}

/* ------------------------------------------- integer dots (src/FastMath.cs:35-214) */

/* C# Math.Round(v, MidpointRounding.AwayFromZero) and Math.Round(v) (to even), on doubles. */
static double round_away(double v) { return v < 0 ? -floor(-v + 0.5) : floor(v + 0.5); }
static double round_even(double v) { return nearbyint(v); }

void wlo_quantize_row(const float *x, int cols, int k, int8_t *q, float *d, int16_t *bsums)
{
    int bs = k ? 256 : 32, nb = cols / bs;
    for (int b = 0; b < nb; b++) {
        const float *xb = x + b * bs;
        int8_t *qb = q + b * bs;
        if (!k) {                                             /* src/FastMath.cs:54-61 */
            float amax = 0;
            for (int j = 0; j < 32; j++) { float ax = fabsf(xb[j]); if (ax > amax) amax = ax; }
            float dd = amax / 127.0f, id = dd != 0 ? 1.0f / dd : 0.0f;
            for (int j = 0; j < 32; j++) qb[j] = (int8_t)(int)round_away((double)(xb[j] * id));
            d[b] = wlo_half_round(dd);
        } else {                                              /* src/FastMath.cs:62-86 */
            float max = 0, amax = 0;
            for (int j = 0; j < 256; j++) { float ax = fabsf(xb[j]); if (ax > amax) { amax = ax; max = xb[j]; } }
            if (amax == 0) {
                d[b] = 0;
                memset(qb, 0, 256);
                for (int j = 0; j < 16; j++) bsums[b * 16 + j] = 0;
                continue;
            }
            float iscale = -127.0f / max;
            for (int j = 0; j < 256; j++) {
                int v = (int)round_even((double)(iscale * xb[j]));
                qb[j] = (int8_t)(v > 127 ? 127 : v);
            }
            for (int j = 0; j < 16; j++) {
                int s = 0;
                for (int l = 0; l < 16; l++) s += qb[j * 16 + l];
                bsums[b * 16 + j] = (int16_t)s;
            }
            d[b] = 1.0f / iscale;
        }
    }
}

int wlo_int_dot(int t, const uint8_t *b, const int8_t *q, const float *d, const int16_t *bsums, int n, float *out)
{
    switch (t) {
    case WLO_Q8_0: {                                          /* src/FastMath.cs:111-122 */
        float sum = 0;
        for (int i = 0; i < n / 32; i++, b += 34, q += 32) {
            const int8_t *w = (const int8_t *)(b + 2);
            int s0 = 0, s1 = 0;
            for (int j = 0; j < 32; j += 2) { s0 += w[j] * q[j]; s1 += w[j + 1] * q[j + 1]; }
            sum += H(b) * d[i] * (float)(s0 + s1);
        }
        *out = sum;
        return 0;
    }
    case WLO_Q4_0: {                                          /* src/FastMath.cs:123-134 */
        float sum = 0;
        for (int i = 0; i < n / 32; i++, b += 18, q += 32) {
            const uint8_t *w = b + 2;
            int s0 = 0, s1 = 0;
            for (int j = 0; j < 16; j++) { s0 += ((w[j] & 0xF) - 8) * q[j]; s1 += ((w[j] >> 4) - 8) * q[j + 16]; }
            sum += H(b) * d[i] * (float)(s0 + s1);
        }
        *out = sum;
        return 0;
    }
    case WLO_Q5_K: {                                          /* src/FastMath.cs:158-184 */
        float sum = 0;
        for (int i = 0; i < n / 256; i++, b += 176, q += 256, bsums += 16) {
            float dd = H(b), dmin = H(b + 2);
            const uint8_t *sc = b + 4, *qh = b + 16, *ql = b + 48;
            int sumi = 0, summ = 0, u1 = 1, u2 = 2;
            for (int j = 0; j < 4; j++, ql += 32, u1 <<= 2, u2 <<= 2) {
                int s1, m1, s2, m2;
                scale_min_k4(2 * j, sc, &s1, &m1);
                scale_min_k4(2 * j + 1, sc, &s2, &m2);
                const int8_t *qa = q + 64 * j, *qb = qa + 32;
                int a1 = 0, a2 = 0;
                for (int l = 0; l < 32; l++) {
                    a1 += ((ql[l] & 0xF) + ((qh[l] & u1) ? 16 : 0)) * qa[l];
                    a2 += ((ql[l] >> 4) + ((qh[l] & u2) ? 16 : 0)) * qb[l];
                }
                sumi += s1 * a1 + s2 * a2;
                summ += m1 * (bsums[4 * j] + bsums[4 * j + 1]) + m2 * (bsums[4 * j + 2] + bsums[4 * j + 3]);
            }
            sum += d[i] * (dd * (float)sumi - dmin * (float)summ);
        }
        *out = sum;
        return 0;
    }
    case WLO_Q4_K: {                                          /* src/FastMath.cs:135-157 */
        float sum = 0;
        for (int i = 0; i < n / 256; i++, b += 144, q += 256, bsums += 16) {
            float dd = H(b), dmin = H(b + 2);
            const uint8_t *sc = b + 4, *w = b + 16;
            int sumi = 0, summ = 0;
            for (int j = 0; j < 4; j++, w += 32) {
                int s1, m1, s2, m2;
                scale_min_k4(2 * j, sc, &s1, &m1);
                scale_min_k4(2 * j + 1, sc, &s2, &m2);
                const int8_t *qa = q + 64 * j, *qb = qa + 32;
                int a1 = 0, a2 = 0;
                for (int l = 0; l < 32; l++) { a1 += (w[l] & 0xF) * qa[l]; a2 += (w[l] >> 4) * qb[l]; }
                sumi += s1 * a1 + s2 * a2;
                summ += m1 * (bsums[4 * j] + bsums[4 * j + 1]) + m2 * (bsums[4 * j + 2] + bsums[4 * j + 3]);
            }
            sum += d[i] * (dd * (float)sumi - dmin * (float)summ);
        }
        *out = sum;
        return 0;
    }
    case WLO_Q6_K: {                                          /* src/FastMath.cs:185-211 */
        float sum = 0;
        int acc[8];
        for (int i = 0; i < n / 256; i++, b += 210, q += 256) {
            float dd = H(b + 208);
            const uint8_t *ql = b, *qh = b + 128;
            const int8_t *sc = (const int8_t *)(b + 192), *x = q;
            for (int k = 0; k < 2; k++, ql += 64, qh += 32, sc += 8, x += 128) {
                for (int g = 0; g < 8; g++) acc[g] = 0;
                for (int l = 0; l < 32; l++) {
                    int s = l >> 4;
                    acc[s] += (((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32) * x[l];
                    acc[s + 2] += (((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32) * x[l + 32];
                    acc[s + 4] += (((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32) * x[l + 64];
                    acc[s + 6] += (((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32) * x[l + 96];
                }
                int part = 0;
                for (int g = 0; g < 8; g++) part += sc[g] * acc[g];
                sum += d[i] * dd * (float)part;
            }
        }
        *out = sum;
        return 0;
    }
    }
    return -1;
}

int wlo_can_int_dot(int t)
{
    return t == WLO_Q8_0 || t == WLO_Q4_0 || t == WLO_Q4_K || t == WLO_Q5_K || t == WLO_Q6_K;
}

static int int_needs_k(int t) { return t == WLO_Q4_K || t == WLO_Q5_K || t == WLO_Q6_K; }

int wlo_int_fits(int t, int cols) { return cols > 0 && cols % (int_needs_k(t) ? 256 : 32) == 0; }

int wlo_int_matmul(int type, const uint8_t *data, int rows, int cols, int64_t row_bytes,
                   const float *x, int T, float *y, int threads)
{
    if (!wlo_can_int_dot(type) || !wlo_int_fits(type, cols)) return -1;
    int k = int_needs_k(type), nb = cols / (k ? 256 : 32), nth = n_threads(threads);
    int8_t *q = (int8_t *)malloc((size_t)T * cols);
    float *d = (float *)malloc(sizeof(float) * (size_t)T * nb);
    int16_t *bs = (int16_t *)calloc((size_t)T * (cols / 16), sizeof(int16_t));
    for (int t = 0; t < T; t++)
        wlo_quantize_row(x + (int64_t)t * cols, cols, k, q + (int64_t)t * cols, d + (int64_t)t * nb,
                         bs + (int64_t)t * (cols / 16));
    int rc = 0;
    #pragma omp parallel for schedule(dynamic, 32) num_threads(nth)
    for (int r = 0; r < rows; r++)
        for (int t = 0; t < T; t++)
            if (wlo_int_dot(type, data + (int64_t)r * row_bytes, q + (int64_t)t * cols, d + (int64_t)t * nb,
                            bs + (int64_t)t * (cols / 16), cols, y + (int64_t)t * rows + r))
                rc = -1;
    free(q); free(d); free(bs);
    return rc;
}
