/* CPU oracle of COMP's decode path in plain C -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py load this library (through
 * oracle/coracle.py); the product (comp_amd) never does.  It is a second restatement of the reference arithmetic,
 * written independently of oracle/oracle.py (numpy), and the tests require the two to agree:
 *
 *   f16 <-> f32            IEEE binary16 from its definition (bit fields, round to nearest even, gradual underflow,
 *                          overflow to infinity); patches/0001-language-extra-kurn.patch:33-36 and the f16 d of :108
 *   oracle_quant_q8_0      ggml quantize_row_q8_0_ref as patch:104-114 and src/komp/kernels.py:22-33
 *   oracle_quant_q8_K      ggml quantize_row_q8_K_ref as patch:117-131, bsums as src/komp/host.py:50
 *   oracle_block_dots      exact integer block dots, src/komp/verify.py:94-100 (decode: patch:16-19, 39-63)
 *   oracle_reference_dot   the f64 block-order sum, src/komp/verify.py:103-120
 *   oracle_gemv_f32        the kernels' arithmetic: int32 block dot, then f32 scale and accumulate in block order,
 *                          src/komp/kernels.py:93 (q4_0: s * dw * dx) and :141 (tq2_0: dx * dw * s)
 *   oracle_quantize_q4_0   ggml quantize_row_q4_0_ref, the rule BASELINE's workloads quantize their f32 weights
 *                          with (restated as oracle.py quantize_q4_0_weights, which the tests compare it with); the
 *                          large workloads' weights come from here because numpy takes tens of seconds for them
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math: every float operation is one correctly rounded
 * IEEE operation, as the reference's quantizers require).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bits_f32(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}

static uint32_t f32_bits(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}

float oracle_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu;
  const uint32_t m = h & 0x3FFu;
  if (e == 0x1F) return bits_f32(sign | 0x7F800000u | (m << 13));
  if (e == 0) return (h & 0x8000u ? -1.0f : 1.0f) * ((float)m * 0x1p-24f); /* exact: m * 2^-24 */
  return bits_f32(sign | ((e - 15 + 127) << 23) | (m << 13));
}

uint16_t oracle_f32_to_f16(float f) {
  const uint32_t x = f32_bits(f);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t a = x & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7E00u;              /* NaN */
  if (a >= 0x477FF000u) return sign | 0x7C00u;             /* >= 65520 rounds to infinity */
  if (a >= 0x38800000u) {                                  /* normal binary16 */
    uint32_t r = (((a >> 23) - 112u) << 10) | ((a >> 13) & 0x3FFu);
    const uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r += 1; /* a carry into the exponent is still correct */
    return sign | (uint16_t)r;
  }
  /* subnormal binary16: round(|f| / 2^-24) to nearest even; |f| = M * 2^(E - 150) */
  const uint32_t E = a >> 23;
  const uint32_t M = E ? ((a & 0x7FFFFFu) | 0x800000u) : (a & 0x7FFFFFu);
  const uint32_t shift = 126u - (E ? E : 1u);
  if (shift >= 25) return sign;
  uint32_t q = M >> shift;
  const uint32_t rem = M & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (q & 1u))) q += 1;
  return sign | (uint16_t)q;
}

/* x [nblocks * 32] -> q [nblocks * 32], d [nblocks] = f32(f16(d)) */
void oracle_quant_q8_0(const float* x, int8_t* q, float* d, int64_t nblocks) {
  for (int64_t b = 0; b < nblocks; ++b) {
    const float* xb = x + b * 32;
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(xb[i]));
    const float dd = amax / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    for (int i = 0; i < 32; ++i) q[b * 32 + i] = (int8_t)roundf(xb[i] * id);
    d[b] = oracle_f16_to_f32(oracle_f32_to_f16(dd));
  }
}

/* x [nblocks * 256] -> q [nblocks * 256], d [nblocks], bsums [nblocks * 16] (NULL allowed) */
void oracle_quant_q8_K(const float* x, int8_t* q, float* d, int16_t* bsums, int64_t nblocks) {
  for (int64_t b = 0; b < nblocks; ++b) {
    const float* xb = x + b * 256;
    float amax = 0.0f, mx = 0.0f;
    for (int i = 0; i < 256; ++i) {
      const float ax = fabsf(xb[i]);
      if (ax > amax) { /* strict: the first index wins ties */
        amax = ax;
        mx = xb[i];
      }
    }
    if (amax == 0.0f) {
      memset(q + b * 256, 0, 256);
      d[b] = 0.0f;
    } else {
      const float iscale = -127.0f / mx;
      for (int i = 0; i < 256; ++i) {
        const float v = nearbyintf(iscale * xb[i]); /* round to nearest even in the default mode */
        q[b * 256 + i] = (int8_t)(v > 127.0f ? 127.0f : v);
      }
      d[b] = 1.0f / iscale;
    }
    if (bsums) {
      for (int g = 0; g < 16; ++g) {
        int s = 0;
        for (int i = 0; i < 16; ++i) s += q[b * 256 + g * 16 + i];
        bsums[b * 16 + g] = (int16_t)s;
      }
    }
  }
}

/* value v of a block from its quant bytes: q4_0 byte v % 16, nibble v / 16; tq2_0 byte (v/128)*32 + v%32, crumb
 * (v%128)/32 */
static int weight_value(int fmt, const uint8_t* qs, int v) {
  if (fmt == 0) return ((qs[v & 15] >> (4 * (v >> 4))) & 15) - 8;
  return ((qs[(v >> 7) * 32 + (v & 31)] >> (2 * ((v & 127) >> 5))) & 3) - 1;
}

/* exact block dots S [M][N][K/blk] (int64) of split planes WQ [N][SW] with XQ [M][K] */
void oracle_block_dots(int fmt, const uint8_t* wq, const int8_t* xq, int64_t* s, int64_t M, int64_t N, int64_t K,
                       int64_t SW) {
  const int blk = fmt == 0 ? 32 : 256, bb = fmt == 0 ? 16 : 64;
  const int64_t nb = K / blk;
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t* qs = wq + n * SW + b * bb;
      int vals[256];
      for (int v = 0; v < blk; ++v) vals[v] = weight_value(fmt, qs, v);
      for (int64_t m = 0; m < M; ++m) {
        const int8_t* x = xq + m * K + b * blk;
        int64_t acc = 0;
        for (int v = 0; v < blk; ++v) acc += (int64_t)vals[v] * x[v];
        s[(m * N + n) * nb + b] = acc;
      }
    }
  }
}

/* f64 reference outputs R [M][N] from the block dots, summed block by block (src/komp/verify.py:103-120) */
void oracle_reference_dot(int fmt, const int16_t* ws, const float* xd, const int64_t* s, double* r, int64_t M,
                          int64_t N, int64_t nb) {
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) {
      double total = 0.0;
      for (int64_t b = 0; b < nb; ++b) {
        const double dw = (double)oracle_f16_to_f32((uint16_t)ws[n * nb + b]);
        const double dx = (double)xd[m * nb + b];
        const double sv = (double)s[(m * N + n) * nb + b];
        total += fmt == 0 ? (dw * dx) * sv : (dx * dw) * sv;
      }
      r[m * N + n] = total;
    }
  }
}

/* the kernels' arithmetic on the CPU: Y [M][N] f32 with int32 block dots and f32 scaling, block order */
void oracle_gemv_f32(int fmt, const uint8_t* wq, const int16_t* ws, const int8_t* xq, const float* xd, float* y,
                     int64_t M, int64_t N, int64_t K, int64_t SW) {
  const int blk = fmt == 0 ? 32 : 256, bb = fmt == 0 ? 16 : 64;
  const int64_t nb = K / blk;
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t m = 0; m < M; ++m) {
      float acc = 0.0f;
      for (int64_t b = 0; b < nb; ++b) {
        const uint8_t* qs = wq + n * SW + b * bb;
        const int8_t* x = xq + m * K + b * blk;
        int32_t sdot = 0;
        if (fmt == 0) {
          for (int i = 0; i < 16; ++i) sdot += ((qs[i] & 15) - 8) * x[i] + ((qs[i] >> 4) - 8) * x[i + 16];
        } else {
          for (int h = 0; h < 2; ++h)
            for (int j = 0; j < 4; ++j)
              for (int i = 0; i < 32; ++i) sdot += (((qs[h * 32 + i] >> (2 * j)) & 3) - 1) * x[h * 128 + j * 32 + i];
        }
        const float dw = oracle_f16_to_f32((uint16_t)ws[n * nb + b]);
        const float dx = xd[m * nb + b];
        acc += fmt == 0 ? ((float)sdot * dw) * dx : (dx * dw) * (float)sdot;
      }
      y[m * N + n] = acc;
    }
  }
}

/* f32 weights w [nblocks * 32] -> ggml q4_0 blocks out [nblocks * 18] (ggml quantize_row_q4_0_ref): max = the signed
 * value of the first largest |x|; d = max / -8; id = d != 0 ? 1 / d : 0; q = min(15, trunc(x * id + 8.5)); bytes
 * f16(d), then q[j] | q[j + 16] << 4 */
void oracle_quantize_q4_0(const float* w, uint8_t* out, int64_t nblocks) {
  for (int64_t b = 0; b < nblocks; ++b) {
    const float* x = w + b * 32;
    float amax = 0.0f, mx = 0.0f;
    for (int i = 0; i < 32; ++i) {
      if (fabsf(x[i]) > amax) {
        amax = fabsf(x[i]);
        mx = x[i];
      }
    }
    const float d = mx / -8.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t q[32];
    for (int i = 0; i < 32; ++i) {
      const float v = x[i] * id + 8.5f; /* two roundings: -ffp-contract=off keeps them apart */
      float t = truncf(v);
      if (t > 15.0f) t = 15.0f;
      q[i] = (uint8_t)(t < 0.0f ? 0 : t);
    }
    uint8_t* o = out + b * 18;
    const uint16_t h = oracle_f32_to_f16(d);
    o[0] = (uint8_t)(h & 0xFF);
    o[1] = (uint8_t)(h >> 8);
    for (int j = 0; j < 16; ++j) o[2 + j] = (uint8_t)(q[j] | (q[j + 16] << 4));
  }
}
