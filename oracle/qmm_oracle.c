/*
 * CPU restatement of MLX affine dequantize / quantized_matmul / gather_qmm.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (as a cross-check of
 * oracle/oracle.py) and by bench.py's cpu_baseline leg (timed on the host
 * cores as the CPU baseline).  The mlxturbo_amd package never links it.
 *
 * Arithmetic (reference citations into /root/reference):
 *   unpack:   code j of word i is element i*(32/bits)+j at bit bits*j
 *             (mlxturbo/fast_qmm.py:96-106; kernels/_steel_flat.py:1251-1254)
 *   dequant:  T(float(s)*q + float(b)), T = bf16/fp16 rounded to nearest even
 *             (kernels/_steel_flat.py:1169-1256)
 *   matmul:   out[m,n] = sum_k x[m,k] * deq[n,k], accumulated in float32 over
 *             the T-rounded weights (bench/test_qmm_wide_shapes.py:35-42)
 *   gather:   out[p] = x[lhs[p]] . deq(w[rhs[p]])^T
 *             (kernels/moe_verify_gather.py:11-27)
 *
 * dtype codes: 0 = bfloat16, 1 = float16 (16-bit storage as uint16 bits).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bits_to_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_to_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static inline float bf16_to_f32(uint16_t h) { return bits_to_f32((uint32_t)h << 16); }

static inline uint16_t f32_to_bf16(float f) {
  uint32_t u = f32_to_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(((u >> 16) & 0x8000u) | 0x7fc0u);
  uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7fffu + lsb) >> 16);
}

static inline float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24, exact in float32 */
    float v = (float)man * 5.9604644775390625e-08f;
    return bits_to_f32(f32_to_bits(v) | sign);
  }
  if (exp == 31) return bits_to_f32(sign | 0x7f800000u | (man << 13));
  return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* float32 -> IEEE half, round to nearest even (integer formulation). */
static inline uint16_t f32_to_f16(float f) {
  uint32_t u = f32_to_bits(f);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);       /* NaN */
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);      /* >= 65520: inf */
  if (a < 0x38800000u) {                                        /* < 2^-14: subnormal */
    if (a < 0x33000000u) return (uint16_t)sign;                 /* < 2^-25: rounds to 0 */
    uint32_t e = a >> 23;
    uint32_t m = (a & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e;                                  /* 14..24 */
    uint32_t q = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t r = a - 0x38000000u;            /* rebias exponent 127 -> 15 */
  uint32_t lsb = (r >> 13) & 1u;
  r = (r + 0xfffu + lsb) >> 13;
  return (uint16_t)(sign | r);
}

static inline float load_t(const uint16_t* p, int dtype) {
  return dtype == 0 ? bf16_to_f32(*p) : f16_to_f32(*p);
}
static inline uint16_t store_t(float f, int dtype) {
  return dtype == 0 ? f32_to_bf16(f) : f32_to_f16(f);
}

int oracle_version(void) { return 1; }

uint16_t oracle_round_bf16(float f) { return f32_to_bf16(f); }
uint16_t oracle_round_f16(float f) { return f32_to_f16(f); }

/* Dequantize one row of K codes into float32 values already rounded to T. */
static void deq_row(const uint32_t* w, const uint16_t* s, const uint16_t* b, float* out,
                    int64_t K, int gs, int bits, int dtype) {
  const int per = 32 / bits;
  const uint32_t mask = (1u << bits) - 1u;
  for (int64_t k = 0; k < K; ++k) {
    uint32_t word = w[k / per];
    uint32_t q = (word >> (bits * (k % per))) & mask;
    float sc = load_t(&s[k / gs], dtype);
    float bi = load_t(&b[k / gs], dtype);
    float v = sc * (float)q + bi;   /* sc*q exact; one rounding */
    out[k] = load_t(&(uint16_t){store_t(v, dtype)}, dtype);
  }
}

int oracle_dequantize(const uint32_t* w, const uint16_t* s, const uint16_t* b, uint16_t* out,
                      int64_t N, int64_t K, int gs, int bits, int dtype) {
  if (bits != 2 && bits != 4 && bits != 8) return -1;
  if (K % gs || K % (32 / bits)) return -1;
  const int64_t Kw = K * bits / 32, G = K / gs;
#pragma omp parallel
  {
    float* row = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      deq_row(w + n * Kw, s + n * G, b + n * G, row, K, gs, bits, dtype);
      for (int64_t k = 0; k < K; ++k) out[n * K + k] = store_t(row[k], dtype);
    }
    free(row);
  }
  return 0;
}

/* out[M,N] float32 = x[M,K] . deq(W[N,K])^T, float32 accumulation. */
int oracle_qmm(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
               float* out, int64_t M, int64_t N, int64_t K, int gs, int bits, int dtype,
               int threads) {
  if (bits != 2 && bits != 4 && bits != 8) return -1;
  if (K % gs || K % (32 / bits)) return -1;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#else
  (void)threads;
#endif
  const int64_t Kw = K * bits / 32, G = K / gs;
  float* xf = (float*)malloc(sizeof(float) * (size_t)(M * K));
  for (int64_t i = 0; i < M * K; ++i) xf[i] = load_t(&x[i], dtype);
#pragma omp parallel
  {
    float* row = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
    for (int64_t n = 0; n < N; ++n) {
      deq_row(w + n * Kw, s + n * G, b + n * G, row, K, gs, bits, dtype);
      for (int64_t m = 0; m < M; ++m) {
        const float* xr = xf + m * K;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int64_t k = 0;
        for (; k + 8 <= K; k += 8)
          for (int j = 0; j < 8; ++j) acc[j] += xr[k + j] * row[k + j];
        for (; k < K; ++k) acc[0] += xr[k] * row[k];
        out[m * N + n] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) +
                         ((acc[4] + acc[5]) + (acc[6] + acc[7]));
      }
    }
    free(row);
  }
  free(xf);
  return 0;
}

/* Gather: x[B,M,K], w[E,N,Kw]; out[P,M,N] float32. */
int oracle_gather_qmm(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                      const int32_t* lhs, const int32_t* rhs, float* out, int64_t P, int64_t M,
                      int64_t N, int64_t K, int64_t E, int64_t B, int gs, int bits, int dtype,
                      int threads) {
  const int64_t Kw = K * bits / 32, G = K / gs;
  for (int64_t p = 0; p < P; ++p) {
    if (lhs[p] < 0 || lhs[p] >= B || rhs[p] < 0 || rhs[p] >= E) return -2;
    int r = oracle_qmm(x + (int64_t)lhs[p] * M * K, w + (int64_t)rhs[p] * N * Kw,
                       s + (int64_t)rhs[p] * N * G, b + (int64_t)rhs[p] * N * G,
                       out + p * M * N, M, N, K, gs, bits, dtype, threads);
    if (r) return r;
  }
  return 0;
}
