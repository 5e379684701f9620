/*
 * fp64emu_oracle.c -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.
 *
 * CPU restatement of the reference RARE emulated-FP64 GEMM pipeline
 * (CharlesCNorton/fp64-emu, fp64_emu_cuda/fp64_emu.cu and
 * torch-ext/fp64_emu/__init__.py), used only as the checker of the HIP path:
 * by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 * Nothing on the product path may link or call it.
 *
 * Every stage follows the reference's own arithmetic, including the parts
 * where the HIP build chose a different but equivalent method (three 18-bit
 * limbs + 31-bit Barrett residues here, exact fp64 nearest-quotient
 * reductions on the GPU), so bit parity between the two is a real check.
 * Floating point: compile with -ffp-contract=off; the reference's
 * `ss += v * v` and `acc * m + a` are contracted to FMA by nvcc (default
 * --fmad=true), so those are written as explicit fma() here.
 *
 * Pinning (tests/test_oracle_*.py): tables against modular-inverse and
 * CRT-round-trip invariants; rne/extraction against exact rational rounding
 * (Python Fraction) on special cases; Barrett against % exhaustively;
 * GEMM against numpy int64; reconstruction against big-integer CRT and
 * correctly rounded Fraction->float; end to end against exact integer
 * products (the reference's tests/test_fp64_emu.py KATs re-expressed) and
 * the double-double oracle's correct-bit floor.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_MAXP 20
#define OR_GROUPS ((OR_MAXP + 3) / 4)
#define OR_THREADS 256

typedef __int128 i128;

/* ---- tables: fp64_emu_cuda/fp64_emu.cu:958-993 and :1052 ---------------- */

/* Brute-force inverse, fp64_emu.cu:959-963. */
static int or_modinv(int a, int m) {
  a %= m;
  if (a < 0) a += m;
  for (int x = 1; x < m; x++)
    if ((long long)a * x % m == 1) return x;
  return 0;
}

/* minv[t] = (M_t mod p_t)^-1; mppack[t*5+g] = balanced int8 (M_u mod p_t),
 * u = 4g..4g+3, zero for u >= t; m64 = group products of 7; log2M = float
 * sum of (float)log2(p) (fp64_emu.cu:1052). */
void or_tables(const int32_t* primes, int P, int32_t* minv, int32_t* mppack, int64_t* m64,
               float* log2M) {
  memset(mppack, 0, sizeof(int32_t) * (size_t)P * OR_GROUPS);
  for (int g = 0; g < 2; g++) {
    long long prod = 1;
    for (int t = g * 7; t < (g * 7 + 7 < P ? g * 7 + 7 : P); t++) prod *= primes[t];
    m64[g] = prod;
  }
  for (int t = 0; t < P; t++) {
    const long long pt = primes[t];
    long long run = 1 % pt;
    for (int u = 0; u < P; u++) {
      if (u == t) minv[t] = or_modinv((int)run, (int)pt);
      if (u < t) {
        int bal = (int)run;
        if (bal > ((int)pt - 1) / 2) bal -= (int)pt;
        mppack[(size_t)t * OR_GROUPS + (u >> 2)] |= ((int)(unsigned char)(signed char)bal)
                                                    << ((u & 3) * 8);
      }
      run = run * (primes[u] % pt) % pt;
    }
  }
  float l = 0.0f;
  for (int t = 0; t < P; t++) l += (float)log2((double)primes[t]);
  *log2M = l;
}

/* ---- sizing: fp64_emu_cuda/fp64_emu.cu:107-231 --------------------------- */

static void or_row_finish(double m, double s2, int bits, int16_t* sft, float* lg) {
  const int e = (m > 0.0 && isfinite(m)) ? ilogb(m) : 0;
  const int sh = (bits - 1) - e;
  const float l = (s2 > 0.0 && isfinite(s2)) ? (float)(0.5 * log2(s2) + sh)
                                             : (m > 0.0 ? INFINITY : -INFINITY);
  *sft = (int16_t)sh;
  *lg = l;
}

/* row_shift_kernel (fp64_emu.cu:111-146) with its summation order: 256
 * thread-strided FMA partial sums, then the 128..1 tree. */
void or_size_rows(const double* X, int64_t rows, int64_t cols, int bits, int16_t* sft, float* lg) {
  double mx[OR_THREADS], ss[OR_THREADS];
  for (int64_t r = 0; r < rows; r++) {
    const double* x = X + r * cols;
    for (int t = 0; t < OR_THREADS; t++) {
      double m = 0.0, s = 0.0;
      for (int64_t c = t; c < cols; c += OR_THREADS) {
        const double v = x[c];
        m = fmax(m, fabs(v));
        s = fma(v, v, s);
      }
      mx[t] = m;
      ss[t] = s;
    }
    for (int s = OR_THREADS / 2; s > 0; s >>= 1)
      for (int t = 0; t < s; t++) {
        mx[t] = fmax(mx[t], mx[t + s]);
        ss[t] = ss[t] + ss[t + s];
      }
    or_row_finish(mx[0], ss[0], bits, &sft[r], &lg[r]);
  }
}

/* Slab split of fp64_emu.cu:1159-1162. */
static void or_slabs(int64_t NF, int64_t K, int64_t* kslab, int* nslab) {
  if (K <= 0 || NF <= 0) { *kslab = 0; *nslab = 0; return; }
  int64_t nsl0 = 131072 / NF;
  if (nsl0 < 1) nsl0 = 1;
  if (nsl0 > 128) nsl0 = 128;
  *kslab = (K + nsl0 - 1) / nsl0;
  *nslab = (int)((K + *kslab - 1) / *kslab);
}

/* col_shift_partial_kernel + col_shift_finalize_kernel (fp64_emu.cu:148-189)
 * for X = [batch, K, N]: per-column slab FMA sums in k order, slabs added in
 * order. */
void or_size_cols(const double* X, int64_t batch, int64_t K, int64_t N, int bits, int16_t* sft,
                  float* lg) {
  const int64_t NF = batch * N;
  int64_t kslab;
  int nslab;
  or_slabs(NF, K, &kslab, &nslab);
  for (int64_t j = 0; j < NF; j++) {
    const int64_t b = j / N, n = j - b * N;
    const double* base = X + b * K * N + n;
    double m = 0.0, s = 0.0;
    for (int sl = 0; sl < nslab; sl++) {
      const int64_t k0 = (int64_t)sl * kslab;
      const int64_t k1 = (k0 + kslab < K) ? k0 + kslab : K;
      double pm = 0.0, ps = 0.0;
      for (int64_t k = k0; k < k1; k++) {
        const double v = base[k * N];
        pm = fmax(pm, fabs(v));
        ps = fma(v, v, ps);
      }
      m = fmax(m, pm);
      s = s + ps;
    }
    or_row_finish(m, s, bits, &sft[j], &lg[j]);
  }
}

/* pick_bits_kernel (fp64_emu.cu:193-231); returns bits_eff and folds the
 * gain into the shifts. */
int or_pick_bits(const float* lgA, int64_t m, const float* lgB, int64_t n, float log2M, int bits,
                 int16_t* sftA, int16_t* sftB) {
  float a = -INFINITY, b = -INFINITY;
  for (int64_t i = 0; i < m; i++) a = fmaxf(a, lgA[i]);
  for (int64_t j = 0; j < n; j++) b = fmaxf(b, lgB[j]);
  const float need = a + b + 0.5f;
  int g = 0;
  if (isfinite(need)) g = (int)floorf((log2M - 1.0f - need) * 0.5f);
  if (g > 53 - bits) g = 53 - bits;
  int be = bits + g;
  if (be < 16) be = 16;
  g = be - bits;
  if (g) {
    for (int64_t i = 0; i < m; i++) sftA[i] = (int16_t)(sftA[i] + g);
    for (int64_t j = 0; j < n; j++) sftB[j] = (int16_t)(sftB[j] + g);
  }
  return be;
}

/* ---- extraction: fp64_emu_cuda/fp64_emu.cu:238-397 ----------------------- */

/* rne_shr, fp64_emu.cu:292-299. */
uint64_t or_rne_shr(uint64_t mag, int s) {
  if (s <= 0) return (-s < 64) ? (mag << (-s)) : 0ULL;
  if (s > 63) return 0ULL;
  const uint64_t keep = mag >> s;
  const uint64_t rem = mag & ((1ULL << s) - 1ULL);
  const uint64_t half = 1ULL << (s - 1);
  return keep + ((rem > half || (rem == half && (keep & 1ULL))) ? 1ULL : 0ULL);
}

/* split, fp64_emu.cu:300-321: returns td + 2^bits, writes hi7/q7 when
 * do_corr. */
uint64_t or_split(double x, int srow, int bits, int do_corr, int8_t* h, int8_t* q) {
  uint64_t xb;
  memcpy(&xb, &x, 8);
  const int neg = (int64_t)xb < 0;
  const int e = (int)((xb >> 52) & 0x7FF);
  const uint64_t m = xb & 0xFFFFFFFFFFFFFULL;
  const uint64_t mag = e ? ((1ULL << 52) | m) : m;
  const int t = (e ? e : 1) - 1075 + srow + 52;
  const uint64_t Tu = or_rne_shr(mag, 52 - t);
  const long long td = neg ? -(long long)Tu : (long long)Tu;
  if (do_corr) {
    const long long r8 = (long long)or_rne_shr(mag, 44 - t) - (long long)(Tu << 8);
    const long long h8 = (long long)or_rne_shr(Tu, bits - 7);
    const long long hs = neg ? -h8 : h8;
    const long long qs = neg ? -r8 : r8;
    *h = (int8_t)(hs > 127 ? 127 : (hs < -127 ? -127 : hs));
    *q = (int8_t)(qs > 127 ? 127 : (qs < -127 ? -127 : qs));
  }
  return (uint64_t)(td + ((long long)1 << bits));
}

/* residue, fp64_emu.cu:260-287: three 18-bit limbs, bias-cancelling
 * constant, 31-bit Barrett with one conditional subtract, balance. */
int8_t or_residue(uint64_t uu, int p, int bits) {
  const uint32_t up = (uint32_t)p;
  const uint32_t mu32 = (uint32_t)((1u << 31) / up);
  const uint32_t c36 = (uint32_t)(((uint64_t)1 << 36) % up);
  const uint32_t c18 = (uint32_t)(((uint64_t)1 << 18) % up);
  const uint32_t cb = up - (uint32_t)(((uint64_t)1 << bits) % up);
  const uint32_t a = (uint32_t)(uu >> 36), b = (uint32_t)((uu >> 18) & 0x3FFFFu),
                 c = (uint32_t)(uu & 0x3FFFFu);
  const uint32_t v = a * c36 + b * c18 + c + cb;
  const uint32_t qq = (uint32_t)(((uint64_t)v * mu32) >> 31);
  uint32_t r = v - qq * up;
  if (r >= up) r -= up;
  int rb = (int)r;
  if (rb > ((int)up - 1) / 2) rb -= (int)up;
  return (int8_t)rb;
}

/* One operand to logical planes.  kn = 0: X is [batch, R, K] with one shift
 * per row; kn = 1: X is [batch, K, R] (the mm_nt Bt layout) with one shift
 * per column.  res: [batch][P][R][K]; hi, q: [batch][R][K] (when do_corr). */
void or_extract_operand(const double* X, int64_t batch, int64_t R, int64_t K, int kn,
                        const int16_t* sft, int bits_eff, const int32_t* primes, int P,
                        int do_corr, int8_t* res, int8_t* hi, int8_t* q) {
  /* Rows are independent (each element's split and residues depend on it
   * and its row shift alone): OpenMP over rows. */
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t br = 0; br < batch * R; br++) {
      const int64_t b = br / R, r = br % R;
      const int s = sft[b * R + r];
      for (int64_t k = 0; k < K; k++) {
        const double x = kn ? X[(b * K + k) * R + r] : X[(b * R + r) * K + k];
        int8_t h = 0, qq = 0;
        const uint64_t uu = or_split(x, s, bits_eff, do_corr, &h, &qq);
        for (int t = 0; t < P; t++)
          res[((b * P + t) * R + r) * K + k] = or_residue(uu, primes[t], bits_eff);
        if (do_corr) {
          hi[(b * R + r) * K + k] = h;
          q[(b * R + r) * K + k] = qq;
        }
      }
    }
}

/* ---- modular GEMM: fp64_emu_cuda/fp64_emu.cu:494-657 --------------------- */

/* bal8, fp64_emu.cu:613-620: 31-bit Barrett of an int32 to balanced int8. */
int8_t or_bal8(int32_t v, int p) {
  const uint32_t up = (uint32_t)p;
  const uint32_t mu31 = (1u << 31) / up;
  const uint32_t off = (0x80000000u / up) * up;
  const uint32_t xu = (uint32_t)v + off;
  uint32_t r = xu - (uint32_t)(((uint64_t)xu * mu31) >> 31) * up;
  while (r >= up) r -= up;
  int rb = (int)r;
  if (rb > p / 2) rb -= p;
  return (int8_t)rb;
}

/* C = A B^T exact in int32 (A [M,K], B [N,K] int8).  p > 0: out8 = bal8(C);
 * p == 0: out32 = C.  Returns 1 if any |C| reached 2^31 (outside the
 * reference's single-launch bound), else 0. */
int or_modgemm(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K, int p,
               int8_t* out8, int32_t* out32, int nthreads) {
  int overflow = 0;
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for num_threads(nthreads) reduction(| : overflow) schedule(static)
#endif
  for (int64_t i = 0; i < M; i++) {
    const int8_t* a = A + i * K;
    for (int64_t j = 0; j < N; j++) {
      const int8_t* bb = B + j * K;
      int64_t acc = 0;
      /* int32 partial sums over 65536-deep chunks stay exact (65536 * 128^2 = 2^30). */
      for (int64_t k0 = 0; k0 < K; k0 += 65536) {
        const int64_t k1 = (k0 + 65536 < K) ? k0 + 65536 : K;
        int32_t part = 0;
        for (int64_t k = k0; k < k1; k++) part += (int32_t)a[k] * (int32_t)bb[k];
        acc += part;
      }
      if (acc >= 2147483648LL || acc < -2147483648LL) overflow = 1;
      if (p > 0) out8[i * N + j] = or_bal8((int32_t)acc, p);
      else out32[i * N + j] = (int32_t)acc;
    }
  }
  (void)nthreads;
  return overflow;
}

/* ---- reconstruction: fp64_emu_cuda/fp64_emu.cu:39-105, 849-952 ---------- */

/* barrett_bal32, fp64_emu.cu:42-51. */
int or_barrett_bal32(int y, int p, uint32_t mu32, uint32_t bias) {
  const uint32_t xu = (uint32_t)((long long)y + (long long)bias);
  const uint32_t qq = (uint32_t)(((uint64_t)xu * mu32) >> 31);
  uint32_t r = xu - qq * (uint32_t)p;
  while (r >= (uint32_t)p) r -= (uint32_t)p;
  int rb = (int)r;
  if (rb > (p - 1) / 2) rb -= p;
  return rb;
}

/* s128_to_double, fp64_emu.cu:94-105: top 64 bits plus sticky, one RN
 * conversion, exact scale. */
double or_i128_to_double(i128 v) {
  const int neg = v < 0;
  unsigned __int128 u = neg ? (unsigned __int128)(-v) : (unsigned __int128)v;
  const uint64_t hi = (uint64_t)(u >> 64), lo = (uint64_t)u;
  if (hi == 0) {
    const double m = (double)lo;
    return neg ? -m : m;
  }
  const int sh = 64 - __builtin_clzll(hi);
  uint64_t top, tail;
  if (sh == 64) { top = hi; tail = lo; }
  else { top = (hi << (64 - sh)) | (lo >> sh); tail = lo & ((1ULL << sh) - 1ULL); }
  const double m = ldexp((double)(top | (tail != 0ULL ? 1ULL : 0ULL)), sh);
  return neg ? -m : m;
}

/* Balanced Garner digits of one element (fp64_emu.cu:899-920, dp4a as a
 * plain int8 dot product). */
static void or_digits(const int* r, int P, const int32_t* primes, const int32_t* minv,
                      const int32_t* mppack, int* d) {
  for (int t = 0; t < P; t++) {
    const int p = primes[t];
    const uint32_t mu32 = (uint32_t)((1u << 31) / (unsigned)p);
    int acc = 0;
    for (int u = 0; u < t; u++) {
      const int f = (int)(signed char)(uint8_t)((uint32_t)mppack[t * OR_GROUPS + (u >> 2)] >> ((u & 3) * 8));
      acc += d[u] * f;
    }
    const int y = (r[t] - acc) * minv[t];
    d[t] = or_barrett_bal32(y, p, mu32, (uint32_t)p << 21);
  }
}

/* Per-element value (fp64_emu.cu:921-949) before the final ldexp. */
static double or_combine(const int* d, int P, const int32_t* primes, const int64_t* m64,
                         long long corr, int cshift, int exact) {
  const int ng = (P + 6) / 7;
  long long a0 = 0, a1 = 0, a2 = 0;
  for (int t = P - 1; t >= 0; t--) {
    if (t >= 14) a2 = a2 * primes[t] + d[t];
    else if (t >= 7) a1 = a1 * primes[t] + d[t];
    else a0 = a0 * primes[t] + d[t];
  }
  if (exact) {
    i128 acc = (i128)(ng == 3 ? a2 : (ng == 2 ? a1 : a0));
    if (ng == 3) acc = acc * (i128)m64[1] + a1;
    if (ng >= 2) acc = acc * (i128)m64[0] + a0;
    acc += (i128)corr * ((i128)1 << cshift);
    return or_i128_to_double(acc);
  }
  double acc = (double)(ng == 3 ? a2 : (ng == 2 ? a1 : a0));
  if (ng == 3) acc = fma(acc, (double)m64[1], (double)a1);
  if (ng >= 2) acc = fma(acc, (double)m64[0], (double)a0);
  acc += ldexp((double)corr, cshift);
  return acc;
}

/* reconstruct_kernel (fp64_emu.cu:854-952) for one batch member: res
 * [P][M*N] int8; the correction as int32 planes c1/c2 or int64 planes
 * d1/d2 (the K-segmented path's accumulators), NULL = none. */
static void or_reconstruct_any(const int8_t* res, const int32_t* c1, const int32_t* c2,
                               const int64_t* d1, const int64_t* d2, int64_t M, int64_t N,
                               const int32_t* primes, int P, int bits_eff, const int16_t* sftA,
                               const int16_t* sftB, int exact, double* out) {
  int32_t minv[OR_MAXP], mppack[OR_MAXP * OR_GROUPS];
  int64_t m64[2];
  float l2;
  or_tables(primes, P, minv, mppack, m64, &l2);
  const int cshift = bits_eff - 15;
  const int64_t total = M * N;
  /* Elements are independent: OpenMP over rows. */
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t i = 0; i < M; i++)
    for (int64_t j = 0; j < N; j++) {
      const int64_t idx = i * N + j;
      int r[OR_MAXP], d[OR_MAXP];
      for (int t = 0; t < P; t++) r[t] = res[(int64_t)t * total + idx];
      or_digits(r, P, primes, minv, mppack, d);
      const long long corr = (c1 ? (long long)c1[idx] : 0LL) + (c2 ? (long long)c2[idx] : 0LL) +
                             (d1 ? (long long)d1[idx] : 0LL) + (d2 ? (long long)d2[idx] : 0LL);
      const double v = or_combine(d, P, primes, m64, corr, cshift, exact);
      out[idx] = ldexp(v, -(int)sftA[i] - (int)sftB[j]);
    }
}

void or_reconstruct(const int8_t* res, const int32_t* c1, const int32_t* c2, int64_t M, int64_t N,
                    const int32_t* primes, int P, int bits_eff, const int16_t* sftA,
                    const int16_t* sftB, int exact, double* out) {
  or_reconstruct_any(res, c1, c2, NULL, NULL, M, N, primes, P, bits_eff, sftA, sftB, exact, out);
}

void or_reconstruct64(const int8_t* res, const int64_t* d1, const int64_t* d2, int64_t M,
                      int64_t N, const int32_t* primes, int P, int bits_eff, const int16_t* sftA,
                      const int16_t* sftB, int exact, double* out) {
  or_reconstruct_any(res, NULL, NULL, d1, d2, M, N, primes, P, bits_eff, sftA, sftB, exact, out);
}

/* Fold of the K-segmented residue sums (reduce_planes_kernel with kdepth =
 * 1, fp64_emu.cu:833-847, 1570-1574): barrett_bal32 with the bias
 * p * ceil((p/2)^2 / p), exact while |acc| <= that bias (at least 86 segments
 * of balanced residues for every modulus). */
int or_fold_residue(int32_t acc, int p) {
  const uint64_t half = (uint64_t)(p / 2), maxabs = half * half;
  const uint32_t bias = (uint32_t)((uint64_t)p * ((maxabs + (uint64_t)p - 1) / (uint64_t)p));
  return or_barrett_bal32(acc, p, (uint32_t)((1u << 31) / (unsigned)p), bias);
}

/* One 65536-column segment of a row-major [R, K] int8 plane, made contiguous. */
static void or_segment(const int8_t* src, int64_t R, int64_t K, int64_t k0, int64_t kc, int8_t* dst) {
  for (int64_t r = 0; r < R; r++) memcpy(dst + r * kc, src + r * K + k0, (size_t)kc);
}

/* run_crt_bigk (fp64_emu.cu:1479-1579) for one batch member with B [N, K]:
 * 65536-column segments; per segment the modular GEMMs give balanced int8
 * residues, summed in int32, and the two int32 correction products, summed
 * in int64; one fold to int8 and one reconstruction close the sum.
 * Returns 0, or -1 on allocation failure. */
static int or_mm_segmented(const int8_t* resA, const int8_t* hA, const int8_t* qA,
                           const int8_t* resB, const int8_t* hB, const int8_t* qB, int64_t M,
                           int64_t N, int64_t K, const int32_t* primes, int P, int use_corr,
                           int nthreads, int be, const int16_t* sftA, const int16_t* sftB,
                           int exact, double* out) {
  const int64_t Kc = 65536;
  const size_t pa = (size_t)M * K, pb = (size_t)N * K, po = (size_t)M * N;
  int32_t* acc = (int32_t*)calloc(po * P + 1, sizeof(int32_t));
  int64_t* d1 = (int64_t*)calloc(po + 1, sizeof(int64_t));
  int64_t* d2 = (int64_t*)calloc(po + 1, sizeof(int64_t));
  int8_t* sa = (int8_t*)malloc((size_t)M * Kc + 1);
  int8_t* sb = (int8_t*)malloc((size_t)N * Kc + 1);
  int8_t* sa2 = (int8_t*)malloc((size_t)M * Kc + 1);
  int8_t* sb2 = (int8_t*)malloc((size_t)N * Kc + 1);
  int8_t* r8 = (int8_t*)malloc(po + 1);
  int32_t* c32 = (int32_t*)malloc(sizeof(int32_t) * po + 4);
  int8_t* res8 = (int8_t*)malloc(po * P + 1);
  int st = 0;
  if (!acc || !d1 || !d2 || !sa || !sb || !sa2 || !sb2 || !r8 || !c32 || !res8) { st = -1; goto done; }
  for (int64_t k0 = 0; k0 < K; k0 += Kc) {
    const int64_t kc = K - k0 < Kc ? K - k0 : Kc;
    for (int t = 0; t < P; t++) {
      or_segment(resA + t * pa, M, K, k0, kc, sa);
      or_segment(resB + t * pb, N, K, k0, kc, sb);
      or_modgemm(sa, sb, M, N, kc, primes[t], r8, NULL, nthreads);
      for (size_t i = 0; i < po; i++) acc[t * po + i] += r8[i];
    }
    if (use_corr) {
      or_segment(hA, M, K, k0, kc, sa); or_segment(qB, N, K, k0, kc, sb);
      or_segment(qA, M, K, k0, kc, sa2); or_segment(hB, N, K, k0, kc, sb2);
      or_modgemm(sa, sb, M, N, kc, 0, NULL, c32, nthreads);      /* hi7_A q7_B^T */
      for (size_t i = 0; i < po; i++) d1[i] += c32[i];
      or_modgemm(sa2, sb2, M, N, kc, 0, NULL, c32, nthreads);    /* q7_A hi7_B^T */
      for (size_t i = 0; i < po; i++) d2[i] += c32[i];
    }
  }
  for (int t = 0; t < P; t++)
    for (size_t i = 0; i < po; i++) res8[t * po + i] = (int8_t)or_fold_residue(acc[t * po + i], primes[t]);
  or_reconstruct64(res8, use_corr ? d1 : NULL, use_corr ? d2 : NULL, M, N, primes, P, be, sftA,
                   sftB, exact, out);
done:
  free(acc); free(d1); free(d2); free(sa); free(sb); free(sa2); free(sb2); free(r8); free(c32);
  free(res8);
  return st;
}

/* ---- whole pipeline: fp64_emu_cuda/fp64_emu.cu:1127-1407 (fused path),
 * and 1479-1579 (K-segmented) for K > 131071 with B as [N, K] ---
 * A [batch, M, K]; B [batch, N, K] (b_kn = 0, mm/bmm) or [batch, K, N]
 * (b_kn = 1, mm_nt/bmm_nt).  Optional outputs (NULL to skip): the sizing
 * results after the width pick.  Returns 0, or -1 on allocation failure. */
int or_mm(double* out, const double* A, const double* B, int64_t batch, int64_t M, int64_t N,
          int64_t K, int b_kn, const int32_t* primes, int P, int exact, int bits, int use_corr,
          int nthreads, int16_t* sftA_out, int16_t* sftB_out, float* lgA_out, float* lgB_out,
          int* bits_eff_out) {
  const int64_t MF = batch * M, NF = batch * N;
  int32_t minv[OR_MAXP], mppack[OR_MAXP * OR_GROUPS];
  int64_t m64[2];
  float log2M;
  or_tables(primes, P, minv, mppack, m64, &log2M);
  int16_t* sftA = (int16_t*)malloc(sizeof(int16_t) * (MF > 0 ? MF : 1));
  int16_t* sftB = (int16_t*)malloc(sizeof(int16_t) * (NF > 0 ? NF : 1));
  float* lgA = (float*)malloc(sizeof(float) * (MF > 0 ? MF : 1));
  float* lgB = (float*)malloc(sizeof(float) * (NF > 0 ? NF : 1));
  const size_t pa = (size_t)M * K, pb = (size_t)N * K, po = (size_t)M * N;
  int8_t* resA = (int8_t*)malloc(pa * P + 1);
  int8_t* resB = (int8_t*)malloc(pb * P + 1);
  int8_t *hA = NULL, *qA = NULL, *hB = NULL, *qB = NULL;
  if (use_corr) {
    hA = (int8_t*)malloc(pa + 1); qA = (int8_t*)malloc(pa + 1);
    hB = (int8_t*)malloc(pb + 1); qB = (int8_t*)malloc(pb + 1);
  }
  int8_t* res8 = (int8_t*)malloc(po * P + 1);
  int32_t* c1 = (int32_t*)malloc(sizeof(int32_t) * po + 4);
  int32_t* c2 = (int32_t*)malloc(sizeof(int32_t) * po + 4);
  int rc = 0;
  if (!sftA || !sftB || !lgA || !lgB || !resA || !resB || !res8 || !c1 || !c2 ||
      (use_corr && (!hA || !qA || !hB || !qB))) {
    rc = -1;
    goto done;
  }

  or_size_rows(A, MF, K, bits, sftA, lgA);
  if (b_kn) or_size_cols(B, batch, K, N, bits, sftB, lgB);
  else or_size_rows(B, NF, K, bits, sftB, lgB);
  const int be = or_pick_bits(lgA, MF, lgB, NF, log2M < 126.0f ? log2M : 126.0f, bits, sftA, sftB);
  if (sftA_out) memcpy(sftA_out, sftA, sizeof(int16_t) * MF);
  if (sftB_out) memcpy(sftB_out, sftB, sizeof(int16_t) * NF);
  if (lgA_out) memcpy(lgA_out, lgA, sizeof(float) * MF);
  if (lgB_out) memcpy(lgB_out, lgB, sizeof(float) * NF);
  if (bits_eff_out) *bits_eff_out = be;

  for (int64_t b = 0; b < batch; b++) {
    or_extract_operand(A + b * M * K, 1, M, K, 0, sftA + b * M, be, primes, P, use_corr, resA, hA, qA);
    or_extract_operand(B + b * N * K, 1, N, K, b_kn, sftB + b * N, be, primes, P, use_corr, resB,
                       hB, qB);
    if (K > 131071 && !b_kn) {
      if (or_mm_segmented(resA, hA, qA, resB, hB, qB, M, N, K, primes, P, use_corr, nthreads, be,
                          sftA + b * M, sftB + b * N, exact, out + b * M * N)) {
        rc = -1;
        goto done;
      }
      continue;
    }
    for (int t = 0; t < P; t++)
      or_modgemm(resA + t * pa, resB + t * pb, M, N, K, primes[t], res8 + t * po, NULL, nthreads);
    if (use_corr) {
      or_modgemm(hA, qB, M, N, K, 0, NULL, c1, nthreads);   /* hi7_A q7_B^T */
      or_modgemm(qA, hB, M, N, K, 0, NULL, c2, nthreads);   /* q7_A hi7_B^T */
    }
    or_reconstruct(res8, use_corr ? c1 : NULL, use_corr ? c2 : NULL, M, N, primes, P, be,
                   sftA + b * M, sftB + b * N, exact, out + b * M * N);
  }
done:
  /* free(NULL) is a no-op: every buffer goes, whichever allocation failed. */
  free(sftA); free(sftB); free(lgA); free(lgB); free(resA); free(resB); free(res8);
  free(c1); free(c2);
  free(hA); free(qA); free(hB); free(qB);
  return rc;
}

/* ---- double-double reference GEMM: bench/accuracy.py:21-50 ---------------
 * hi + lo ~ A [M,K] @ Bt [K,N] with Dekker's product (no FMA) and the same
 * two-sum sequence per k. */
static void or_two_prod(double a, double b, double* p, double* e) {
  const double split = 134217729.0; /* 2^27 + 1 */
  *p = a * b;
  const double ca = split * a, cb = split * b;
  const double ah = ca - (ca - a), al = a - ah;
  const double bh = cb - (cb - b), bl = b - bh;
  *e = (((ah * bh - *p) + ah * bl) + al * bh) + al * bl;
}

static void or_two_sum(double a, double b, double* s, double* e) {
  *s = a + b;
  const double bb = *s - a;
  *e = (a - (*s - bb)) + (b - bb);
}

void or_ddgemm_nt(double* hi, double* lo, const double* A, const double* Bt, int64_t M, int64_t N,
                  int64_t K, int nthreads) {
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for num_threads(nthreads) schedule(static)
#endif
  for (int64_t i = 0; i < M; i++)
    for (int64_t j = 0; j < N; j++) {
      double h = 0.0, l = 0.0;
      for (int64_t k = 0; k < K; k++) {
        double p, e, s, t;
        or_two_prod(A[i * K + k], Bt[k * N + j], &p, &e);
        or_two_sum(h, p, &s, &t);
        l = l + (t + e);
        or_two_sum(s, l, &h, &l);
      }
      hi[i * N + j] = h;
      lo[i * N + j] = l;
    }
  (void)nthreads;
}

/* ---- array forms of the scalar restatements (for exhaustive pinning) ---- */

void or_bal8_array(const int32_t* v, int64_t n, int p, int8_t* out) {
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
  for (int64_t i = 0; i < n; i++) out[i] = or_bal8(v[i], p);
}

void or_barrett_bal32_array(const int32_t* y, int64_t n, int p, int32_t* out) {
  const uint32_t mu32 = (uint32_t)((1u << 31) / (unsigned)p);
  for (int64_t i = 0; i < n; i++) out[i] = or_barrett_bal32(y[i], p, mu32, (uint32_t)p << 21);
}

/* Extraction of n elements with per-element shifts: td (the signed scaled
 * integer), balanced residues res[n][P], hi7/q7. */
void or_extract_array(const double* x, const int32_t* shift, int64_t n, int bits_eff,
                      const int32_t* primes, int P, int64_t* td, int8_t* res, int8_t* hi,
                      int8_t* q) {
  for (int64_t i = 0; i < n; i++) {
    int8_t h = 0, qq = 0;
    const uint64_t uu = or_split(x[i], shift[i], bits_eff, 1, &h, &qq);
    td[i] = (int64_t)(uu - ((uint64_t)1 << bits_eff));
    for (int t = 0; t < P; t++) res[i * P + t] = or_residue(uu, primes[t], bits_eff);
    hi[i] = h;
    q[i] = qq;
  }
}

/* Correctly rounded conversion of n signed 128-bit integers given as
 * (hi, lo) 64-bit halves. */
void or_i128_array_to_double(const int64_t* hi, const uint64_t* lo, int64_t n, double* out) {
  for (int64_t i = 0; i < n; i++) {
    const i128 v = (i128)(((unsigned __int128)(uint64_t)hi[i] << 64) | lo[i]);
    out[i] = or_i128_to_double(v);
  }
}
