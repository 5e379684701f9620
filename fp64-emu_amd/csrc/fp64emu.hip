// MI355X-native RARE emulated-FP64 GEMM: HIP kernels for gfx950 and the C ABI
// declared in include/fp64emu.h.
//
// Pipeline per call (one HIP stream, no host synchronisation, no allocation):
//   1. sizing      size_rows_cols_kernel (rows of A and columns of a [K, N]
//                  B in one launch) or size_rows_slabs_kernel +
//                  size_cols_final_kernel (deep column slabs), or
//                  size_rows_kernel (rows of both operands); then
//                  pick_width_kernel, or the same pick inside the
//                  extraction for small products: per-row (A) and
//                  per-column (B) power-of-two shifts, the Cauchy-Schwarz
//                  width pick, bits_eff kept on the device.
//   2. extraction  extract_kernel: exact power-of-two scaling and RNE of the
//                  fp64 values, balanced residues for every modulus and the
//                  hi7/q7 correction operands, written directly in the
//                  MFMA fragment order of the GEMM (tile-blocked planes).
//   3. modgemm     modgemm_kernel / modgemm_mixed_kernel: one INT8-MFMA
//                  engine over all (slot, batch member, output tile, K
//                  split) work items, a 4-stage LDS ring fed by direct
//                  global-to-LDS copies, XCD-aware work order, 256 x 256,
//                  256 x 128 or 128 x 128 tiles, residue slots of shallow
//                  products run back to back; the epilogue reduces residue
//                  slots to balanced int8 and stores correction slots as
//                  raw int32.
//   4. reconstruct reconstruct_kernel: balanced Garner digits with
//                  v_dot4_i32_i8, grouped Horner, exact 128-bit combine with
//                  the correction, correctly rounded conversion, rescale.
//
// The arithmetic each stage computes follows fp64_emu_cuda/fp64_emu.cu of the
// reference (line citations at each kernel); the data layouts, launch shapes
// and the modular reductions are this build's own.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>

#include "fp64emu.h"

namespace {

constexpr int kMaxP = FP64EMU_MAXP;
constexpr int kGarnerWords = (kMaxP + 3) / 4;   // packed int8 Garner factors per row
constexpr int kThreads = 256;
constexpr int kTileR = 256;                      // plane tile rows (A and B alike)
constexpr int kTileK = 64;                       // plane tile depth
constexpr int kTileBytes = kTileR * kTileK;      // 16 KiB, one LDS stage per operand
constexpr int kFragBytes = 1024;                 // 16 rows x 64 k in MFMA lane order
constexpr int kOutBlkBytes = 256;                // one 16x16 int8 output block
constexpr int kMaxSlab = 128;
constexpr int64_t kMaxKSingle = 131071;          // int32 accumulator bound: K * 128^2 < 2^31
constexpr int64_t kMaxKFusedCorr = 65536;        // 2K * 127^2 < 2^31: both cross GEMMs in one
constexpr int64_t kSegK = 65536;                 // K-segmented path: segment depth
constexpr int64_t kMaxKDeep = 128 * kSegK;       // the reference's segmented bound
// x + kMagic (|x| < 2^51) lands on the integer grid of [2^52, 2^53): the sum
// rounds x to the nearest integer, ties to even.
constexpr double kMagic = 6755399441055744.0;
// 1/2 + 2^-20: floor(y RN(1/p) + kHalfUp) = floor(y/p + 1/2) for |y| < 2^27.
constexpr double kHalfUp = 0.5 + 0x1p-20;

typedef int v4i __attribute__((ext_vector_type(4)));

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
  g_err = msg;
  return code;
}

// ---------------------------------------------------------------------------
// Modulus tables, passed to the kernels by value (kernarg segment): no device
// allocation and no host-to-device copy, so the first call is already
// capture-safe.  Definitions follow fp64_emu_cuda/fp64_emu.cu:958-993 and
// :1052 (reference), computed here with an extended-Euclid inverse.
struct ModTables {
  int P;
  int p[kMaxP];
  int mib[kMaxP];                  // (M_t mod p_t)^-1 mod p_t, M_t = prod_{u<t} p_u, balanced
  int nmp[kMaxP * kGarnerWords];   // balanced int8 (-M_u minv_t mod p_t) for u < t, 4 per word
  long long m64[2];                // prod of moduli 0..6 and 7..13 (1 if empty)
  double invp[kMaxP];              // RN(1 / p)
  int c31[kMaxP];                  // 2^31 mod p, balanced: |c31| <= p / 2
  float log2M;                     // float sum of (float)log2(p), as the reference
};

__host__ __device__ constexpr int inv_mod(int a, int m) {
  // Extended Euclid on (a mod m, m); m <= 256, gcd 1 by coprimality.
  int r0 = ((a % m) + m) % m, r1 = m, s0 = 1, s1 = 0;
  while (r1 != 0) {
    const int q = r0 / r1;
    int t = r0 - q * r1; r0 = r1; r1 = t;
    t = s0 - q * s1; s0 = s1; s1 = t;
  }
  return ((s0 % m) + m) % m;
}

// Per-modulus constants of the extraction and the reconstruction.  Entry t depends only on
// p_0 .. p_t, so the table of a modulus list serves every prefix of it.
struct GarnerTab {
  int p[kMaxP];
  // Balanced int8 factors of digit t, 4 per word: byte u < t holds
  // -M_u minv_t mod p_t.
  int nmp[kMaxP * kGarnerWords];
  // The same factors as unsigned bytes in [0, p_t), for digits in [0, p).
  uint32_t ump[kMaxP * kGarnerWords];
  int mib[kMaxP];                  // minv_t = (M_t mod p_t)^-1 mod p_t, M_t = prod_{u<t} p_u,
                                   // balanced (an int8)
  double invp[kMaxP];              // RN(1 / p)
  uint32_t mq[kMaxP];              // ceil(2^32 / p): floor(y / p) = mulhi(y, mq) for y < 2^20
  int c31[kMaxP];                  // 2^31 mod p, balanced (the extraction's limb factor)
};

__host__ __device__ constexpr GarnerTab garner_tables(const int* primes, int P) {
  GarnerTab T{};
  for (int t = 0; t < P; ++t) {
    const int pt = primes[t];
    T.p[t] = pt;
    T.invp[t] = 1.0 / (double)pt;
    long long Mt = 1 % pt;         // M_t mod p_t
    for (int u = 0; u < t; ++u) Mt = (Mt * (primes[u] % pt)) % pt;
    const int mi = inv_mod((int)Mt, pt);
    auto put = [&](int u, long long v) {   // v in [0, p_t): balanced byte u
      int bal = (int)v;
      if (bal > (pt - 1) / 2) bal -= pt;
      T.nmp[t * kGarnerWords + (u >> 2)] |= (int)((uint32_t)(uint8_t)(int8_t)bal << (8 * (u & 3)));
      T.ump[t * kGarnerWords + (u >> 2)] |= (uint32_t)v << (8 * (u & 3));
    };
    long long Mu = 1 % pt;         // M_u mod p_t, running over u
    for (int u = 0; u < t; ++u) {
      put(u, ((pt - Mu) % pt) * mi % pt);
      Mu = (Mu * (primes[u] % pt)) % pt;
    }
    T.mib[t] = 2 * mi > pt ? mi - pt : mi;
    T.mq[t] = (uint32_t)(((1ULL << 32) + (unsigned long long)pt - 1) / (unsigned long long)pt);
    const int c31 = (int)((1LL << 31) % pt);
    T.c31[t] = 2 * c31 > pt ? c31 - pt : c31;
  }
  return T;
}

// The reference's modulus list (fp64_emu/__init__.py:20-22), every plan a
// prefix of it: the modulus-count-specialised reconstruction takes its
// constants from this table at compile time.
constexpr int kDefaultModuli[kMaxP] = {256, 255, 253, 251, 247, 241, 239, 233, 229, 227,
                                       223, 217, 211, 199, 197, 193, 191, 181, 179, 173};
__device__ constexpr GarnerTab kDefaultTab = garner_tables(kDefaultModuli, kMaxP);
// The default-list reconstruction computes the mixed-radix digits of
// X + M/2 (in [0, p_t)) instead of X's balanced ones: since every default
// modulus is 256 or odd, M/2 = sum_t (p_t >> 1) W_t, so digit t of X + M/2 is
// X's balanced digit plus p_t >> 1, and X + M/2 has X's residues except
// r_0 + 128 for p_0 = 256 (M/2 is a multiple of every odd p_t).  Group g's
// balanced value (digits 7g .. 7g+6 at their weights inside the group) is
// then the unsigned one minus this offset.
constexpr long long default_digit_offset(int P, int g) {
  long long off = 0, w = 1;
  for (int t = 7 * g; t < 7 * g + 7 && t < P; ++t) {
    off += (long long)(kDefaultModuli[t] >> 1) * w;
    w *= kDefaultModuli[t];
  }
  return off;
}
// The extraction's default-list kernel takes the 24-bit residue path for
// every plane without a tie fix: each default modulus is 256 or odd, and >= 171.
constexpr bool default_moduli_plain() {
  for (int t = 0; t < kMaxP; ++t) {
    const int p = kDefaultModuli[t];
    if (p < 171 || (!(p & 1) && p != 256)) return false;
  }
  return true;
}
static_assert(default_moduli_plain(), "default moduli: 256 or odd, and >= 171");

int gcd_int(int a, int b) {
  while (b) { const int t = a % b; a = b; b = t; }
  return a;
}

ModTables make_tables(const int32_t* primes, int P) {
  ModTables T;
  std::memset(&T, 0, sizeof(T));
  T.P = P;
  for (int g = 0; g < 2; ++g) {
    long long prod = 1;
    for (int t = 7 * g; t < std::min(7 * g + 7, P); ++t) prod *= primes[t];
    T.m64[g] = prod;
  }
  int pr[kMaxP] = {};
  for (int t = 0; t < P; ++t) pr[t] = primes[t];
  const GarnerTab G = garner_tables(pr, P);
  float l2 = 0.0f;
  for (int t = 0; t < P; ++t) {
    T.p[t] = G.p[t];
    T.mib[t] = G.mib[t];
    T.invp[t] = G.invp[t];
    T.c31[t] = G.c31[t];
    for (int g = 0; g < kGarnerWords; ++g) T.nmp[t * kGarnerWords + g] = G.nmp[t * kGarnerWords + g];
    l2 += (float)std::log2((double)primes[t]);
  }
  T.log2M = l2;
  return T;
}

// ---------------------------------------------------------------------------
// Workspace map.
constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }
int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Division of a work-group index (n < 2^31) by a launch constant d >= 1 with
// one 32 x 32 high multiply, an add and a shift (Granlund and Montgomery,
// "Division by invariant integers using multiplication", 1994, round-up
// form): l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1, and
// n / d = (mulhi(m, n) + n) >> l, exact for every n < 2^31 (the sum stays
// below 2^32).  Work-group indices are uniform, so the divisions stay on the
// scalar unit instead of the vector unit's float-reciprocal sequence.
struct FastDiv {
  uint32_t d, m, l;
  __device__ __forceinline__ uint32_t div(uint32_t n) const { return (__umulhi(m, n) + n) >> l; }
};

FastDiv make_fastdiv(int64_t d) {
  FastDiv f;
  f.d = (uint32_t)std::max<int64_t>(d, 1);
  f.l = 0;
  while ((1ull << f.l) < f.d) ++f.l;
  f.m = (uint32_t)(((1ull << 32) * ((1ull << f.l) - f.d)) / f.d + 1);
  return f;
}

// Column-sizing slab split of a [K, N] operand; the same split as
// fp64_emu_cuda/fp64_emu.cu:1159-1162 so the fp64 sum order matches.
void slab_split(int64_t NF, int64_t K, int64_t* kslab, int* nslab) {
  if (K <= 0 || NF <= 0) { *kslab = 0; *nslab = 0; return; }
  const int64_t nsl0 = std::min<int64_t>(std::max<int64_t>(131072 / NF, 1), kMaxSlab);
  *kslab = (K + nsl0 - 1) / nsl0;
  *nslab = (int)((K + *kslab - 1) / *kslab);
}

// GEMM K-split.  Output tiles x slots are the GEMM's work items; when they
// are few against the 256 CUs (small or skinny products), S groups per tile
// each take a contiguous K range, and reconstruction sums the S residue
// (and correction) planes.  S minimises an estimate of the GEMM's time plus
// the split planes' traffic:
//   max((items S / 256 + 1/2) (k-steps per group + 3) x the time of one
//       k-step,  the planes' bytes / HBM rate)
//   + S x (residue + correction bytes of one output set) / HBM rate
// (fractional rounds of groups plus half a group of tail; the split planes
// cost their reconstruction reads, the GEMM's writes overlapping its MFMAs),
// and a larger S must gain 3%; at least 8 k-steps per group.  Measured in one
// process (whole calls), this picks the best S of {1, 2, 4, 8, 16} or one
// within 2% on 16 of 17 shapes from 128 x 128 x 4096 to 8192^3 (1536^2 x
// 4096 keeps S = 1, 4% slower than 2); the former makespan model,
// ceil(items S / 256) (k-steps + 6), split too little at few tiles
// (1024^2 x 4096: 0.169 against 0.154 ms at S = 2; 1024^2 x 8192: 0.307
// against 0.264 ms) and too much for deep skinny ones (512^2 x 20000: 16
// splits 0.292 ms, 8 splits 0.281 ms).  A function of the shapes only, so
// the workspace size is too.
constexpr int kCUs = 256;
// Item streams: items per work group (see stream_order), for items of more
// than kRunMaxSteps and at most kStreamMaxSteps k-steps.  Measured against
// one item per group, whole calls in one process: 4096^2 x 2560 0.784 ->
// 0.766 ms, 4096^2 x 3072 0.900 -> 0.873, 3000^3 0.554 -> 0.537, 4096^3
// 1.120 -> 1.100 at 8 items per group (2 and 4 gained less, 16 the same as
// 8: 4096^3 1.123 against 1.126 ms, one group per CU there); even at
// 6144^2 x 3072, 6144^2 x 4096 and 8192^2 x 4096; slower from 80 k-steps
// (5120^3 2.02 -> 2.05, 4096^2 x 8192 2.017 -> 2.04, 8192^3 7.14 -> 7.30 at
// 2 items, 7.45 at one group per CU), where the GEMM runs at the part's
// power limit and the time between items is no longer what bounds it.
constexpr int kStreamChain = 8;
constexpr int64_t kStreamMaxSteps = 64;
// Split streams: a last tile column of at most kXMax columns is computed
// beside the wide tiles (modgemm_tile's kXc).
constexpr int kXMax = 2;
constexpr int kMaxSplit = 16;

int choose_ksplit(int64_t batch, int64_t tiles, int64_t nkt, int P, int ncorr, int64_t out_elems,
                  int64_t plane_bytes) {
  constexpr double kStepSeconds = 0.73e-6;   // one k-step of a 256 x 256 group (8192^3)
  constexpr double kHbmBytesPerSecond = 5.0e12;
  const int64_t items = batch * tiles * (P + (ncorr == 1 ? 2 : ncorr));  // fused corr: 2x deep
  const double floor_s = (double)plane_bytes / kHbmBytesPerSecond;
  int best = 1;
  double best_t = 1e300;
  for (int S = 1; S <= kMaxSplit; S *= 2) {
    if (S > 1 && nkt / S < 8) break;
    const double steps = (double)((nkt + S - 1) / S) + 3.0;
    const double gemm = std::max(((double)(items * S) / kCUs + 0.5) * steps * kStepSeconds, floor_s);
    const int nc = (S > 1 && ncorr == 1) ? 2 : ncorr;   // a K-split unfuses the correction
    const double split = (double)S * (double)out_elems * (P + 4.0 * nc) / kHbmBytesPerSecond;
    const double t = gemm + split;
    if (t < best_t * 0.97) { best_t = t; best = S; }
  }
  return best;
}

// The narrow GEMM (256 x 128 tiles, two groups per CU):
// - for products whose 256-column tiles are mostly padding: 128-column tiles
//   cover N with at most 127 padded columns, worth it where that cuts the
//   MFMA work by more than the narrow loop's ~10% lower efficiency at depth
//   (e.g. N = 128: half the work);
// - for a single modulus (no slot run) whose groups are short (k-steps <=
//   kNarrowMaxSteps; the fused correction slot runs twice as many) and
//   numerous enough to give every CU two, so that groups overlap their
//   prologues and epilogues.  Shallow products with two or more moduli run
//   slot runs on 256 x 256 tiles instead (use_slot_runs) when they have a
//   256 x 256 tile per CU, and narrow tiles otherwise (make_layout).
constexpr int64_t kNarrowMaxSteps = 16;

bool use_narrow_gemm(const fp64emu_layout_t& L) {
  if (L.deep) return false;
  const int64_t cols128 = (L.N + 127) / 128 * 128;
  const int64_t rows128 = (std::max<int64_t>(L.M, 1) + 127) / 128 * 128;
  // 128-column tiles save padded work (> ~9%).  Deep products (128 k-steps
  // and more) whose groups stay deep after the K-split (64 k-steps and
  // more), where the narrow loop's extra operand traffic per operation tells,
  // take them only with 128-row tiles too (128 x 128: M padded less as well)
  // or a saving of 40% and more.  Measured at K = 8192: 2048 x 300, 2048 x
  // 640 and 4096 x 384 (two splits of 64 k-steps) ran 5-8% faster on 256 x
  // 256 tiles, 300 x 300 to 640 x 1152 7-13% faster on 128 x 128 tiles;
  // 512 x 384 x 20000 (eight splits of 40) 7% faster on the narrow tiles; at
  // K <= 4096 the narrow tiles won or tied.
  const int64_t nkt = L.Kp / kTileK;
  const bool rows_save = L.nchunk == 1 && rows128 * 11 < L.Mp * 10;
  const bool deep_groups = nkt >= 128 && (nkt + L.ksplit - 1) / L.ksplit >= 64;
  if (cols128 * 11 < L.Np * 10 && (rows_save || !deep_groups || cols128 * 5 <= L.Np * 3))
    return true;
  if (L.ksplit != 1 || L.Kp / kTileK > kNarrowMaxSteps || L.nprimes >= 2) return false;
  const int64_t groups = (int64_t)(L.nprimes + L.ncorr) * L.batch * (L.chunk_rows / kTileR) *
                         (cols128 / 128);
  return groups >= 2 * kCUs;
}

// Slot runs: a shallow product's groups (at most kRunMaxSteps k-steps per
// slot, no K-split) each run residue slots of their tile back to back, so
// the operand copies stream across slots instead of every short group waiting
// for its first stage.  Not for tiles of the mixed launch (a last tile column
// of at most 128 columns under 256-column tiles).  The depth limit, measured
// against one slot per group: runs gain to 32 k-steps (8 x 2048^3 batched
// 1.56 -> 1.51 ms, 8192 x 8192 x 2048 2.47 -> 2.38 ms, 64 x 512^2 x 1536 1.17
// -> 1.14 ms), are even at 64 (4096^3 1.136 against 1.133 ms) and lose at 128
// (8192^3 7.22 -> 7.51 ms).
constexpr int64_t kRunMaxSteps = 32;
// Mixed tiles: 256-column tiles whose last tile column holds at most 128
// columns of N run that column as 128-column tiles in the same launch.
bool use_mixed_tiles(const fp64emu_layout_t& L) {
  return !L.deep && !L.gemm_split && L.gemm_tile_cols == 256 && L.Np / kTileR >= 2 &&
         L.N % kTileR != 0 && L.N % kTileR <= 128;
}

// Only 256 x 256 tiles run slots: the 256 x 128 and 128 x 128 launches hold
// two groups per CU, whose prologues and epilogues already overlap each
// other's MFMAs, and runs there measured even or slower than one slot per
// group (batched 16 x 1000 x 300 x 512: 0.239 against 0.212 ms; 32 x 512 x
// 300 x 1024: 0.412 against 0.355 ms; 8192 x 640 x 2048: 0.373 against 0.325
// ms; 128 x 128^2 x 512: 0.201 against 0.192 ms; even at 256 x 100 x 90 x 320
// and 512 x 64^2 x 256).
bool use_slot_runs(const fp64emu_layout_t& L) {
  if (L.deep || L.ksplit != 1 || L.nprimes < 2 || L.Kp / kTileK > kRunMaxSteps) return false;
  return L.gemm_tile_cols == 256 && !use_mixed_tiles(L);
}

// Residue slots per run.  Slot runs reach only products of at least one
// 256 x 256 output tile per CU (fewer tiles take 256 x 128 or 128 x 128 tiles
// in make_layout).  One run of all P slots per tile when the tiles fill whole
// rounds of CUs, else three runs per tile, whose shorter groups even out the
// last round (batched 512^3 against one run: 68 members 0.612 -> 0.559 ms, 80
// members 0.685 -> 0.625 ms, 200 members 1.558 -> 1.513 ms; 1000 x 256^3 1.89
// -> 1.85 ms; at 64 and 128 members, whole rounds, one run was 0.5-1%
// faster).  One slot per group when the split leaves runs of one.
int slot_run_length(const fp64emu_layout_t& L) {
  const int64_t tiles = L.batch * (L.chunk_rows / kTileR) * (L.Np / kTileR);
  if (tiles <= 0) return 1;   // empty product: no GEMM launch
  const int64_t per_tile = tiles % kCUs == 0 ? 1 : 3;
  const int r = (int)((L.nprimes + per_tile - 1) / per_tile);
  return r >= 2 ? r : 1;
}

// Split streams: a deep product of 256 x 256 tiles for which the planner
// chose a K-split runs one work group per CU instead of rounds of split
// groups.  Its units are the K-deep (tile, slot) products (the correction
// products as two slots) in stream_item's order, in blocks of 32 units (a
// block of tiles sharing their operand panels).  XCD x's 32 groups walk the
// x-th eighth of the blocks' k-steps, group j taking unit j of each block:
// the XCD's groups run the same k-steps of one block together, sharing its
// panels in that XCD's L2, and every XCD has the same number of k-steps.
// With at least eight blocks an eighth spans at least one block, so a unit
// falls into at most two K ranges (stored as the two planes of a K-split of
// 2).  The K-split's rounds leave their last round partly empty (1088
// groups of 256 k-steps on 256 CUs: 5 rounds for 4.25 of work), though the
// part then runs its busy CUs at a higher clock, so that measured whole
// calls, one process, against the K-split: 1024 x 2048 x 32768 1.576 ->
// 1.520 ms, 1024^2 x 32768 (K-split 4) 1.009 -> 0.969, 1024 x 2048 x 16384
// 0.851 -> 0.830, 4 x 512 x 1024 x 16384 batched 1.176 -> 1.168.  Only
// where that was measured to gain: units of at least kSplitMinSteps k-steps
// (1024^2 x 8192: 0.273 -> 0.280 ms, 1024^2 x 4096: 0.150 -> 0.162, where
// the groups' stores at their common end are exposed), and tile counts per
// member and slot that divide or are divided by 32, so that a block's tiles
// belong to one slot (36 and 48 tiles: 1500^2 x 30000 1.501 -> 1.534 ms,
// 3000 x 1000 x 20000 1.364 -> 1.374).  Not with a last tile column of at
// most 128 columns (the mixed launch's half-width tiles).
constexpr int64_t kSplitMinSteps = 256;
// Extra columns: N mod 256 in 1 .. kXMax past at least one wide tile column.
int split_extra_cols(const fp64emu_layout_t& L) {
  const int r = (int)(L.N % kTileR);
  return (L.Np / kTileR >= 2 && r >= 1 && r <= kXMax) ? r : 0;
}
bool use_split_streams(const fp64emu_layout_t& L) {
  if (L.deep || L.nchunk != 1 || L.ksplit < 2 || use_narrow_gemm(L)) return false;
  const int xc = split_extra_cols(L);
  if (!xc && L.Np / kTileR >= 2 && L.N % kTileR != 0 && L.N % kTileR <= 128) return false;
  if (L.Kp / kTileK < kSplitMinSteps) return false;
  const int64_t tiles = (L.Mp / kTileR) * (L.Np / kTileR - (xc ? 1 : 0));
  if (tiles % 32 != 0 && 32 % tiles != 0) return false;
  const int64_t units = (int64_t)(L.nprimes + (L.use_corr ? 2 : 0)) * L.batch * tiles;
  return (units + 31) / 32 >= 8;
}

// nchunk_req > 1 (batch 1, not K-segmented): the planes of A and the output
// planes hold one chunk of ceil(TM / nchunk_req) row tiles at a time.
void make_layout(int64_t batch, int64_t M, int64_t N, int64_t K, int P, bool corr,
                 fp64emu_layout_t* L, int64_t nchunk_req = 1) {
  std::memset(L, 0, sizeof(*L));
  L->batch = batch; L->M = M; L->N = N; L->K = K;
  L->nprimes = P; L->use_corr = corr ? 1 : 0;
  // K-segmented (K > 131071, B as [N, K]): planes hold one segment; each
  // segment's correction is one fused GEMM; the GEMMs accumulate into int32
  // residue sums and one int64 correction sum.
  L->deep = K > kMaxKSingle ? 1 : 0;
  L->kseg = L->deep ? kSegK : K;
  L->nseg = L->deep ? (int)((K + kSegK - 1) / kSegK) : 1;
  L->ncorr = corr ? ((L->deep || K <= kMaxKFusedCorr) ? 1 : 2) : 0;
  int64_t kslab; int nslab;
  slab_split(batch * N, K, &kslab, &nslab);
  L->nslab = nslab;
  L->Mp = round_up(std::max<int64_t>(M, 1), kTileR);
  L->Np = round_up(std::max<int64_t>(N, 1), kTileR);
  L->Kp = round_up(L->kseg, kTileK);
  const int64_t TM = L->Mp / kTileR;
  int64_t ctiles = TM;
  if (nchunk_req > 1 && batch == 1 && !L->deep) ctiles = (TM + nchunk_req - 1) / nchunk_req;
  L->nchunk = (int)((TM + ctiles - 1) / ctiles);
  L->chunk_rows = ctiles * kTileR;
  L->planeA_bytes = L->chunk_rows * L->Kp;
  L->planeB_bytes = L->Np * L->Kp;
  const int nplanes = P + (corr ? 2 : 0);   // the correction plane is 2*Kp deep
  L->memberA_bytes = (int64_t)nplanes * L->planeA_bytes;
  L->memberB_bytes = (int64_t)nplanes * L->planeB_bytes;
  L->outplane_bytes = L->chunk_rows * L->Np;
  // (K-segmented: per segment launch; each split keeps its own int32 residue
  // and int64 correction sums across the segments.)
  L->ksplit = choose_ksplit(batch, ctiles * (L->Np / kTileR), L->Kp / kTileK, P, L->ncorr,
                            batch * L->outplane_bytes, batch * (L->memberA_bytes + L->memberB_bytes));
  // Under a K-split the two correction products run as two K-deep slots
  // (two int32 planes): a fused 2K-deep slot would make its groups twice as
  // long as every residue group (choose_ksplit already counts it as two).
  if (L->ksplit > 1 && L->ncorr == 1) L->ncorr = 2;
  if (use_split_streams(*L)) {
    L->gemm_split = 1;
    L->ksplit = 2;
  }
  size_t o = 0;
  auto take = [&](size_t bytes) { const size_t at = o; o = align_up(o + bytes); return at; };
  L->off_sftA = take(sizeof(int16_t) * batch * M);
  L->off_sftB = take(sizeof(int16_t) * batch * N);
  L->off_lgA = take(sizeof(float) * batch * M);
  L->off_lgB = take(sizeof(float) * batch * N);
  L->off_bits = take(sizeof(int) * 4);
  L->off_pmax = take(sizeof(double) * (size_t)nslab * batch * N);
  L->off_pss = take(sizeof(double) * (size_t)nslab * batch * N);
  L->off_planesA = take((size_t)(batch * L->memberA_bytes));
  L->off_planesB = take((size_t)(batch * L->memberB_bytes));
  L->off_res8 = take((L->deep ? sizeof(int32_t) : 1) *
                     (size_t)(L->ksplit * batch * P * L->outplane_bytes));
  L->off_corr = take((L->deep ? sizeof(int64_t) : sizeof(int32_t)) *
                     (size_t)(L->ksplit * batch * L->ncorr * L->outplane_bytes));
  L->total = o;
  L->gemm_tile_cols = (!L->gemm_split && use_narrow_gemm(*L)) ? 128 : 256;
  // 128 x 128 tiles where 128-row tiles also cut the padded work by > 10%
  // (M <= 128: half): two groups per CU, a quarter of the 256 x 256 work.
  const int64_t rows128 = (std::max<int64_t>(M, 1) + 127) / 128 * 128;
  L->gemm_tile_rows = (L->gemm_tile_cols == 128 && L->nchunk == 1 && rows128 * 11 < L->Mp * 10)
                          ? 128 : 256;
  // Shallow products (at most kRunMaxSteps k-steps, no K-split, two moduli or
  // more) with fewer 256 x 256 output tiles than CUs run one slot per group
  // on 256 x 128 tiles, two groups per CU (128 x 128 tiles at 40 tiles or
  // fewer): measured against 256 x 256 tiles in runs split to fill the chip,
  // 3-18% faster on 17 of 19 shapes from 512^3 and batched 8 x 512^3 to
  // 3584^2 x 1536 (e.g. 2 x 2048^3 batched 0.506 -> 0.421 ms, 3072^2 x 1024
  // 0.302 -> 0.257 ms, 1500^3 0.147 -> 0.121 ms on 128 x 128), even on the
  // other two; from 256 tiles on the 256 x 256 runs stay faster (c4 0.490
  // against 0.516 ms, 80 x 512^3 0.620 against 0.627 ms).
  {
    const int64_t tiles = batch * (L->chunk_rows / kTileR) * (L->Np / kTileR);
    if (!L->deep && L->ksplit == 1 && P >= 2 && L->Kp / kTileK <= kRunMaxSteps && tiles > 0 &&
        tiles < kCUs) {
      L->gemm_tile_cols = 128;
      if (L->nchunk == 1 && tiles <= 40) L->gemm_tile_rows = 128;
    }
  }
  L->gemm_run = use_slot_runs(*L) ? slot_run_length(*L) : 1;
  // Plane rows the GEMM reads: 128-row (128-column) tiles read only the
  // first half of a 256-row plane tile past the last one holding data, so
  // the extraction skips the all-padding half there; a split stream's extra
  // columns read only the last tile's first 16 rows (a 64-row group).
  L->ext_rowsA = L->gemm_tile_rows == 128 ? round_up(std::max<int64_t>(M, 1), 128) : L->chunk_rows;
  if (L->gemm_split && split_extra_cols(*L) > 0)
    L->ext_rowsB = round_up(N, 64);
  else
    L->ext_rowsB = (L->gemm_tile_cols == 128 || use_mixed_tiles(*L))
                       ? round_up(std::max<int64_t>(N, 1), 128) : L->Np;
}

// ---------------------------------------------------------------------------
// Sizing.  Per row: max|x| and the fp64 sum of squares with the reference's
// order (thread-strided partial sums, FMA accumulate, 256-wide tree), so the
// Cauchy-Schwarz decision is reproducible by the CPU restatement.
// fp64_emu_cuda/fp64_emu.cu:107-146.
__device__ __forceinline__ void row_stats_out(double m, double s2, int bits, int16_t* sft,
                                              float* lg) {
  const int e = (m > 0.0 && isfinite(m)) ? ilogb(m) : 0;
  const int sh = (bits - 1) - e;
  float l;
  if (s2 > 0.0 && isfinite(s2)) l = (float)(0.5 * log2(s2) + (double)sh);
  else l = (m > 0.0) ? INFINITY : -INFINITY;
  *lg = l;
  *sft = (int16_t)sh;
}

// One wave per row (four rows per block).  Lane l stands for the partial
// sums l, l + 64, l + 128 and l + 192 of a 256-thread row pass: element c
// goes to sum c % 256, FMA-accumulated in increasing c, and the 256 sums
// fold by the same pairwise tree (strides 128 and 64 inside the lane, 32 .. 1
// across lanes), so the sum of squares is the one the 256-thread form gives.
constexpr int kRowsPerBlock = kThreads / 64;

template <int kBlocks>
__device__ __forceinline__ void row_pass(const double* __restrict__ x, int64_t c, double& mx,
                                         double (&ss)[4]) {
  double v[4 * kBlocks];
#pragma unroll
  for (int u = 0; u < 4 * kBlocks; ++u) v[u] = x[c + 64 * u];
#pragma unroll
  for (int u = 0; u < 4 * kBlocks; ++u) {
    mx = fmax(mx, fabs(v[u]));
    ss[u & 3] = fma(v[u], v[u], ss[u & 3]);
  }
}

// kGroup: few rows (not enough waves to fill the chip): a 256-thread group
// per row, its wave w running sum 64 w + l alone (sixteen of its loads in
// flight), the four waves' sums meeting in LDS before the same fold.  A
// block of kWaves waves holds kWaves / 4 such groups, or kWaves rows (one
// per wave) otherwise.
template <bool kGroup, int kWaves>
__device__ __forceinline__ void size_rows_body(int64_t bid, const double* __restrict__ A, int64_t rowsA,
                                               const double* __restrict__ B, int64_t rows, int64_t K,
                                               int bits, int16_t* __restrict__ sftA,
                                               float* __restrict__ lgA, int16_t* __restrict__ sftB,
                                               float* __restrict__ lgB) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row = kGroup ? bid * (kWaves / 4) + (wave >> 2) : bid * kWaves + wave;
  const bool isA = row < rowsA;
  const int64_t r = isA ? row : row - rowsA;
  const double* __restrict__ x = (isA ? A : B) + r * K + lane;
  double mx = 0.0, ss[4] = {0.0, 0.0, 0.0, 0.0};
  if constexpr (kGroup) {
    // Every wave reaches the barrier; rows past the last only skip loads.
    const int wg = wave & 3;
    const double* __restrict__ xw = x + 64 * wg;
    double sw = 0.0, mw = 0.0;
    // Elements past K read as 0, which leaves both the max and the sum
    // (never -0) unchanged.
    if (row < rows) {
      for (int64_t c = 0; c < K; c += 4096) {
        double v[16];
#pragma unroll
        for (int i = 0; i < 16; ++i)
          v[i] = c + 256 * i + 64 * wg + lane < K ? xw[c + 256 * i] : 0.0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          mw = fmax(mw, fabs(v[i]));
          sw = fma(v[i], v[i], sw);
        }
      }
    }
    __shared__ double sh_ss[kWaves][64], sh_mx[kWaves][64];
    sh_ss[wave][lane] = sw;
    sh_mx[wave][lane] = mw;
    __syncthreads();
    if (wg != 0 || row >= rows) return;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      ss[u] = sh_ss[wave + u][lane];
      mx = fmax(mx, sh_mx[wave + u][lane]);
    }
  } else {
    if (row >= rows) return;
    // Sixteen loads in flight, then eight, then guarded 256-element blocks.
    int64_t c = 0;
    for (; c + 1024 <= K; c += 1024) row_pass<4>(x, c, mx, ss);
    if (c + 512 <= K) {
      row_pass<2>(x, c, mx, ss);
      c += 512;
    }
    for (; c < K; c += 256) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (c + 64 * u + lane < K) {
          const double v = x[c + 64 * u];
          mx = fmax(mx, fabs(v));
          ss[u] = fma(v, v, ss[u]);
        }
      }
    }
  }
  double t = (ss[0] + ss[2]) + (ss[1] + ss[3]);
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) {
    t = t + __shfl_down(t, s);
    mx = fmax(mx, __shfl_down(mx, s));
  }
  if (lane == 0) {
    if (isA) row_stats_out(mx, t, bits, &sftA[r], &lgA[r]);
    else row_stats_out(mx, t, bits, &sftB[r], &lgB[r]);
  }
}

template <bool kGroup>
__global__ void __launch_bounds__(kThreads)
size_rows_kernel(const double* __restrict__ A, int64_t rowsA, const double* __restrict__ B,
                 int64_t rows, int64_t K, int bits, int16_t* __restrict__ sftA,
                 float* __restrict__ lgA, int16_t* __restrict__ sftB, float* __restrict__ lgB) {
  size_rows_body<kGroup, kThreads / 64>(blockIdx.x, A, rowsA, B, rows, K, bits, sftA, lgA, sftB, lgB);
}

// A wave per row when the rows give the chip at least four waves per SIMD,
// else a 256-thread group per row.
constexpr int64_t kRowsGroupBelow = 4096;

void launch_size_rows(int64_t rows, hipStream_t s, const double* A, int64_t rowsA, const double* B,
                      int64_t K, int bits, int16_t* sftA, float* lgA, int16_t* sftB, float* lgB) {
  if (rows < kRowsGroupBelow)
    hipLaunchKernelGGL(size_rows_kernel<true>, dim3((unsigned)rows), dim3(kThreads), 0, s, A, rowsA,
                       B, rows, K, bits, sftA, lgA, sftB, lgB);
  else
    hipLaunchKernelGGL(size_rows_kernel<false>, dim3((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock)),
                       dim3(kThreads), 0, s, A, rowsA, B, rows, K, bits, sftA, lgA, sftB, lgB);
}

// The sizing of A's rows and of the [K, N] operand's columns in one launch
// of 1024-thread groups.  Column statistics follow fp64_emu_cuda/fp64_emu.cu:148-189,
// which takes them in two launches (slab partials, then their fold): per
// column, nslab k-slabs of kslab rows (slab_split), each slab's max |x| and
// FMA-accumulated sum of squares taken over its rows in order, then folded
// in slab order.  Here a column group holds cpw = 1024 / nslab columns and
// every slab of each: thread t takes slab t / cpw of column t % cpw (adjacent
// threads read adjacent columns of one operand row), its partials meet in
// LDS, and one thread per column folds them, so no partials go through
// memory and no second launch waits for them.  The column groups come
// first: each thread walks its slab's rows in one dependent chain, so they
// are the launch's longest groups, and starting them first lets the row
// groups (16 rows per group, a wave each; 4 rows of 256 threads when the
// rows are few) fill in around them.
// For slabs of at most kFusedSlabRows rows.  Past that the ~128 column
// groups (nslab x columns is about 131072 from 1024 columns on) hold long
// chains on half the CUs, and the two-launch form, whose slab groups spread
// over every CU, measured faster (1023 x 2049 x 32769: 1.62 against 1.66 ms
// per call; 100 x 20000 x 3000: 0.673 against 0.704 ms); at 128-row slabs
// the single launch was even or faster (batched 64 x 512^3 0.497 -> 0.485
// ms, 4096^3 even), and on small products it saves the second launch
// (128 x 128 x 4096 48.3 -> 46.2 us, 512^3 43.5 -> 38.8 us, 1000^3 70.9 ->
// 66.3 us).
constexpr int kSizeThreads = 1024;
constexpr int64_t kFusedSlabRows = 256;

template <bool kGroup>
__global__ void __launch_bounds__(kSizeThreads)
size_rows_cols_kernel(const double* __restrict__ A, int64_t rowsA, int64_t ncolgrp, int64_t K, int bits,
                      int16_t* __restrict__ sftA, float* __restrict__ lgA,
                      const double* __restrict__ X, int64_t totalcols, int64_t cols_per,
                      int64_t kslab, int nslab, int cpw, int16_t* __restrict__ sftB,
                      float* __restrict__ lgB) {
  const int64_t bid = blockIdx.x;
  if (bid >= ncolgrp) {
    size_rows_body<kGroup, kSizeThreads / 64>(bid - ncolgrp, A, rowsA, A, rowsA, K, bits, sftA, lgA,
                                              nullptr, nullptr);
    return;
  }
  __shared__ double sh_m[kSizeThreads], sh_s[kSizeThreads];
  const int t = threadIdx.x;
  const int sl = t / cpw, c = t - sl * cpw;
  const int64_t j = bid * cpw + c;
  double mx = 0.0, ss = 0.0;
  if (sl < nslab && j < totalcols) {
    const int64_t b = j / cols_per, n = j - b * cols_per;
    const int64_t k0 = (int64_t)sl * kslab;
    const int64_t k1 = min(k0 + kslab, K);
    const double* __restrict__ base = X + b * K * cols_per + n;
    // Sixteen rows in flight per thread; the fma chain keeps the slab order.
    int64_t k = k0;
    for (; k + 16 <= k1; k += 16) {
      double v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = base[(k + u) * cols_per];
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        mx = fmax(mx, fabs(v[u]));
        ss = fma(v[u], v[u], ss);
      }
    }
    for (; k < k1; ++k) {
      const double v = base[k * cols_per];
      mx = fmax(mx, fabs(v));
      ss = fma(v, v, ss);
    }
  }
  sh_m[t] = mx;
  sh_s[t] = ss;
  __syncthreads();
  if (t >= cpw || j >= totalcols) return;
  // Slabs folded in order, sixteen LDS reads ahead of the adds.
  double fm = 0.0, fs = 0.0;
  int q = 0;
  for (; q + 16 <= nslab; q += 16) {
    double m[16], v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      m[u] = sh_m[(q + u) * cpw + t];
      v[u] = sh_s[(q + u) * cpw + t];
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      fm = fmax(fm, m[u]);
      fs = fs + v[u];
    }
  }
  for (; q < nslab; ++q) {
    fm = fmax(fm, sh_m[q * cpw + t]);
    fs = fs + sh_s[q * cpw + t];
  }
  row_stats_out(fm, fs, bits, &sftB[j], &lgB[j]);
}

// Column partials of a [K, N] operand (per batch member): thread j owns
// global column j, blockIdx.y a k-slab summed in order.
// fp64_emu_cuda/fp64_emu.cu:148-169.
__device__ __forceinline__ void size_cols_partial_body(int64_t bx, int64_t by, const double* __restrict__ X,
                                                       int64_t totalcols, int64_t rows_per,
                                                       int64_t cols_per, int64_t kslab,
                                                       double* __restrict__ pmax,
                                                       double* __restrict__ pss) {
  const int64_t j = bx * kThreads + threadIdx.x;
  if (j >= totalcols) return;
  const int64_t b = j / cols_per, n = j - b * cols_per;
  const int64_t k0 = by * kslab;
  const int64_t k1 = min(k0 + kslab, rows_per);
  const double* __restrict__ base = X + b * rows_per * cols_per + n;
  double mx = 0.0, ss = 0.0;
  // Sixteen rows in flight per thread; the fma chain keeps the slab order.
  int64_t k = k0;
  for (; k + 16 <= k1; k += 16) {
    double v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = base[(k + u) * cols_per];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      mx = fmax(mx, fabs(v[u]));
      ss = fma(v[u], v[u], ss);
    }
  }
  for (; k < k1; ++k) {
    const double v = base[k * cols_per];
    mx = fmax(mx, fabs(v));
    ss = fma(v, v, ss);
  }
  pmax[by * totalcols + j] = mx;
  pss[by * totalcols + j] = ss;
}

// Deep columns (slabs of more than kFusedSlabRows rows): the sizing of A's
// rows and of the [K, N] operand's column slabs in one launch of 256-thread
// groups, groups [0, ncol) taking column slabs (x fastest), the rest rows;
// size_cols_final_kernel then folds the slabs.
// The slab groups come first: each thread walks its slab's rows in one
// dependent chain, so they are the launch's longest groups, and starting
// them first lets the row groups fill in around them instead of leaving
// them as a tail.
template <bool kGroup>
__global__ void __launch_bounds__(kThreads)
size_rows_slabs_kernel(const double* __restrict__ A, int64_t rowsA, int64_t ncol, int64_t K, int bits,
                       int16_t* __restrict__ sftA, float* __restrict__ lgA,
                       const double* __restrict__ X, int64_t totalcols, int64_t cols_per,
                       int64_t kslab, int64_t gcx, double* __restrict__ pmax,
                       double* __restrict__ pss) {
  const int64_t bid = blockIdx.x;
  if (bid < ncol) {
    size_cols_partial_body(bid % gcx, bid / gcx, X, totalcols, K, cols_per, kslab, pmax, pss);
  } else {
    size_rows_body<kGroup, kThreads / 64>(bid - ncol, A, rowsA, A, rowsA, K, bits, sftA, lgA, nullptr,
                                          nullptr);
  }
}

// Slabs folded in order.  fp64_emu_cuda/fp64_emu.cu:171-189.  A group
// covers 64 columns: its 256 threads bring the columns' slab partials into
// LDS (up to 64 loads in flight each, one round trip), then one lane per
// column folds them in slab order.
constexpr int kFinalCols = 64;

__global__ void __launch_bounds__(kThreads)
size_cols_final_kernel(const double* __restrict__ pmax, const double* __restrict__ pss,
                       int64_t totalcols, int nslab, int bits, int16_t* __restrict__ sft,
                       float* __restrict__ lg) {
  __shared__ double sh_m[kMaxSlab * kFinalCols], sh_s[kMaxSlab * kFinalCols];
  const int tid = threadIdx.x;
  const int64_t j0 = (int64_t)blockIdx.x * kFinalCols;
  const int n = nslab * kFinalCols;                      // entries f = slab * 64 + column
  constexpr int kPer = kMaxSlab * kFinalCols / kThreads;  // 32
  double vm[kPer], vs[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int f = tid + kThreads * i;
    const int64_t j = j0 + (f & (kFinalCols - 1));
    const bool ok = f < n && j < totalcols;
    const int64_t at = (int64_t)(f / kFinalCols) * totalcols + j;
    vm[i] = ok ? pmax[at] : 0.0;
    vs[i] = ok ? pss[at] : 0.0;
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int f = tid + kThreads * i;
    if (f < n) {
      sh_m[f] = vm[i];
      sh_s[f] = vs[i];
    }
  }
  __syncthreads();
  const int64_t j = j0 + tid;
  if (tid >= kFinalCols || j >= totalcols) return;
  double mx = 0.0, ss = 0.0;
  int sl = 0;
  for (; sl + 16 <= nslab; sl += 16) {   // sixteen LDS reads ahead of the adds
    double m[16], v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      m[u] = sh_m[(sl + u) * kFinalCols + tid];
      v[u] = sh_s[(sl + u) * kFinalCols + tid];
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      mx = fmax(mx, m[u]);
      ss = ss + v[u];
    }
  }
  for (; sl < nslab; ++sl) {
    mx = fmax(mx, sh_m[sl * kFinalCols + tid]);
    ss = ss + sh_s[sl * kFinalCols + tid];
  }
  row_stats_out(mx, ss, bits, &sft[j], &lg[j]);
}

// Width pick: g = floor((log2M - 1 - (max lgA + max lgB + 0.5)) / 2),
// g <= 53 - bits, be = max(bits + g, 16).  bits_eff[0] = be and
// bits_eff[1] = be - bits, the amount every per-row and per-column shift
// grows by; the consumers add it on the fly, so the shifts are never
// rewritten.  fp64_emu_cuda/fp64_emu.cu:191-231.
constexpr int kPickThreads = 1024;

__device__ __forceinline__ float max4(float4 v) { return fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)); }

// Max of lg[0, n) over a block of T threads: eight float4 loads in flight
// per thread (the workspace slices are 256-byte aligned), a scalar tail.
template <int T>
__device__ __forceinline__ float block_max_lg(const float* __restrict__ lg, int64_t n, int tid) {
  const float4* __restrict__ v4 = reinterpret_cast<const float4*>(lg);
  const int64_t n4 = n / 4;
  float a = -INFINITY;
  int64_t i = tid;
  for (; i + 7 * T < n4; i += 8 * T) {
    float4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = v4[i + u * T];
#pragma unroll
    for (int u = 0; u < 8; ++u) a = fmaxf(a, max4(v[u]));
  }
  for (; i < n4; i += T) a = fmaxf(a, max4(v4[i]));
  if (tid < n - 4 * n4) a = fmaxf(a, lg[4 * n4 + tid]);
  return a;
}

// max lgA[0, m) and max lgB[0, n), in every thread of a block of T (the
// values are +-inf or finite, so the order of the maxima does not matter).
template <int T>
__device__ __forceinline__ void block_max_lg_pair(const float* __restrict__ lgA, int64_t m,
                                                  const float* __restrict__ lgB, int64_t n, float& a,
                                                  float& b) {
  __shared__ float sa[T / 64], sb[T / 64];
  const int tid = threadIdx.x;
  a = block_max_lg<T>(lgA, m, tid);
  b = block_max_lg<T>(lgB, n, tid);
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) {
    a = fmaxf(a, __shfl_xor(a, s));
    b = fmaxf(b, __shfl_xor(b, s));
  }
  if ((tid & 63) == 0) {
    sa[tid >> 6] = a;
    sb[tid >> 6] = b;
  }
  __syncthreads();
  a = sa[0];
  b = sb[0];
#pragma unroll
  for (int w = 1; w < T / 64; ++w) {
    a = fmaxf(a, sa[w]);
    b = fmaxf(b, sb[w]);
  }
}

// be from the maxima of the row and column log2-norms.
__device__ __forceinline__ int pick_width(float a, float b, float log2M, int bits) {
  const float need = a + b + 0.5f;
  int g = 0;
  if (isfinite(need)) g = (int)floorf((log2M - 1.0f - need) * 0.5f);
  g = min(g, 53 - bits);
  return max(bits + g, 16);
}

__global__ void __launch_bounds__(kPickThreads)
pick_width_kernel(const float* __restrict__ lgA, int64_t m, const float* __restrict__ lgB,
                  int64_t n, float log2M, int bits, int* __restrict__ bits_eff) {
  float a, b;
  block_max_lg_pair<kPickThreads>(lgA, m, lgB, n, a, b);
  if (threadIdx.x == 0) {
    const int be = pick_width(a, b, log2M, bits);
    bits_eff[0] = be;
    bits_eff[1] = be - bits;
  }
}

// Products of at most kPickInExtractMax rows and columns in all (one row
// chunk, one K segment) take the width pick inside the extraction instead:
// every extraction group reads both log2-norm vectors (at most 16 KiB) and
// reduces them itself, and group 0 stores bits_eff for the reconstruction,
// which saves the pick's launch (small products are bound by their chain of
// launches).  Measured against the separate launch: 512^3 mm_nt 43.5 ->
// 37.8 us with the single column-sizing launch, mm 36.9 -> 35.3 us, 1000^3
// 64.7 -> 62.6 us (mm); up to kPickInExtractBytes of those reads over the
// launch (2048^3: 32 MiB, still 3% faster); past it the reads cost more
// than the launch (1023 x 2049 x 32769: 295 MiB, 1.609 against 1.620 ms).
constexpr int64_t kPickInExtractMax = 4096;
constexpr int64_t kPickInExtractBytes = 64ll << 20;

// ---------------------------------------------------------------------------
// Extraction.  Element semantics follow fp64_emu_cuda/fp64_emu.cu:288-321
// (RNE scaling of |x| by 2^shift, hi7/q7 correction summaries), computed
// here with exact power-of-two fp64 operations instead of integer shifts of
// the IEEE encoding; the residue reduction is this build's: the signed integer
// td = +-round(|x| 2^s) splits as th * 2^27 + tl (th signed, tl < 2^27),
// v = th * (2^27 mod p) + tl is exact in fp64 (|v| < 2^35), and
// r = v - p * RNE(v / p) is exact: the quotient error (< 2^-26) stays far
// below the distance 1/(2p) of v/p from a half-integer for odd p, and 1/256
// is exact.  r is the balanced residue; p = 256 may give +128, whose byte is
// the reference's -128.
//
// Plane layout (per batch member, per plane): 256-row x 64-k tiles, row tile
// major, k tile minor; a tile holds 16 fragments of 16 rows x 64 k, fragment
// f = row % 256 / 16, each 1 KiB in the operand order of
// v_mfma_i32_16x16x64_i8: lane l = 16 * (k % 64 / 16) + (row % 16) holds
// k % 16 at byte 16 * l + k % 16 (A's rows and B's columns alike, so any
// order of the 16 k inside a lane pairs up in the dot product).  The correction plane is one 2*Kp-deep
// plane: A = [hi7 | q7], B = [q7 | hi7], so one GEMM accumulates
// hi7_A q7_B^T + q7_A hi7_B^T.

// Balanced residue of an int32: acc - q p with q the nearest integer to
// acc RN(1/p), read off the low word of fma(acc, RN(1/p), kMagic) (the sum's
// mantissa holds 2^51 + q); exact while |q| < 2^23, for the 24-bit
// multiply-add.  A modular-GEMM group of klen <= 131071 k-terms of balanced
// residues gives |acc| <= klen p^2/4, so |q| <= klen p/4 + 1 < 2^23.
__device__ __forceinline__ int acc_residue(int acc, double ip, int negp) {
  const int q = __double2loint(fma((double)acc, ip, kMagic));
  return __mul24(q, negp) + acc;
}

// sdot4 of two packed int8 words with a zero accumulator, in the VOP3P form
// (the builtin with a constant accumulator becomes a move and the in-place
// VOP2 form).
__device__ __forceinline__ int sdot4_zero(uint32_t a, uint32_t b) {
  int r;
  asm("v_dot4_i32_i8 %0, %1, %2, 0" : "=v"(r) : "v"(a), "s"(b));
  return r;
}

// Low bytes of four ints, packed little-endian into one dword.
__device__ __forceinline__ uint32_t pack_bytes(int r0, int r1, int r2, int r3) {
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)r1, (uint32_t)r0, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)r3, (uint32_t)r2, 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

struct ExtractCore {
  const double* A;
  const double* B;
  int64_t M, N, K, batch;   // K: depth extracted by this launch (one segment)
  int64_t lda, k0;          // full operand depth and this segment's first k
  int b_kn;          // B given as [K, N] (mm_nt / bmm_nt)
  int use_corr;
  int64_t nkt;       // Kp / 64
  int64_t planeA, planeB, memberA, memberB;
  int64_t rgA, rgB;  // 64-row groups per member the GEMM reads (0: B not extracted)
  int64_t rgA_data, rgB_data;   // those holding operand rows: ceil(M / 64), ceil(N / 64)
  // Dividers of the work-group decomposition: by nkt, and by the row-group
  // count of each segment (A data, B data, A padding, B padding).
  FastDiv div_nkt, div_rg[4];
  const int16_t* sftA;
  const int16_t* sftB;
  const int* bits_eff;
  // pick != 0: the width pick from lgA[0, nlgA) and lgB[0, nlgB) in every
  // group; group 0 stores bits_eff (bits_out) for the reconstruction.
  int pick, bits;
  float log2M;
  const float* lgA;
  const float* lgB;
  int64_t nlgA, nlgB;
  int* bits_out;
  int8_t* planesA;
  int8_t* planesB;
  int P;             // modulus count
};

// The kernels of the default modulus list take its constants at compile time
// and no tables: a smaller kernel-argument block (about 1 KiB less), which a
// dependent launch waits for (a 1 KiB block cost ~1.4 us per launch in a
// back-to-back probe).  Any other list takes its tables by value.
template <bool kTab> struct ExtractArgs : ExtractCore { ModTables tab; };
template <> struct ExtractArgs<false> : ExtractCore {};

// kDefault: the modulus list is a prefix of the default one, whose constants
// the plane loop takes at compile time (no scalar load and wait per plane,
// which dominated small launches); otherwise the tables of the arguments.
template <bool kDefault>
__global__ void __launch_bounds__(kThreads)
extract_kernel(ExtractArgs<!kDefault> a) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // The width pick, when this launch takes it: every wave reaches the
  // block's barrier before any returns.
  int pick_be = 0;
  if (a.pick) {
    float ma, mb;
    block_max_lg_pair<kThreads>(a.lgA, a.nlgA, a.lgB, a.nlgB, ma, mb);
    pick_be = pick_width(ma, mb, a.log2M, a.bits);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
      a.bits_out[0] = pick_be;
      a.bits_out[1] = pick_be - a.bits;
    }
  }
  // Work groups: the row groups holding operand rows of A, then of B, then
  // the all-padding row groups of A and of B (zero stores only), so that the
  // work spreads evenly over the XCDs (group i runs on XCD i % 8) whatever
  // the padding.
  uint32_t wg = blockIdx.x;
  const uint32_t nA = (uint32_t)(a.batch * a.rgA_data * a.nkt), nB = (uint32_t)(a.batch * a.rgB_data * a.nkt);
  const uint32_t nAp = (uint32_t)(a.batch * (a.rgA - a.rgA_data) * a.nkt);
  bool isA;
  int seg;
  int64_t rg_off = 0;
  if (wg < nA) {
    isA = true; seg = 0;
  } else if ((wg -= nA) < nB) {
    isA = false; seg = 1;
  } else if ((wg -= nB) < nAp) {
    isA = true; seg = 2; rg_off = a.rgA_data;
  } else {
    wg -= nAp;
    isA = false; seg = 3; rg_off = a.rgB_data;
  }
  const FastDiv& rgd = a.div_rg[seg];
  const bool kn = !isA && a.b_kn;
  // Work group -> (member, 64-row group, k tile).  Row-major operands walk k
  // fastest (consecutive groups read consecutive bytes of the same rows);
  // the [K, N] operand walks the 64-column group fastest.
  int64_t b, rg, kt;
  if (kn) {
    const uint32_t t = rgd.div(wg);
    rg = wg - t * rgd.d;
    const uint32_t bb = a.div_nkt.div(t);
    kt = t - bb * a.div_nkt.d;
    b = bb;
  } else {
    const uint32_t t = a.div_nkt.div(wg);
    kt = wg - t * a.div_nkt.d;
    const uint32_t bb = rgd.div(t);
    rg = t - bb * rgd.d;
    b = bb;
  }
  rg += rg_off;
  const int64_t R = isA ? a.M : a.N;
  const int64_t K = a.K;
  // Wave w covers rows 64 rg + 16 w .. +16 and the whole k tile: one
  // 16 x 64 fragment, lane l = 16 (k / 16) + row % 16 holding 16 k.
  const int64_t rblk = rg * 4 + wave;                            // 16-row block
  const int64_t r = rblk * 16 + (lane & 15);                     // plane row (A row or B column)
  const int64_t k0 = kt * kTileK + (lane >> 4) * 16;             // first of 16 k
  const bool rowok = r < R;

  // A fragment that is all padding (its 16 rows or its 64 k past the
  // operand) only stores zeros: no loads and no residue arithmetic.
  const int P = a.P;
  const int64_t nkt = a.nkt;
  const int64_t rt = rblk >> 4, fr = rblk & 15;
  const int64_t plane = isA ? a.planeA : a.planeB;
  int8_t* base = (isA ? a.planesA : a.planesB) + b * (isA ? a.memberA : a.memberB);
  const int64_t off = (rt * nkt + kt) * kTileBytes + fr * kFragBytes + lane * 16;
  if (__builtin_amdgcn_readfirstlane((int)(rblk * 16 >= R || kt * kTileK >= K))) {
    const v4i z = v4i{0, 0, 0, 0};
    for (int pi = 0; pi < P; ++pi) *reinterpret_cast<v4i*>(base + pi * plane + off) = z;
    if (a.use_corr) {
      int8_t* cb = base + (int64_t)P * plane;
      const int64_t o1 = (rt * 2 * nkt + kt) * kTileBytes + fr * kFragBytes + lane * 16;
      *reinterpret_cast<v4i*>(cb + o1) = z;
      *reinterpret_cast<v4i*>(cb + o1 + nkt * kTileBytes) = z;
    }
    return;
  }

  double x[16];
  if (!rowok || k0 >= K) {
#pragma unroll
    for (int j = 0; j < 16; ++j) x[j] = 0.0;
  } else if (kn) {
    const double* __restrict__ src = a.B + (b * a.lda + a.k0 + k0) * a.N + r;
#pragma unroll
    for (int j = 0; j < 16; ++j) x[j] = (k0 + j < K) ? src[(int64_t)j * a.N] : 0.0;
  } else {
    const double* __restrict__ src = (isA ? a.A : a.B) + (b * R + r) * a.lda + a.k0 + k0;
    if (k0 + 16 <= K) {
#pragma unroll
      for (int j = 0; j < 16; ++j) x[j] = src[j];
    } else {
#pragma unroll
      for (int j = 0; j < 16; ++j) x[j] = (k0 + j < K) ? src[j] : 0.0;
    }
  }

  // Shift: per row of A / of B [N,K]; per column of B [K,N] -- one per lane.
  // Read after the operand loads are issued, so one round trip covers both.
  const int16_t* sfts = isA ? a.sftA : a.sftB;
  const int be = a.pick ? pick_be : a.bits_eff[0];
  const int shift = rowok ? (int)sfts[b * R + r] + (a.pick ? pick_be - a.bits : a.bits_eff[1]) : 0;

  // Split every element first: th, tl as exact doubles, hi7/q7 bytes.  All
  // scalings are by powers of two and exact: y = |x| 2^shift (< 2^be, or
  // rounds to a subnormal far below 1/2, whose rounding is then 0 anyway),
  // Tu = RNE(y) is the integer-only RNE of the reference, d = y - Tu is exact
  // (|d| <= 1/2), and RNE(256 y) - 256 Tu = RNE(256 d) because 256 Tu is even,
  // so the tie parity is unchanged.  td = +-Tu (|td| <= 2^53) splits as
  // th 2^31 + tl with th = RNE(td / 2^31), |th| <= 2^22, and |tl| <= 2^30,
  // both exact int32s.
  int th[16], tl[16];
  uint32_t hw[4] = {0u, 0u, 0u, 0u}, qw[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int jj = 0; jj < 16; ++jj) {
    // Infinities and NaNs scale to 0, as the reference's integer split of
    // their encoding does (the shift that carries exponent 0x7FF is far past
    // 64 bits); every finite y is below 2^53.
    double y = ldexp(fabs(x[jj]), shift);
    y = y <= 0x1p54 ? y : 0.0;
    const double Tu = rint(y);
    const double td = copysign(Tu, x[jj]);
    if (a.use_corr) {
      const double h8 = rint(ldexp(Tu, 7 - be));
      const double r8 = rint(ldexp(y - Tu, 8));
      const bool neg = signbit(x[jj]);
      const int hs = (int)fmin(fmax(neg ? -h8 : h8, -127.0), 127.0);   // h8 >= 0
      const int qs = (int)fmin(fmax(neg ? -r8 : r8, -127.0), 127.0);   // r8 signed
      hw[jj >> 2] |= ((uint32_t)hs & 0xFFu) << (8 * (jj & 3));
      qw[jj >> 2] |= ((uint32_t)qs & 0xFFu) << (8 * (jj & 3));
    }
    const double hi = rint(ldexp(td, -31));
    th[jj] = (int)hi;
    tl[jj] = (int)fma(-hi, 2147483648.0, td);      // in [-2^30, 2^30]
  }

  // One plane at a time: 16 residues -> one 16-byte chunk per lane, 1 KiB
  // contiguous per wave.  v = th (2^31 mod p) + tl is an exact int32
  // (|v| <= 2^21 p + 2^30 < 2^31) congruent to td; its balanced residue
  // v - p RNE(v / p) lies in [-p/2, p/2] (for odd p the quotient v RN(1/p) is
  // at most 2^-30 off v / p, which never comes within 1/(2p) of a
  // half-integer; 1/256 is exact; for p = 256 a residue +128 has the byte of
  // -128).  For p >= 171 the quotient stays below 2^23 and the residue is
  // acc_residue's one fma and two 24-bit multiply-adds; smaller moduli (only
  // in a caller's own list) take the quotient in fp64.  Another even p turns
  // a tie's +p/2 into barrett_bal32's -p/2.  Each variant is its own copy
  // of the loop, so the usual moduli carry no extra compare.
  auto plane_residues = [&](auto int_path, auto tie_fix, int pi) {
    int pt, c31;
    double ip;
    if constexpr (kDefault) {
      pt = kDefaultTab.p[pi]; c31 = kDefaultTab.c31[pi]; ip = kDefaultTab.invp[pi];
    } else {
      pt = a.tab.p[pi]; c31 = a.tab.c31[pi]; ip = a.tab.invp[pi];
    }
    uint32_t w4[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      int r[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int v = __mul24(th[4 * g + u], c31) + tl[4 * g + u];
        if (decltype(int_path)::value) {
          r[u] = acc_residue(v, ip, -pt);
        } else {
          const double vd = (double)v;
          const double q = fma(vd, ip, kMagic) - kMagic;
          r[u] = (int)fma(-q, (double)pt, vd);
        }
        if (decltype(tie_fix)::value) r[u] = r[u] == (pt >> 1) ? -(pt >> 1) : r[u];
      }
      w4[g] = pack_bytes(r[0], r[1], r[2], r[3]);
    }
    *reinterpret_cast<v4i*>(base + pi * plane + off) =
        v4i{(int)w4[0], (int)w4[1], (int)w4[2], (int)w4[3]};
  };
  if constexpr (kDefault) {
    // Every default modulus is 256 or odd, and >= 171.
#pragma unroll
    for (int pi = 0; pi < kMaxP; ++pi)
      if (pi < P) plane_residues(std::true_type{}, std::false_type{}, pi);
  } else {
    for (int pi = 0; pi < P; ++pi) {
      const int pt = a.tab.p[pi];
      const bool tie = !(pt & 1) && pt != 256;
      if (pt >= 171) {
        if (!tie) plane_residues(std::true_type{}, std::false_type{}, pi);
        else plane_residues(std::true_type{}, std::true_type{}, pi);
      } else {
        if (!tie) plane_residues(std::false_type{}, std::false_type{}, pi);
        else plane_residues(std::false_type{}, std::true_type{}, pi);
      }
    }
  }
  if (a.use_corr) {
    // Correction plane: row tile stride 2*nkt tiles; A = [hi | q], B = [q | hi].
    int8_t* cb = base + (int64_t)P * plane;
    const int64_t o1 = (rt * 2 * nkt + kt) * kTileBytes + fr * kFragBytes + lane * 16;
    const int64_t o2 = o1 + nkt * kTileBytes;
    const v4i hv = v4i{(int)hw[0], (int)hw[1], (int)hw[2], (int)hw[3]};
    const v4i qv = v4i{(int)qw[0], (int)qw[1], (int)qw[2], (int)qw[3]};
    *reinterpret_cast<v4i*>(cb + o1) = isA ? hv : qv;
    *reinterpret_cast<v4i*>(cb + o2) = isA ? qv : hv;
  }
}

// ---------------------------------------------------------------------------
// Modular GEMM engine.  Work item = (slot, batch member, 256x256 output tile);
// slot = correction GEMM(s) first (they are twice as deep), then one slot per
// modulus (slot runs group a tile's slots; under one run per tile the fused
// correction slot leads the run).  Exact int32 C = A_plane B_plane^T per slot
// (fp64_emu_cuda/fp64_emu.cu:491-657); epilogue: balanced int8 residue for
// modulus slots (the reference's bal8, :613-620, here as an exact fp64
// nearest-quotient reduction), raw int32 for correction slots.
//
// 4 waves in a 2x2 arrangement, 128x128 per wave = 8x8 v_mfma_i32_16x16x64_i8
// tiles (256 accumulator registers; the 16x16 form draws less power per
// operation than 32x32x32, so under the power cap the clock runs higher).
// Operand tiles stream into a 4-stage LDS
// ring with direct global->LDS copies (prefetch distance 3 k-steps); the
// planes are stored in fragment order, so each stage is a linear copy and
// every fragment read is 16 contiguous bytes per lane (bank-conflict free).
// Fragments are double-buffered in registers: while the MFMAs of k-step kt
// run, the fragments of kt+1 are read, so LDS latency stays off the MFMA
// path.  One explicit wait + barrier per k-step.
//
// Output blocks (res8 / corr planes): 16 rows x 64 columns, row-block major;
// element 16 l + 4 q + v of a block (lane l, accumulator column block q,
// value v) is row 4 (l / 16) + v, column 16 q + l % 16: 16 consecutive bytes
// (int8) or int32 per lane.

struct GemmArgs {
  const int8_t* A;
  const int8_t* B;
  int8_t* res8;
  int32_t* corr;
  int32_t* racc;       // K-segmented: residue sums (instead of res8)
  int64_t* cacc;       // K-segmented: correction sum (instead of corr)
  int first;           // K-segmented: first segment stores, later ones add
  int64_t memberA, memberB, planeA, planeB;
  int64_t outplane;    // Mp * Np
  int64_t total;       // work groups
  int nkt;             // k tiles of a residue plane
  int TM, TN;          // output tiles per member (256 x 256, or 256 x 128 for the narrow kernel)
  int64_t NB;          // 64-column output blocks per output row: Np / 64
  int P, ncorr, nslots, batch;
  int ksplit;          // groups per output tile, each over a contiguous K range
  int run;             // residue slots per run group (1: one slot per group)
  int corr_run;        // 1: each tile's run starts with the (fused) correction slot
  int chain;           // item streams: items per work group
  int xcols;           // split streams: extra columns past the TN wide tile columns
  int p[kMaxP];
  double invp[kMaxP];
};


// s_waitcnt immediate (gfx9 encoding): wait until at most `vm` vector-memory
// operations of this wave are outstanding and all LDS operations are done.
template <int vm>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(vm >= 0 && vm < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((vm & 15) | (7 << 4) | (0 << 8) | ((vm >> 4) << 14));
}

// Work-group barrier without the release/acquire fences of __syncthreads(),
// whose release half drains every outstanding vector-memory operation
// (including the LDS prefetch ring).  Callers wait explicitly
// (wait_vm_lgkm0) before it; the empty asm statements keep the compiler from
// moving memory accesses across.
__device__ __forceinline__ void barrier_lds() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

typedef __attribute__((address_space(3))) int8_t lds_i8;

// Direct global->LDS copy of 16 bytes per lane: lane l's 16 bytes at g (its
// own address) + kOff land at l (the wave's LDS base) + kOff + 16 l.  The
// instruction's offset field is 13 bits, signed: the compiler encodes a
// larger offset wrapped into the field without moving the address or M0
// (4096 becomes -4096, so the copy reads 4 KiB before g: an out-of-bounds
// read that faulted the GPU in a probe), so every copy keeps its offset in
// [0, 4096) and larger steps advance the pointers instead.
template <int kOff>
__device__ __forceinline__ void copy_lds16(const int8_t* g, lds_i8* l) {
  static_assert(kOff >= 0 && kOff < 4096, "global_load_lds: offset outside its 13-bit field");
  __builtin_amdgcn_global_load_lds(g, l, 16, kOff, 0);
}

// One accumulator element read at its point of use.  With plain element
// reads the compiler copies all 256 accumulators to VGPRs at the loop exit,
// which overflows the VGPR file and spills; an AGPR operand keeps each value
// in place until its own read.
__device__ __forceinline__ int acc_read(int a) {
  int v;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return v;
}

// One v_mfma_i32_16x16x64_i8 accumulating in place.  Inline assembly ties
// the accumulator to the destination: through the builtin the compiler
// renamed the 64 accumulator quads between k-steps and copied them back
// (hundreds of v_accvgpr_mov per step).  The hardware chains MFMAs on one
// accumulator; the wait states a compiler would place around MFMAs it can
// see are placed by hand with mfma_fence where the accumulators are written
// or read by other instructions.
__device__ __forceinline__ void mma16(v4i& acc, const v4i& a, const v4i& b) {
  asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// The first k-step's form: the accumulator input is the constant 0, so no
// other instruction ever writes an accumulator an MFMA then reads.
__device__ __forceinline__ void mma16_init(v4i& acc, const v4i& a, const v4i& b) {
  asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, 0" : "=a"(acc) : "v"(a), "v"(b));
}

// acc += the dot product of the four int8 lanes of a and b, as inline
// assembly: as a plain builtin the compiler sank a step's dot products past
// the next barrier (pure arithmetic moves across the fences), bunching them
// ahead of that step's first MFMA; in assembly they keep their place among
// the MFMAs.
__device__ __forceinline__ void dot4_acc(int& acc, int a, int b) {
  asm volatile("v_dot4c_i32_i8 %0, %1, %2" : "+v"(acc) : "v"(a), "v"(b));
}

// 32 wait states, fenced against scheduling: more than any MFMA needs between
// its result and another instruction's read of it.
__device__ __forceinline__ void mfma_fence() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Three tile shapes (kWM x kWN fragments of 16 per wave, 2 x 2 waves):
// (8, 8): 256 x 256 output tiles, each wave 128 x 128 (8 x 8 accumulator
// quads, half the register file: one group per CU), a 4-stage ring of
// 32 KiB.  (8, 4): 256 x 128 tiles, each wave 128 x 64, a 3-stage ring of
// 24 KiB, two groups per CU: for shallow products, whose groups run only a
// few k-steps, one group's prologue and epilogue (operand latency, residue
// stores) overlap the other's MFMAs; and where 128 columns cover N with less
// padding.  (4, 4): 128 x 128 tiles, each wave 64 x 64, a 4-stage ring of
// 16 KiB, two groups per CU: products whose rows and columns both fit 128-wide
// tiles with less padding.  All copy stage kt + 3 during k-step kt.
template <int kWM, int kWN>
struct GemmShape {
  static constexpr int kS = (kWM == 8 && kWN == 4) ? 3 : 4;      // LDS ring stages
  static constexpr int kABytes = kWM * 2048;                      // A tile: 32 kWM rows x 64 k
  static constexpr int kBBytes = kWN * 2048;                      // B tile: 32 kWN columns x 64 k
  static constexpr int kSB = kABytes + kBBytes;                   // stage: A tile then B tile
  static constexpr int kDma = kWM / 2 + kWN / 2;                  // copies per wave per stage
  static constexpr int kHB = kWN / 4;                             // 64-column output blocks per wave
  static constexpr int kGroupsPerCU = (kWM == 8 && kWN == 8) ? 1 : 2;
  // The ring is the kernels' static LDS array: it must fit one CU's 160 KiB
  // for every group the shape puts there.  (No kernel of this library takes
  // dynamic LDS: a launch would need hipFuncAttributeMaxDynamicSharedMemorySize
  // set and checked above 64 KiB.)
  static constexpr int kLdsBytes = kS * kSB;
  static_assert(kLdsBytes * kGroupsPerCU <= 160 * 1024, "LDS ring exceeds the CU's 160 KiB");
};

// Work item of a group: XCD-aware order -- work group i runs on XCD i % 8;
// within each full chunk of 256 groups, XCD x takes logical items
// 32x .. 32x+31, an 8x4 block of tiles sharing 12 operand panels in that
// XCD's L2, while all XCDs work on the same slot (whose planes then stay
// resident in the MALL).
//
// With slot runs (g.run > 1, 256 x 256 tiles) the slot index counts the
// correction slots, then the runs of g.run residue slots of each tile (the
// last run of a tile shorter when g.run does not divide P): a group runs its
// run's slots back to back (nrun of them) on one stream of operand copies.
// With g.corr_run (one run of all P residue slots per tile, and the fused
// correction slot) each tile has one group, whose run starts with the
// correction slot.
struct GemmItem {
  int split, slot, nrun, mt, nt;
  int64_t b;
};

__device__ __forceinline__ GemmItem gemm_item(const GemmArgs& g) {
  const int64_t i = blockIdx.x;
  int64_t L = i;
  if ((i >> 8) < (g.total >> 8)) L = (i & ~255ll) + (i & 7) * 32 + ((i & 255) >> 3);
  const int64_t tiles = (int64_t)g.TM * g.TN;
  const int64_t sbs = L / tiles;                       // (slot, member, split)
  const int tile = (int)(L - sbs * tiles);
  GemmItem it;
  it.split = (int)(sbs % g.ksplit);
  const int64_t sb = sbs / g.ksplit;
  const int v = (int)(sb / g.batch);
  it.b = sb - (int64_t)v * g.batch;
  if (g.corr_run) {
    it.slot = 0;   // the correction slot, then every residue slot
    it.nrun = g.nslots;
  } else if (g.run > 1) {
    // Several runs per tile: the runs (the longest groups) first, the
    // correction slots after them, so that the short groups fill the last
    // round.
    const int nr = (g.P + g.run - 1) / g.run;
    if (v < nr) {
      it.slot = g.ncorr + v * g.run;
      it.nrun = min(g.run, g.nslots - it.slot);
    } else {
      it.slot = v - nr;
      it.nrun = 1;
    }
  } else if (v < g.ncorr) {
    it.slot = v;
    it.nrun = 1;
  } else {
    it.slot = g.ncorr + (v - g.ncorr) * g.run;
    it.nrun = min(g.run, g.nslots - it.slot);
  }
  // Grouped tile order: 8 row tiles per group, column-major inside.
  const int GM = 8;
  const int grp = tile / (GM * g.TN);
  const int first_m = grp * GM;
  const int gm = min(g.TM - first_m, GM);
  const int within = tile - grp * GM * g.TN;
  it.mt = first_m + within % gm;
  it.nt = within / gm;
  return it;
}

// Item streams (one slot per item, no K-split): work group gq runs the
// items q = 256 g.chain (gq / 256) + 256 j + gq % 256, j < g.chain (those
// below g.total).  Item q is the item that group q of the one-item-per-group
// launch takes (gemm_item), so the chip works through the items in the same
// order and XCD placement (group gq runs on XCD gq % 8, as group q would),
// and the hardware still balances the CUs, group by group.
__device__ __forceinline__ uint32_t stream_order(const GemmArgs& g, uint32_t q) {
  return (q >> 8) < (uint32_t)(g.total >> 8) ? (q & ~255u) + (q & 7) * 32 + ((q & 255) >> 3) : q;
}

__device__ __forceinline__ GemmItem stream_item(const GemmArgs& g, uint32_t L) {
  const uint32_t tiles = (uint32_t)(g.TM * g.TN);
  const uint32_t sb = L / tiles;                      // (slot, member)
  const uint32_t tile = L - sb * tiles;
  GemmItem it;
  it.split = 0;
  it.nrun = 1;
  it.slot = (int)(sb / (uint32_t)g.batch);
  it.b = sb - (uint32_t)it.slot * (uint32_t)g.batch;
  const uint32_t GM = 8, TM = (uint32_t)g.TM;
  const uint32_t grp = tile / (GM * (uint32_t)g.TN);
  const uint32_t first_m = grp * GM;
  const uint32_t gm = min(TM - first_m, GM);
  const uint32_t within = tile - grp * GM * (uint32_t)g.TN;
  it.mt = (int)(first_m + within % gm);
  it.nt = (int)(within / gm);
  return it;
}

// Balanced residues of one 16 x 64 output block of the accumulators (row
// block x, column block h of this wave's tile) to `dst` (16 bytes per lane),
// for slot runs.  Stage by stage over the block's 16 values, so that no
// dependent chain is exposed.
template <int kWM, int kWN>
__device__ __forceinline__ void store_residue_block(const v4i (&acc)[kWM][kWN], const int x, const int h,
                                                    const double ip, const int negp, int8_t* dst) {
  int av[16], qv[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) av[v] = acc_read(acc[x][4 * h + v / 4][v % 4]);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int v = 0; v < 16; ++v) qv[v] = __double2loint(fma((double)av[v], ip, kMagic));
  __builtin_amdgcn_sched_barrier(0);
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
    w[q] = pack_bytes(__mul24(qv[4 * q], negp) + av[4 * q], __mul24(qv[4 * q + 1], negp) + av[4 * q + 1],
                      __mul24(qv[4 * q + 2], negp) + av[4 * q + 2], __mul24(qv[4 * q + 3], negp) + av[4 * q + 3]);
  *reinterpret_cast<v4i*>(dst) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
}

// One output tile of one slot (kRun: of it.nrun consecutive residue slots):
// the body of the GEMM kernels, on the group's LDS ring `lds` (the kernel's
// single LDS object).  kStream: an item stream; with kSplitS, a split stream,
// with kXc > 0 computing the kXc extra columns beside the last wide tiles.
template <bool kDeep, int kWM, int kWN, bool kRun = false, bool kStream = false,
          bool kSplitS = false, int kXc = 0>
__device__ __forceinline__ void modgemm_tile(const GemmArgs& g, int8_t* lds, const GemmItem it) {
  using Sh = GemmShape<kWM, kWN>;
  constexpr int kSB = Sh::kSB, kDma = Sh::kDma, kHB = Sh::kHB;
  // LDS ring stages and the prefetch distance: stage kt + kPF is copied
  // during k-step kt, into the ring slot of a stage whose fragments every
  // wave has read (a step earlier; the step's wait and barrier retire those
  // reads), so kPF may be as large as kS.  (A five-stage ring with four
  // stages in flight measured no faster on shallow products, whose planes
  // come from HBM.)
  constexpr int kS = Sh::kS, kPF = 3;
  constexpr int kAB = Sh::kABytes;
  const int split = it.split, slot = it.slot, mt = it.mt, nt = it.nt;
  const int64_t b = it.b;

  // Slot -> operand plane, k-tile window and output.
  const bool is_corr = slot < g.ncorr;
  const int plane = is_corr ? g.P : slot - g.ncorr;
  const int rstride = is_corr ? 2 * g.nkt : g.nkt;           // k tiles per row tile
  const int ktot = is_corr ? (g.ncorr == 1 ? 2 * g.nkt : g.nkt) : g.nkt;
  const int klen = (ktot + g.ksplit - 1) / g.ksplit;
  const int kbeg = split * klen;
  // This group's k-steps; 0 for a trailing split past the end (it stores zeros).
  const int nk = max(0, min(klen, ktot - kbeg));
  const int kt0 = ((is_corr && g.ncorr == 2) ? slot * g.nkt : 0) + kbeg;

  // A 128-row (or 128-column) tile is one half (8 fragments) of a 256-row
  // plane tile.
  const int mrt = kWM == 8 ? mt : mt >> 1;
  const int mhalf = kWM == 8 ? 0 : mt & 1;
  const int8_t* At = g.A + b * g.memberA + (int64_t)plane * g.planeA +
                     ((int64_t)mrt * rstride + kt0) * kTileBytes + mhalf * kAB;
  const int nrt = kWN == 8 ? nt : nt >> 1;
  const int nhalf = kWN == 8 ? 0 : nt & 1;
  const int8_t* Bt = g.B + b * g.memberB + (int64_t)plane * g.planeB +
                     ((int64_t)nrt * rstride + kt0) * kTileBytes + nhalf * Sh::kBBytes;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // Each wave copies kWM/2 fragments of the A tile and kWN/2 of the B tile
  // (blocks of 4 or 2 KiB): the instruction offset advances the global and
  // the LDS address alike.
  const uint32_t goff = (uint32_t)(wave * (kWM / 2) * 1024 + lane * 16);
  const uint32_t goffB = (uint32_t)(wave * (kWN / 2) * 1024 + lane * 16);
  // kRun, kStream: the source tiles of the stage being copied, set before its
  // copies (the k-step stream crosses from one slot's planes, or one item's
  // tiles, to the next).
  const int8_t* cpA = At;
  const int8_t* cpB = Bt;
  // Extra columns (kXc > 0, split streams): a product whose last tile column
  // holds at most kXMax columns computes them beside its wide tiles, as VALU
  // dot products over the A fragments a wide tile holds anyway: for each
  // (slot, member, row tile), the unit in tile column (slot-member index mod
  // TN) carries them, so that the carriers rotate over the tile columns and
  // the XCD's groups.  A carrier's waves load the columns' bytes of each
  // k-step straight from B's plane (the first 16 rows of its last tile, the
  // 16 bytes of each column for the lane's k group) two steps ahead, into the
  // buffer XR_F0 or XR_F1 that pairs with the step's fragment buffer (so the
  // buffer of a step is the one its own load filled two steps before); xsrc
  // is that fragment at the piece's first step xg0, xg_last the piece's last
  // step (loads past it reread it).  xon marks a carrier's piece, xacc the
  // partial sums of the wave's rows (the wn = 0 wave its first four 16-row
  // fragments, the wn = 1 wave its last four), summed over the lanes' four k
  // groups at the piece's end.
  // kXon: 1 + the first of the four fragments the k-steps being compiled take
  // (0: none) -- blocks of the split branch redeclare it, so that their steps
  // carry the dot products unconditionally and other steps none.  (The dot
  // products of a k-step sit after its last MFMAs, while those drain: placed
  // between the MFMAs they delayed them, and the whole call, more.)
  bool xon = false;
  constexpr int kXon = 0;
  const int8_t* xsrc = nullptr;
  int xg0 = 0, xg_last = 0;
  v4i XR_F0[kXc > 0 ? kXc : 1], XR_F1[kXc > 0 ? kXc : 1];
  int xacc[kWM][kXc > 0 ? kXc : 1];
#define FP64EMU_SLOT(kt) ((kS == 4) ? ((kt) & 3) : ((kt) % kS))
  // The extra columns' bytes of stream step G into buffer XB.
#define FP64EMU_XLOAD(XB, G)                                                                \
  do {                                                                                      \
    if constexpr (kXc > 0 && kXon > 0) {                                                    \
      const int8_t* xp_ = xsrc + (int64_t)(min((G), xg_last) - xg0) * kTileBytes +          \
                          (lane >> 4) * 256;                                                \
      _Pragma("unroll") for (int ci_ = 0; ci_ < kXc; ++ci_)                                 \
        XB[ci_] = *reinterpret_cast<const v4i*>(xp_ + ci_ * 16);                            \
    }                                                                                       \
  } while (0)
  // The extra columns' dot products of A fragment x_ at dword d_ (XB: the
  // step's X buffer).
#define FP64EMU_XDOT(FC, XB, x_, d_)                                                         \
  do {                                                                                      \
    if constexpr (kXc > 0) {                                                                \
      _Pragma("unroll") for (int ci_ = 0; ci_ < kXc; ++ci_)                                 \
        dot4_acc(xacc[x_][ci_], FC[x_][d_], XB[ci_][d_]);                                   \
    }                                                                                       \
  } while (0)
#define FP64EMU_COPY_A(kt, j)                                                               \
  copy_lds16<(j) * 1024>((kRun || kStream ? cpA : At + (int64_t)(kt) * kTileBytes) + goff,   \
                         (lds_i8*)(lds + FP64EMU_SLOT(kt) * kSB + wave * (kWM / 2) * 1024))
#define FP64EMU_COPY_B(kt, j)                                                               \
  copy_lds16<(j) * 1024>((kRun || kStream ? cpB : Bt + (int64_t)(kt) * kTileBytes) + goffB,  \
                         (lds_i8*)(lds + FP64EMU_SLOT(kt) * kSB + kAB + wave * (kWN / 2) * 1024))
#define FP64EMU_ISSUE(kt)                                                              \
  do {                                                                                 \
    FP64EMU_COPY_A(kt, 0);                                                             \
    FP64EMU_COPY_A(kt, 1);                                                             \
    if constexpr (kWM == 8) {                                                          \
      FP64EMU_COPY_A(kt, 2);                                                           \
      FP64EMU_COPY_A(kt, 3);                                                           \
    }                                                                                  \
    FP64EMU_COPY_B(kt, 0);                                                             \
    FP64EMU_COPY_B(kt, 1);                                                             \
    if constexpr (kWN == 8) {                                                          \
      FP64EMU_COPY_B(kt, 2);                                                           \
      FP64EMU_COPY_B(kt, 3);                                                           \
    }                                                                                  \
  } while (0)
  // Fragments of one k-step: F[0..kWM) = A row blocks kWM wm .. kWM wm +
  // kWM - 1 (16 rows x 64 k each), F[kWM..kWM+kWN) = B column blocks kWN wn ..
  // kWN wn + kWN - 1.
#define FP64EMU_READF(F, kt)                                                               \
  do {                                                                                     \
    const v4i* sa_ = reinterpret_cast<const v4i*>(lds + FP64EMU_SLOT(kt) * kSB);          \
    const v4i* sb_ = sa_ + kAB / 16;                                                       \
    _Pragma("unroll") for (int y = 0; y < kWN; ++y) F[kWM + y] = sb_[(wn * kWN + y) * 64 + lane]; \
    _Pragma("unroll") for (int x = 0; x < kWM; ++x) F[x] = sa_[(wm * kWM + x) * 64 + lane]; \
  } while (0)
#define FP64EMU_MMA(F, MMA)                                                                 \
  do {                                                                                      \
    _Pragma("unroll") for (int x = 0; x < kWM; ++x)                                         \
    _Pragma("unroll") for (int y = 0; y < kWN; ++y) MMA(acc[x][y], F[x], F[kWM + y]);       \
  } while (0)
  // One k-step: stage kt+1 must have landed (own copies: at most one later
  // group in flight), then the barrier makes every wave's copies visible
  // and guarantees every wave finished reading the stage refilled next.
#define FP64EMU_STEP(kt, FC, FN, MMA)                                                    \
  do {                                                                                   \
    if ((kt) + kPF <= nk) wait_vm_lgkm0<(kPF - 2) * kDma>(); else wait_vm_lgkm0<0>();     \
    FP64EMU_STEP_BODY(kt, FC, FN, MMA);                                                  \
  } while (0)
#define FP64EMU_STEP_BODY(kt, FC, FN, MMA)                                               \
  do {                                                                                   \
    barrier_lds();                                                                       \
    if ((kt) + kPF < nk) FP64EMU_ISSUE((kt) + kPF);                                      \
    FP64EMU_READF(FN, (kt) + 1);                                                         \
    FP64EMU_MMA(FC, MMA);                                                                \
    if constexpr (kXc > 0 && kXon > 0) {                                                 \
      _Pragma("unroll") for (int d_ = 0; d_ < 4; ++d_)                                   \
      _Pragma("unroll") for (int x_ = 0; x_ < 4; ++x_)                                   \
        FP64EMU_XDOT(FC, XR_##FC, kXon - 1 + x_, d_);                                    \
      FP64EMU_XLOAD(XR_##FC, (kt) + 2);                                                  \
    }                                                                                    \
  } while (0)
  // Steady-state step (a copy for step kt+3 exists): an unconditional wait,
  // so the compiler's own wait tracking sees every earlier fragment read
  // retired (a conditional wait made it stall on the first read of each
  // step), and the step in four fenced chunks, each 4 times {one fragment
  // read, 4 MFMAs} with a copy before the first and the third: the copies
  // reach the texture unit spread over the step instead of as a burst after
  // the barrier, which delayed the last wave's MFMAs and made every wave wait
  // for it at the next barrier, and each read has 4 MFMAs to land behind.
  // The MFMAs of a k-step walk the kWM x kWN accumulator grid as a serpentine
  // (B blocks ascending along one A block, descending along the next), so
  // consecutive MFMAs change one operand, never both (c2 -0.3%, c3a -0.9%:
  // fewer operand bits toggle, and the chip runs at its power cap).
  // Chunk c: MFMAs of A blocks 2c, 2c+1 against all 8 B blocks; reads of the
  // next step's fragments 4c .. 4c+3 (B 0..7, then A 0..7), so the first
  // chunk of the next step finds its operands read a step ahead.
  // (kWN = 4: three reads and eight MFMAs per chunk -- B 0..3 then A 0..7 --
  // and the six copies spread as A 0, 1 | A 2 | A 3, B 0 | B 1.)
#define FP64EMU_CHUNK(kt, FC, FN, c, MMA)                                                    \
  do {                                                                                       \
    if constexpr (kWM == 4) FP64EMU_CHUNK_S(kt, FC, FN, c, MMA);                             \
    else if constexpr (kWN == 4) FP64EMU_CHUNK_N(kt, FC, FN, c, MMA);                        \
    else FP64EMU_CHUNK_W(kt, FC, FN, c, MMA);                                                \
  } while (0)
#define FP64EMU_CHUNK_W(kt, FC, FN, c, MMA)                                                  \
  do {                                                                                       \
    const v4i* sa_ = reinterpret_cast<const v4i*>(lds + FP64EMU_SLOT((kt) + 1) * kSB);      \
    const v4i* sb_ = sa_ + kTileBytes / 16;                                                  \
    _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                          \
      if (j == 0 && ((c) >> 1) == 0) FP64EMU_COPY_A((kt) + kPF, ((c) & 1) * 2);                \
      if (j == 2 && ((c) >> 1) == 0) FP64EMU_COPY_A((kt) + kPF, ((c) & 1) * 2 + 1);            \
      if (j == 0 && ((c) >> 1) == 1) FP64EMU_COPY_B((kt) + kPF, ((c) & 1) * 2);                \
      if (j == 2 && ((c) >> 1) == 1) FP64EMU_COPY_B((kt) + kPF, ((c) & 1) * 2 + 1);            \
      __builtin_amdgcn_sched_barrier(0);                                                     \
      const int f_ = (c) * 4 + j;                                                            \
      if (f_ < 8) FN[8 + f_] = sb_[(wn * 8 + f_) * 64 + lane];                               \
      else FN[f_ - 8] = sa_[(wm * 8 + f_ - 8) * 64 + lane];                                  \
      __builtin_amdgcn_sched_barrier(0);                                                     \
      _Pragma("unroll") for (int u = 0; u < 4; ++u) {                                        \
        const int m_ = 4 * j + u, x = (c) * 2 + m_ / 8, y = (m_ < 8) ? m_ : 15 - m_;           \
        MMA(acc[x][y], FC[x], FC[8 + y]);                                                    \
      }                                                                                      \
      if constexpr (kXc > 0 && kXon > 0) {                                                   \
        if ((c) == 3 && j == 3) {                                                            \
          _Pragma("unroll") for (int d_ = 0; d_ < 4; ++d_)                                   \
          _Pragma("unroll") for (int x_ = 0; x_ < 4; ++x_)                                   \
            FP64EMU_XDOT(FC, XR_##FC, kXon - 1 + x_, d_);                                    \
          FP64EMU_XLOAD(XR_##FC, (kt) + 2);                                                  \
        }                                                                                    \
      }                                                                                      \
      __builtin_amdgcn_sched_barrier(0);                                                     \
    }                                                                                        \
  } while (0)
#define FP64EMU_CHUNK_N(kt, FC, FN, c, MMA)                                                  \
  do {                                                                                       \
    const v4i* sa_ = reinterpret_cast<const v4i*>(lds + FP64EMU_SLOT((kt) + 1) * kSB);      \
    const v4i* sb_ = sa_ + kTileBytes / 16;                                                  \
    _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                          \
      if (j == 0 && (c) <= 1) FP64EMU_COPY_A((kt) + kPF, (c) <= 1 ? (c) * 2 : 0);              \
      if (j == 2 && (c) == 0) FP64EMU_COPY_A((kt) + kPF, 1);                                   \
      if (j == 0 && (c) == 2) FP64EMU_COPY_A((kt) + kPF, 3);                                   \
      if (j == 2 && (c) == 2) FP64EMU_COPY_B((kt) + kPF, 0);                                   \
      if (j == 0 && (c) == 3) FP64EMU_COPY_B((kt) + kPF, 1);                                   \
      __builtin_amdgcn_sched_barrier(0);                                                     \
      if (j < 3) {                                                                           \
        const int f_ = (c) * 3 + j;                                                          \
        if (f_ < 4) FN[8 + f_] = sb_[(wn * 4 + f_) * 64 + lane];                             \
        else FN[f_ - 4] = sa_[(wm * 8 + f_ - 4) * 64 + lane];                                \
      }                                                                                      \
      __builtin_amdgcn_sched_barrier(0);                                                     \
      _Pragma("unroll") for (int u = 0; u < 2; ++u) {                                        \
        const int m_ = 2 * j + u, x = (c) * 2 + m_ / 4, y = (m_ < 4) ? m_ : 7 - m_;            \
        MMA(acc[x][y], FC[x], FC[8 + y]);                                                    \
      }                                                                                      \
      __builtin_amdgcn_sched_barrier(0);                                                     \
    }                                                                                        \
  } while (0)
  // (4, 4): chunk c runs A block c against B 0..3 (four MFMAs) with two reads
  // of the next step's fragments (B 0, 1 | B 2, 3 | A 0, 1 | A 2, 3) and one
  // copy (A 0 | A 1 | B 0 | B 1).
#define FP64EMU_CHUNK_S(kt, FC, FN, c, MMA)                                                  \
  do {                                                                                       \
    const v4i* sa_ = reinterpret_cast<const v4i*>(lds + FP64EMU_SLOT((kt) + 1) * kSB);      \
    const v4i* sb_ = sa_ + kAB / 16;                                                         \
    if constexpr ((c) <= 1) FP64EMU_COPY_A((kt) + kPF, (c));                                   \
    else FP64EMU_COPY_B((kt) + kPF, (c) - 2);                                                  \
    _Pragma("unroll") for (int j = 0; j < 2; ++j) {                                          \
      __builtin_amdgcn_sched_barrier(0);                                                     \
      const int f_ = (c) * 2 + j;                                                            \
      if (f_ < 4) FN[4 + f_] = sb_[(wn * 4 + f_) * 64 + lane];                               \
      else FN[f_ - 4] = sa_[(wm * 4 + f_ - 4) * 64 + lane];                                  \
      __builtin_amdgcn_sched_barrier(0);                                                     \
      _Pragma("unroll") for (int u = 0; u < 2; ++u) {                                       \
        const int y_ = ((c) & 1) ? 3 - (2 * j + u) : 2 * j + u;                             \
        MMA(acc[(c)][y_], FC[(c)], FC[4 + y_]);                                              \
      }                                                                                      \
      __builtin_amdgcn_sched_barrier(0);                                                     \
    }                                                                                        \
  } while (0)
#define FP64EMU_STEP_FULL(kt, FC, FN, MMA)                                                   \
  do {                                                                                       \
    wait_vm_lgkm0<(kPF - 2) * kDma>();                                                       \
    barrier_lds();                                                                           \
    FP64EMU_CHUNK(kt, FC, FN, 0, MMA);                                                       \
    FP64EMU_CHUNK(kt, FC, FN, 1, MMA);                                                       \
    FP64EMU_CHUNK(kt, FC, FN, 2, MMA);                                                       \
    FP64EMU_CHUNK(kt, FC, FN, 3, MMA);                                                       \
  } while (0)

  v4i acc[kWM][kWN];
  // Outputs are blocks of 16 rows x 64 columns; this wave's 16 kWM x 16 kWN
  // holds kWM row blocks x kWN/4 column blocks.  Element 16 l + 4 q + v of a
  // block is lane l's value v of accumulator column block q (row
  // 4 (l / 16) + v, column 16 q + l % 16).
  // Streams (kRun, kStream): k-step G of the group's stream of nk k-steps,
  // whose copy (stage G + kPF) exists while G + kPF < nk; next_src() sets the
  // copy sources of the next stage.
#define FP64EMU_RSTEP(G, FC, FN, MMA)                                                       \
  do {                                                                                      \
    if ((G) + kPF < nk) next_src();                                                         \
    FP64EMU_STEP(G, FC, FN, MMA);                                                           \
  } while (0)
#define FP64EMU_RSTEP_FULL(G, FC, FN)                                                       \
  do {                                                                                      \
    next_src();                                                                             \
    FP64EMU_STEP_FULL(G, FC, FN, mma16);                                                    \
  } while (0)
  // The first k-step G0 of a slot (or item) leaves the previous one's stores
  // in flight: the stage it waits for (G0 + 1) was copied at step G0 - 2, and
  // the copies of stage G0 + 2 (step G0 - 1) and then the stores were issued
  // after it, so at most kRelax younger operations outstanding proves that
  // it landed, by the in-order retirement below; the stores retire during
  // that step instead of stalling its start.  (A correction slot stores four
  // times as many: a larger margin.  A stream's first slot follows the
  // prologue, which waited for everything.)
  constexpr int kRelax = (kPF - 2) * kDma + kWM * kHB;
  static_assert(kRelax < 64, "vmcnt field");
#define FP64EMU_RSTEP_R(G, FC, FN, MMA)                                                     \
  do {                                                                                      \
    if ((G) + kPF < nk) next_src();                                                         \
    if ((G) + kPF <= nk) wait_vm_lgkm0<kRelax>(); else wait_vm_lgkm0<0>();                  \
    FP64EMU_STEP_BODY(G, FC, FN, MMA);                                                      \
  } while (0)
  // One slot (or item) of a stream: k-steps G0 .. G0 + nj - 1, its first
  // stage landed and visible (the wait and barrier of the stream's previous
  // step, or the prologue's), no copy targeting it before its first step.
#define FP64EMU_STREAM_SLOT(G0, nj)                                                         \
  do {                                                                                      \
    v4i F0[kWM + kWN], F1[kWM + kWN];                                                       \
    FP64EMU_READF(F0, (G0));                                                                \
    if constexpr (kXc > 0 && kXon > 0) {                                                    \
      FP64EMU_XLOAD(XR_F0, (G0));                                                           \
      FP64EMU_XLOAD(XR_F1, (G0) + 1);                                                       \
      _Pragma("unroll") for (int x_ = 0; x_ < 4; ++x_)                                      \
      _Pragma("unroll") for (int ci_ = 0; ci_ < kXc; ++ci_) xacc[kXon - 1 + x_][ci_] = 0;   \
    }                                                                                       \
    FP64EMU_RSTEP_R((G0), F0, F1, mma16_init);                                              \
    int kt_ = 1;                                                                            \
    const int kf_ = nk - kPF - (G0);   /* steps kt_ < kf_ copy stage G0 + kt_ + kPF */      \
    for (; kt_ + 2 <= (nj) && kt_ + 1 < kf_; kt_ += 2) {                                    \
      FP64EMU_RSTEP_FULL((G0) + kt_, F1, F0);                                               \
      FP64EMU_RSTEP_FULL((G0) + kt_ + 1, F0, F1);                                           \
    }                                                                                       \
    for (; kt_ + 2 <= (nj); kt_ += 2) {                                                     \
      FP64EMU_RSTEP((G0) + kt_, F1, F0, mma16);                                             \
      FP64EMU_RSTEP((G0) + kt_ + 1, F0, F1, mma16);                                         \
    }                                                                                       \
    if (kt_ < (nj)) FP64EMU_RSTEP((G0) + kt_, F1, F0, mma16);                               \
    mfma_fence();                                                                           \
  } while (0)
  if constexpr (kRun) {
    const int64_t NB = g.NB;
    const int64_t rb0 = (int64_t)mt * (2 * kWM) + wm * kWM, cb0 = (int64_t)nt * (kWN / 2) + wn * kHB;
    // Residue slots slot .. slot + nrun - 1 (planes one stride apart, nk
    // k-steps each) as one stream of nrun nk k-steps: the copies run ahead
    // across slot boundaries, so only the first slot waits for its operands;
    // each slot's first k-step starts the accumulators and its last one is
    // followed by that slot's residue stores.  The stores count in the same
    // vector-memory counter as the copies, and the first k-step after them
    // waits for the counter to fall to kDma: that proves the stage it needs
    // (issued before the stores) has landed because gfx9-family counters
    // retire vector-memory operations in issue order (CDNA3 ISA, "Data
    // dependency resolution": reads and writes return in the order issued),
    // so the count reaches kDma only after every operation older than the
    // last kDma -- the stage and everything before it.
    // A run that starts with the correction slot (g.corr_run) streams its
    // 2 nkt k-steps first, from the correction plane (At, Bt: row-tile stride
    // 2 nkt; A = [hi | q], B = [q | hi], so the two halves accumulate
    // without a store between them), then the residue slots from plane 0.
    const bool crun = is_corr;
    const int nks = crun ? g.nkt : nk;       // k-steps of a residue slot
    const int nkc = crun ? 2 * g.nkt : 0;    // k-steps of the correction slot
    const int8_t* ArA = crun ? g.A + b * g.memberA + (int64_t)mrt * g.nkt * kTileBytes : At;
    const int8_t* ArB = crun ? g.B + b * g.memberB + (int64_t)nrt * g.nkt * kTileBytes : Bt;
    const int nkr = nkc + (it.nrun - (crun ? 1 : 0)) * nks;
    // The copy side: the next stage's sources nA, nB, in residue slot cj of
    // the run (-1: the correction slot), cleft stages left in that slot.
    // The step advances two pointers; a slot crossing (rare) moves them to
    // the next plane.
    int cj = crun ? -1 : 0, cleft = crun ? nkc : nks;
    const int8_t* nA = crun ? At : ArA;
    const int8_t* nB = crun ? Bt : ArB;
    auto next_src = [&]() {
      cpA = nA;
      cpB = nB;
      nA += kTileBytes;
      nB += kTileBytes;
      if (__builtin_expect(--cleft == 0, 0)) {
        ++cj;
        nA = ArA + (int64_t)cj * g.planeA;
        nB = ArB + (int64_t)cj * g.planeB;
        cleft = nks;
      }
    };
    auto store_corr = [&]() {
      int32_t* cdst = g.corr + (b * g.ncorr) * g.outplane;
#pragma unroll
      for (int x = 0; x < kWM; ++x)
#pragma unroll
        for (int h = 0; h < kHB; ++h) {
          v4i* d = reinterpret_cast<v4i*>(cdst + ((rb0 + x) * NB + cb0 + h) * 1024 + lane * 16);
#pragma unroll
          for (int q = 0; q < 4; ++q)
            d[q] = v4i{acc_read(acc[x][4 * h + q][0]), acc_read(acc[x][4 * h + q][1]),
                       acc_read(acc[x][4 * h + q][2]), acc_read(acc[x][4 * h + q][3])};
          __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto store_slot = [&](const int s_) {
      const int t = s_ - g.ncorr;
      const double ip = g.invp[t];
      const int negp = -g.p[t];
      int8_t* rdst = g.res8 + (b * g.P + t) * g.outplane;
#pragma unroll
      for (int x = 0; x < kWM; ++x)
#pragma unroll
        for (int h = 0; h < kHB; ++h) {
          store_residue_block<kWM, kWN>(acc, x, h, ip, negp,
                                        rdst + ((rb0 + x) * NB + cb0 + h) * 1024 + lane * 16);
          __builtin_amdgcn_sched_barrier(0);
        }
    };
    {
      const int nk = nkr;   // the STEP macros' end of stream
#pragma unroll
      for (int s = 0; s < kPF; ++s)
        if (s < nk) { next_src(); FP64EMU_ISSUE(s); }
      wait_vm_lgkm0<0>();
      barrier_lds();
      for (int j = 0; j < it.nrun; ++j) {
        // Slot j of the run.
        const bool jc = crun && j == 0;
        const int nj = jc ? nkc : nks;
        const int G0 = jc ? 0 : nkc + (j - (crun ? 1 : 0)) * nks;
        FP64EMU_STREAM_SLOT(G0, nj);
        if (jc) store_corr();
        else store_slot(slot + j);
      }
      // No copy or store may still be in flight when the group retires.
      wait_vm_lgkm0<0>();
    }
  } else if constexpr (kSplitS) {
    // Split stream (use_split_streams): one group per CU, group j = blockIdx.x
    // / 8 of XCD x = blockIdx.x % 8.  The g.total units (stream_item order) form
    // nblk blocks of 32 of g.nkt k-steps each; XCD x's share is block-steps
    // [x Tb / 8, (x + 1) Tb / 8) of the Tb = nblk g.nkt, and group j runs
    // unit 32 bl + j of each block bl in it, the pieces (one block's k range
    // each) as one stream of k-steps whose copies run ahead across pieces.
    // A piece starting at k-step 0 stores its sums as split 0, else as split
    // 1; a piece covering its unit whole also stores zeros as split 1.
    const int x = (int)(blockIdx.x & 7u);
    const uint32_t jl = blockIdx.x >> 3;
    // Extra columns: the unit in tile column nt of slot-member sb carries them.
    auto x_carrier = [&](const int nt_, const uint32_t sb_) {
      return nt_ == (int)(sb_ % (uint32_t)g.TN);
    };
    const uint32_t U = (uint32_t)g.total;
    const uint32_t nblk = (U + 31u) >> 5;
    const int64_t Tb = (int64_t)nblk * g.nkt;
    const int64_t s0 = (int64_t)x * Tb / 8;
    int64_t e0 = (int64_t)(x + 1) * Tb / 8;
    // The last block holds U - 32 (nblk - 1) units: later groups stop before it.
    if (jl >= U - 32u * (nblk - 1u)) e0 = min(e0, (int64_t)(nblk - 1u) * g.nkt);
    if (s0 >= e0) return;
    const int nk = (int)(e0 - s0);
    const uint32_t bfirst = (uint32_t)(s0 / g.nkt);          // the first piece's block
    const int kfirst = (int)(s0 - (int64_t)bfirst * g.nkt);  // and its first k-step
    uint32_t cbl = bfirst;                                   // block of the copy side's piece
    // The copy side: the next stage's sources nA, nB, cleft stages left in
    // the piece; a piece crossing moves to k-step 0 of the next block's unit.
    int cleft = 0;
    const int8_t* nA = nullptr;
    const int8_t* nB = nullptr;
    int64_t cend = e0 - (int64_t)cbl * g.nkt;               // stream end, from the piece's block
    auto copy_piece = [&](const int k) {
      const GemmItem t = stream_item(g, cbl * 32u + jl);
      const bool ic = t.slot < g.ncorr;                     // ncorr is 2 (or 0) here
      const int pl = ic ? g.P : t.slot - g.ncorr;
      const int rs = ic ? 2 * g.nkt : g.nkt;                // k tiles per row tile
      const int k0 = (ic ? t.slot * g.nkt : 0) + k;
      nA = g.A + t.b * g.memberA + (int64_t)pl * g.planeA + ((int64_t)t.mt * rs + k0) * kTileBytes;
      nB = g.B + t.b * g.memberB + (int64_t)pl * g.planeB + ((int64_t)t.nt * rs + k0) * kTileBytes;
      cleft = (int)min<int64_t>(g.nkt, cend) - k;
    };
    copy_piece(kfirst);
    auto next_src = [&]() {
      cpA = nA;
      cpB = nB;
      nA += kTileBytes;
      nB += kTileBytes;
      if (__builtin_expect(--cleft == 0, 0) && cend > g.nkt) {
        ++cbl;
        cend -= g.nkt;
        copy_piece(0);
      }
    };
    const int64_t NB = g.NB;
#pragma unroll
    for (int s = 0; s < kPF; ++s)
      if (s < nk) { next_src(); FP64EMU_ISSUE(s); }
    wait_vm_lgkm0<0>();
    barrier_lds();
    int G0 = 0;
    uint32_t bl = bfirst;
    int k0 = kfirst;
    while (G0 < nk) {
      const int nj = min(g.nkt - k0, nk - G0);
      const GemmItem t = stream_item(g, bl * 32u + jl);
      // A carrier of the extra columns: this wave's fragments 4 wn .. 4 wn + 3,
      // their bytes from B's tile g.TN of the unit's plane at the piece's k.
      xon = kXc > 0 && x_carrier(t.nt, (bl * 32u + jl) / (uint32_t)(g.TM * g.TN));
      if (kXc > 0 && xon) {
        const bool ic = t.slot < g.ncorr;
        const int pl = ic ? g.P : t.slot - g.ncorr;
        const int rs = ic ? 2 * g.nkt : g.nkt;
        const int kx = (ic ? t.slot * g.nkt : 0) + k0;
        xsrc = g.B + t.b * g.memberB + (int64_t)pl * g.planeB + ((int64_t)g.TN * rs + kx) * kTileBytes;
        xg0 = G0;
        xg_last = G0 + nj - 1;
      }
      if (kXc > 0 && xon && wn == 0) {
        constexpr int kXon = 1;
        FP64EMU_STREAM_SLOT(G0, nj);
      } else if (kXc > 0 && xon) {
        constexpr int kXon = 5;
        FP64EMU_STREAM_SLOT(G0, nj);
      } else {
        FP64EMU_STREAM_SLOT(G0, nj);
      }
      const bool whole = k0 == 0 && nj == g.nkt;
      const int64_t sbm = (int64_t)(k0 == 0 ? 0 : 1) * g.batch + t.b;   // split-major planes
      const int64_t rb0 = (int64_t)t.mt * (2 * kWM) + wm * kWM, cb0 = (int64_t)t.nt * (kWN / 2) + wn * kHB;
      // Extra columns: sums over the four k groups (lanes l, l ^ 16, l ^ 32,
      // l ^ 48 hold row l % 16's); lane r < 16 then stores row r of each
      // fragment, element 256 (r / 4) + 16 ci + r % 4 of the 16 x 64 output
      // block (column ci) in column block 4 g.TN.
      const int64_t cbX = (int64_t)g.TN * 4;
      const int xel = 256 * (lane >> 2) + (lane & 3);
      auto xsum = [&]() {
        if constexpr (kXc > 0) {
#pragma unroll
          for (int x_ = 0; x_ < kWM; ++x_)
#pragma unroll
            for (int ci_ = 0; ci_ < kXc; ++ci_) {
              if ((x_ >> 2) != wn) continue;   // the other wave's fragment
              int v = xacc[x_][ci_];
              v += __shfl_xor(v, 16);
              v += __shfl_xor(v, 32);
              xacc[x_][ci_] = v;
            }
        }
      };
      if (t.slot < g.ncorr) {
        int32_t* cdst = g.corr + (sbm * g.ncorr + t.slot) * g.outplane;
        const int64_t zoff = (int64_t)g.batch * g.ncorr * g.outplane;   // split 1, in int32s
#pragma unroll
        for (int x_ = 0; x_ < kWM; ++x_)
#pragma unroll
          for (int h = 0; h < kHB; ++h) {
            int32_t* c = cdst + ((rb0 + x_) * NB + cb0 + h) * 1024 + lane * 16;
            v4i* d = reinterpret_cast<v4i*>(c);
#pragma unroll
            for (int q = 0; q < 4; ++q)
              d[q] = v4i{acc_read(acc[x_][4 * h + q][0]), acc_read(acc[x_][4 * h + q][1]),
                         acc_read(acc[x_][4 * h + q][2]), acc_read(acc[x_][4 * h + q][3])};
            if (whole) {
              v4i* z = reinterpret_cast<v4i*>(c + zoff);
#pragma unroll
              for (int q = 0; q < 4; ++q) z[q] = v4i{0, 0, 0, 0};
            }
            __builtin_amdgcn_sched_barrier(0);
          }
        if constexpr (kXc > 0) {
          if (xon) {
            xsum();
            if (lane < 16) {
#pragma unroll
              for (int x_ = 0; x_ < kWM; ++x_)
#pragma unroll
                for (int ci_ = 0; ci_ < kXc; ++ci_) {
                  if ((x_ >> 2) != wn) continue;   // the other wave's fragment
                  int32_t* c = cdst + ((rb0 + x_) * NB + cbX) * 1024 + xel + 16 * ci_;
                  *c = xacc[x_][ci_];
                  if (whole) c[zoff] = 0;
                }
            }
          }
        }
      } else {
        const int tp = t.slot - g.ncorr;
        const double ip = g.invp[tp];
        const int negp = -g.p[tp];
        int8_t* rdst = g.res8 + (sbm * g.P + tp) * g.outplane;
        const int64_t zoff = (int64_t)g.batch * g.P * g.outplane;        // split 1
#pragma unroll
        for (int x_ = 0; x_ < kWM; ++x_)
#pragma unroll
          for (int h = 0; h < kHB; ++h) {
            int8_t* d = rdst + ((rb0 + x_) * NB + cb0 + h) * 1024 + lane * 16;
            store_residue_block<kWM, kWN>(acc, x_, h, ip, negp, d);
            if (whole) *reinterpret_cast<v4i*>(d + zoff) = v4i{0, 0, 0, 0};
            __builtin_amdgcn_sched_barrier(0);
          }
        if constexpr (kXc > 0) {
          if (xon) {
            xsum();
            if (lane < 16) {
#pragma unroll
              for (int x_ = 0; x_ < kWM; ++x_)
#pragma unroll
                for (int ci_ = 0; ci_ < kXc; ++ci_) {
                  if ((x_ >> 2) != wn) continue;   // the other wave's fragment
                  const int v = xacc[x_][ci_];
                  const int q = __double2loint(fma((double)v, ip, kMagic));
                  int8_t* d = rdst + ((rb0 + x_) * NB + cbX) * 1024 + xel + 16 * ci_;
                  *d = (int8_t)(__mul24(q, negp) + v);   // the balanced residue's byte
                  if (whole) d[zoff] = 0;
                }
            }
          }
        }
      }
      G0 += nj;
      ++bl;
      k0 = 0;
    }
    // No copy or store may still be in flight when the group retires.
    wait_vm_lgkm0<0>();
  } else if constexpr (kStream) {
    // Item stream (256 x 256 tiles, no K-split): the group runs its items
    // (stream_order, stream_item) as one stream of k-steps, the copies
    // running ahead across item boundaries as a run's do across slots, so
    // that an item's first stages land while the previous item ends and
    // stores its outputs, and no item waits on its own group's launch and
    // prologue.
    const uint32_t q0 = (blockIdx.x >> 8) * (uint32_t)(256 * g.chain) + (blockIdx.x & 255);
    if (q0 >= g.total) return;   // the last groups of a partial last round
    const int nitems = (int)min<int64_t>(g.chain, (g.total - q0 + 255) / 256);
    // Items below corr_end (in launch order) are correction slots: csteps
    // k-steps each (the fused pair: twice a residue slot's).
    const uint32_t corr_end = (uint32_t)(g.ncorr * g.batch) * (uint32_t)(g.TM * g.TN);
    const int csteps = g.ncorr == 1 ? 2 * g.nkt : g.nkt;
    int nk = 0;
    for (int j = 0; j < nitems; ++j)
      nk += stream_order(g, q0 + (uint32_t)j * 256) < corr_end ? csteps : g.nkt;
    // The copy side: the next stage's sources nA, nB, in item cj, cleft
    // stages left in that item.  The step advances two pointers; an item
    // crossing (rare) decodes the next item.
    int cj = 0, cleft = 0;
    const int8_t* nA = nullptr;
    const int8_t* nB = nullptr;
    auto copy_item = [&](const int j) {
      const GemmItem t = stream_item(g, stream_order(g, q0 + (uint32_t)j * 256));
      const bool ic = t.slot < g.ncorr;
      const int pl = ic ? g.P : t.slot - g.ncorr;
      const int rs = ic ? 2 * g.nkt : g.nkt;                       // k tiles per row tile
      const int k0 = (ic && g.ncorr == 2) ? t.slot * g.nkt : 0;
      nA = g.A + t.b * g.memberA + (int64_t)pl * g.planeA + ((int64_t)t.mt * rs + k0) * kTileBytes;
      nB = g.B + t.b * g.memberB + (int64_t)pl * g.planeB + ((int64_t)t.nt * rs + k0) * kTileBytes;
      cleft = ic ? csteps : g.nkt;
    };
    copy_item(0);
    auto next_src = [&]() {
      cpA = nA;
      cpB = nB;
      nA += kTileBytes;
      nB += kTileBytes;
      if (__builtin_expect(--cleft == 0, 0) && cj + 1 < nitems) copy_item(++cj);
    };
    const int64_t NB = g.NB;
#pragma unroll
    for (int s = 0; s < kPF; ++s)
      if (s < nk) { next_src(); FP64EMU_ISSUE(s); }
    wait_vm_lgkm0<0>();
    barrier_lds();
    int G0 = 0;
    for (int j = 0; j < nitems; ++j) {
      const GemmItem t = stream_item(g, stream_order(g, q0 + (uint32_t)j * 256));
      const bool ic = t.slot < g.ncorr;
      const int nj = ic ? csteps : g.nkt;
      FP64EMU_STREAM_SLOT(G0, nj);
      const int64_t rb0 = (int64_t)t.mt * (2 * kWM) + wm * kWM, cb0 = (int64_t)t.nt * (kWN / 2) + wn * kHB;
      if (ic) {
        int32_t* cdst = g.corr + (t.b * g.ncorr + t.slot) * g.outplane;
#pragma unroll
        for (int x = 0; x < kWM; ++x)
#pragma unroll
          for (int h = 0; h < kHB; ++h) {
            v4i* d = reinterpret_cast<v4i*>(cdst + ((rb0 + x) * NB + cb0 + h) * 1024 + lane * 16);
#pragma unroll
            for (int q = 0; q < 4; ++q)
              d[q] = v4i{acc_read(acc[x][4 * h + q][0]), acc_read(acc[x][4 * h + q][1]),
                         acc_read(acc[x][4 * h + q][2]), acc_read(acc[x][4 * h + q][3])};
            __builtin_amdgcn_sched_barrier(0);
          }
      } else {
        const int tp = t.slot - g.ncorr;
        const double ip = g.invp[tp];
        const int negp = -g.p[tp];
        int8_t* rdst = g.res8 + (t.b * g.P + tp) * g.outplane;
#pragma unroll
        for (int x = 0; x < kWM; ++x)
#pragma unroll
          for (int h = 0; h < kHB; ++h) {
            store_residue_block<kWM, kWN>(acc, x, h, ip, negp,
                                          rdst + ((rb0 + x) * NB + cb0 + h) * 1024 + lane * 16);
            __builtin_amdgcn_sched_barrier(0);
          }
      }
      G0 += nj;
    }
    // No copy or store may still be in flight when the group retires.
    wait_vm_lgkm0<0>();
  } else if (nk == 0) {
    // A trailing K-split group past the end: its outputs are zeros.
#pragma unroll
    for (int x = 0; x < kWM; ++x)
#pragma unroll
      for (int y = 0; y < kWN; ++y) acc[x][y] = v4i{0, 0, 0, 0};
  } else {
#pragma unroll
    for (int s = 0; s < kPF; ++s)
      if (s < nk) FP64EMU_ISSUE(s);
    v4i F0[kWM + kWN], F1[kWM + kWN];
    // Stage 0 landed (the copies of stages 1 and 2 may still be in flight:
    // k-step 0 waits for stage 1 like every step).
    if (nk >= kPF) wait_vm_lgkm0<(kPF - 1) * kDma>(); else wait_vm_lgkm0<0>();
    barrier_lds();
    FP64EMU_READF(F0, 0);
    // k-step 0 starts the accumulators; then pairs of steps alternate the
    // fragment buffers.  Reading fragments of k-step nk (one past the end)
    // touches a stale stage and is never used; no copy targets it.
    if (nk >= 4) FP64EMU_STEP_FULL(0, F0, F1, mma16_init);
    else FP64EMU_STEP(0, F0, F1, mma16_init);
    int kt = 1;
    for (; kt + 2 <= nk - kPF; kt += 2) {    // copies for kt + kPF and kt + kPF + 1 exist
      FP64EMU_STEP_FULL(kt, F1, F0, mma16);
      FP64EMU_STEP_FULL(kt + 1, F0, F1, mma16);
    }
    for (; kt + 2 <= nk; kt += 2) {
      FP64EMU_STEP(kt, F1, F0, mma16);
      FP64EMU_STEP(kt + 1, F0, F1, mma16);
    }
    if (kt < nk) {
      wait_vm_lgkm0<0>();
      FP64EMU_MMA(F1, mma16);
    }
    // No copy may still target this work group's LDS when it retires.
    wait_vm_lgkm0<0>();
    mfma_fence();   // the last MFMAs' results before anything reads them
  }
#undef FP64EMU_ISSUE
#undef FP64EMU_READF
#undef FP64EMU_MMA
#undef FP64EMU_STEP
#undef FP64EMU_STEP_BODY
#undef FP64EMU_CHUNK
#undef FP64EMU_CHUNK_W
#undef FP64EMU_CHUNK_N
#undef FP64EMU_CHUNK_S
#undef FP64EMU_STEP_FULL
#undef FP64EMU_RSTEP
#undef FP64EMU_RSTEP_FULL
#undef FP64EMU_RSTEP_R
#undef FP64EMU_STREAM_SLOT
#undef FP64EMU_COPY_A
#undef FP64EMU_COPY_B
#undef FP64EMU_XLOAD
#undef FP64EMU_XDOT
#undef FP64EMU_SLOT

  // Epilogue (of a single slot; a run stores each slot as it ends).
  const int64_t NB = g.NB;
  const int64_t rb0 = (int64_t)mt * (2 * kWM) + wm * kWM, cb0 = (int64_t)nt * (kWN / 2) + wn * kHB;
  if constexpr (kRun || kStream) {
  } else if (kDeep && is_corr) {
    // K-segmented: this segment's correction products join the int64 sum.
    typedef long long v2l __attribute__((ext_vector_type(2)));
    int64_t* dst = g.cacc + (((int64_t)split * g.batch + b) * g.ncorr + slot) * g.outplane;
#pragma unroll
    for (int x = 0; x < kWM; ++x)
#pragma unroll
      for (int h = 0; h < kHB; ++h) {
        v2l* d = reinterpret_cast<v2l*>(dst + ((rb0 + x) * NB + cb0 + h) * 1024 + lane * 16);
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            v2l v = v2l{(long long)acc_read(acc[x][4 * h + q][2 * u]),
                        (long long)acc_read(acc[x][4 * h + q][2 * u + 1])};
            if (!g.first) v += d[2 * q + u];
            d[2 * q + u] = v;
          }
        __builtin_amdgcn_sched_barrier(0);
      }
  } else if (kDeep) {
    // K-segmented: balanced residues of this segment join the int32 sums.
    const int t = plane;
    const double ip = g.invp[t];
    const int negp = -g.p[t];
    // bal8's range [-(p/2 - 1), p/2] for even p (for p = 256 the same bytes).
    const bool tie_fix = !(g.p[t] & 1) && g.p[t] != 256;
    const int half_lo = -(g.p[t] >> 1);
    int32_t* dst = g.racc + (((int64_t)split * g.batch + b) * g.P + t) * g.outplane;
#pragma unroll
    for (int x = 0; x < kWM; ++x)
#pragma unroll
      for (int h = 0; h < kHB; ++h) {
        v4i* d = reinterpret_cast<v4i*>(dst + ((rb0 + x) * NB + cb0 + h) * 1024 + lane * 16);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          v4i v;
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            int r = acc_residue(acc_read(acc[x][4 * h + q][u]), ip, negp);
            if (tie_fix) r = r == half_lo ? -half_lo : r;
            // +p/2 (p = 256) is -p/2 in the balanced range: the int8 value
            v[u] = (int)(int8_t)r;
          }
          if (!g.first) v += d[q];
          d[q] = v;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
  } else {
    // One block at a time, the slot kind a uniform branch inside: both kinds
    // keep the same live ranges (two separate loops made the compiler spill
    // an accumulator tile at the split).
    const int t = is_corr ? 0 : plane;
    const double ip = g.invp[t];
    const int negp = -g.p[t];
    // Residues in [-p/2, p/2]: bal8's range for odd p and, bytewise, for
    // p = 256; another even p has its ties' -p/2 turned into bal8's +p/2 by
    // tie_fix_kernel after this launch.
    const int64_t sbm = (int64_t)split * g.batch + b;   // split-major output planes
    int32_t* cdst = g.corr + (sbm * g.ncorr + (is_corr ? slot : 0)) * g.outplane;
    int8_t* rdst = g.res8 + (sbm * g.P + t) * g.outplane;
#pragma unroll
    for (int x = 0; x < kWM; ++x)
#pragma unroll
      for (int h = 0; h < kHB; ++h) {
        const int64_t blk = ((rb0 + x) * NB + cb0 + h) * 1024 + lane * 16;
        if (is_corr) {
          v4i* d = reinterpret_cast<v4i*>(cdst + blk);
#pragma unroll
          for (int q = 0; q < 4; ++q)
            d[q] = v4i{acc_read(acc[x][4 * h + q][0]), acc_read(acc[x][4 * h + q][1]),
                       acc_read(acc[x][4 * h + q][2]), acc_read(acc[x][4 * h + q][3])};
        } else {
          // Stage by stage over the block's 16 values: with one wave per
          // SIMD nothing else hides the latency of a dependent chain.  (The
          // same steps as store_residue_block; written out here, where a
          // call by reference made the compiler shuffle accumulators.)
          int av[16], qv[16];
#pragma unroll
          for (int v = 0; v < 16; ++v) av[v] = acc_read(acc[x][4 * h + v / 4][v % 4]);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int v = 0; v < 16; ++v) qv[v] = __double2loint(fma((double)av[v], ip, kMagic));
          __builtin_amdgcn_sched_barrier(0);
          uint32_t w[4];
#pragma unroll
          for (int q = 0; q < 4; ++q)
            w[q] = pack_bytes(__mul24(qv[4 * q], negp) + av[4 * q], __mul24(qv[4 * q + 1], negp) + av[4 * q + 1],
                              __mul24(qv[4 * q + 2], negp) + av[4 * q + 2], __mul24(qv[4 * q + 3], negp) + av[4 * q + 3]);
          *reinterpret_cast<v4i*>(rdst + blk) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
        }
        __builtin_amdgcn_sched_barrier(0);
      }
  }
}

template <bool kDeep, int kWM, int kWN, bool kRun = false, bool kStream = false>
__global__ void __launch_bounds__(kThreads, (kWM == 8 && kWN == 8) ? 1 : 2)
modgemm_kernel(GemmArgs g) {
  static_assert(!(kRun || kStream) || (kWM == 8 && kWN == 8 && !kDeep),
                "slot runs and item streams: 256 x 256 tiles only");
  using Sh = GemmShape<kWM, kWN>;
  __shared__ __attribute__((aligned(1024))) int8_t lds[Sh::kLdsBytes];
  if constexpr (kStream) {
    modgemm_tile<false, kWM, kWN, false, true>(g, lds, GemmItem{});
    return;
  }
  const GemmItem it = gemm_item(g);
  if constexpr (kRun) {
    if (it.nrun > 1) {
      modgemm_tile<false, kWM, kWN, true>(g, lds, it);
      return;
    }
  }
  modgemm_tile<kDeep, kWM, kWN>(g, lds, it);
}

// 256-column tiles, except that the last tile column holds at most 128
// columns of N: its groups run the narrow body on the tile's first half
// (half the MFMA work of a 256-column tile of mostly padding).
__global__ void __launch_bounds__(kThreads, 1)
modgemm_mixed_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) int8_t lds[GemmShape<8, 8>::kLdsBytes];
  GemmItem it = gemm_item(g);
  if (it.nt == g.TN - 1) {
    it.nt *= 2;
    modgemm_tile<false, 8, 4>(g, lds, it);
  } else {
    modgemm_tile<false, 8, 8>(g, lds, it);
  }
}

// Split streams (use_split_streams): 256 groups, one per CU, each running
// its share of the units' k-steps as one stream (modgemm_tile's kSplitS).
__global__ void __launch_bounds__(kThreads, 1)
modgemm_split_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) int8_t lds[GemmShape<8, 8>::kLdsBytes];
  modgemm_tile<false, 8, 8, false, true, true>(g, lds, GemmItem{});
}

// Split streams with kXc = g.xcols extra columns (a last tile column of at
// most kXMax columns), computed beside the wide tiles.
template <int kXc>
__global__ void __launch_bounds__(kThreads, 1)
modgemm_split_x_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) int8_t lds[GemmShape<8, 8>::kLdsBytes];
  modgemm_tile<false, 8, 8, false, true, true, kXc>(g, lds, GemmItem{});
}

// ---------------------------------------------------------------------------
// Reconstruction.  Per output element: balanced Garner digits
//   d_t = bal((r_t - sum_{u<t} d_u (M_u mod p_t)) (M_t mod p_t)^-1 mod p_t)
// with the O(P^2) inner products as v_dot4_i32_i8 over packed digits; Horner
// per group of 7 moduli (the first four steps of a group in int32: a balanced
// mixed-radix value of four digits is below 2^31); exact: 128-bit
// a0 + M0 (a1 + M1 a2) plus the correction (corr1 + corr2) << (be - 15),
// correctly rounded to double, then ldexp by -(sftA + sftB).
// fp64_emu_cuda/fp64_emu.cu:849-952 and the s128 helpers :53-105.
//
// One work group per 16 x 64 output block: thread t reads dword t of each
// blocked int8 plane and int32s 4t .. 4t+3 of each int32 plane (lane t/4 of
// the GEMM's accumulator order, column block t%4), i.e. rows
// 4 (t / 64) + 0..3 of column 16 (t % 4) + (t / 4) % 16 -- coalesced loads,
// 4 elements per thread, processed in lockstep.

typedef __int128 i128;

// The default list's group products M0 = p_0 .. p_6 and M1 = p_7 .. p_13.
constexpr long long default_group_product(int g) {
  long long prod = 1;
  for (int t = 7 * g; t < 7 * g + 7; ++t) prod *= kDefaultModuli[t];
  return prod;
}
constexpr long long kDefaultM64[2] = {default_group_product(0), default_group_product(1)};

// a m + c as a signed 128-bit (hi, lo) for |a| < 2^62, 0 <= m < 2^62 and
// |c| < 2^61, with four signed 32 x 32 -> 64 multiply-adds: a = ah 2^32 + al
// and m = mh 2^32 + ml with al, ml signed 32-bit, then
//   q0 = al ml + c,  q1 = al mh + ah ml + (q0 >> 32),  q2 = ah mh + (q1 >> 32),
// every partial below 2^63, and a m + c = (q0 mod 2^32) + (q1 mod 2^32) 2^32
// + q2 2^64 (arithmetic shifts: floor division, so negative partials carry
// correctly).
__device__ __forceinline__ void mul_add_wide(int64_t a, uint64_t m, int64_t c, uint64_t& lo,
                                             int64_t& hi) {
  const int32_t al = (int32_t)(uint32_t)a;
  const int32_t ah = (int32_t)(uint32_t)((uint64_t)a >> 32) + (int32_t)((uint32_t)a >> 31);
  const int32_t ml = (int32_t)(uint32_t)m;
  const int32_t mh = (int32_t)(uint32_t)(m >> 32) + (int32_t)((uint32_t)m >> 31);
  const int64_t q0 = (int64_t)al * ml + c;
  const int64_t q1 = (int64_t)al * mh + (int64_t)ah * ml + (q0 >> 32);
  const int64_t q2 = (int64_t)ah * mh + (q1 >> 32);
  lo = ((uint64_t)(uint32_t)q1 << 32) | (uint32_t)q0;
  hi = q2;
}

// Loads and stores through a base address the caller knows to be uniform
// across the wave (moved to scalar registers) plus a 32-bit per-lane byte
// offset: the global scalar-base form, instead of a 64-bit vector address
// per access.
typedef __attribute__((address_space(1))) char gchar;

__device__ __forceinline__ gchar* uniform_base(const void* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<gchar*>(((uint64_t)hi << 32) | lo);
}

template <typename T>
__device__ __forceinline__ T load_at(const void* base, uint32_t byte_off) {
  return *reinterpret_cast<const __attribute__((address_space(1))) T*>(uniform_base(base) + byte_off);
}

template <typename T>
__device__ __forceinline__ void store_at(void* base, uint32_t byte_off, T v) {
  *reinterpret_cast<__attribute__((address_space(1))) T*>(uniform_base(base) + byte_off) = v;
}

// Exactly rounded (to nearest, ties to even) double of a signed 64-bit integer:
// the high word scaled by 2^32 is exact, the one fma rounds the sum once.
__device__ __forceinline__ double i64_to_f64(int64_t v) {
  return fma((double)(int)(v >> 32), 4294967296.0, (double)(uint32_t)v);
}

// Round-to-nearest-even double of the two's-complement 128-bit integer
// w3:w2:w1:w0, scaled by 2^sh.  A value beyond 64 bits is shifted so that its
// top 64 bits keep 63 significant bits (one sign bit), the dropped tail ORed
// into the lowest bit (round to odd: floor or ceil, whichever is odd, which
// rounds to nearest exactly as the full value does, 10 bits below the double's
// precision); the shift and sh fold into one ldexp of the rounded double.
__device__ __forceinline__ double i128w_to_f64(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3, int sh) {
  const int64_t hi = (int64_t)(((uint64_t)w3 << 32) | w2);
  const uint64_t lo = ((uint64_t)w1 << 32) | w0;
  const uint64_t hs = (uint64_t)(hi ^ (hi >> 63));      // leading zeros = redundant sign bits
  if (hs == 0 && (int64_t)(hi ^ (int64_t)lo) >= 0)      // the value fits in 64 bits
    return ldexp(i64_to_f64((int64_t)lo), sh);
  const int k = hs == 0 ? 63 : __clzll((long long)hs) - 1;   // 0..63
  uint64_t top = k == 0 ? (uint64_t)hi : ((uint64_t)hi << k) | (lo >> (64 - k));
  top |= (lo << k) != 0ull ? 1ull : 0ull;
  return ldexp(i64_to_f64((int64_t)top), 64 - k + sh);
}

// The same rounding without a branch between long and short values.  k =
// the value's redundant sign bits, capped at 64: the leading zeros of
// V = ((hi ^ s) << 1) | ((lo ^ s) >> 63), s the sign word (V = 0 when the
// value fits in 64 bits).  Shifted left by k, the value's top 64 bits hold 63
// significant bits (k < 64) or all of it (k = 64: lo, whose top bit is the
// sign, so hi << 63 ORs nothing new in); the dropped tail (the low 64 - k bits
// of lo; for k = 64 lo's bit 0, already the result's bit 0) ORs into the
// lowest bit.  A magnitude of 2^126 or more (k = 0, beyond every plan's
// range) takes the general form above.  sh64 = sh + 64.
__device__ __forceinline__ double i128_to_f64(int64_t hi, uint64_t lo, int sh64) {
  const uint32_t s = (uint32_t)(int32_t)(hi >> 63);
  const uint32_t th = (uint32_t)((uint64_t)hi >> 32) ^ s, tl = (uint32_t)hi ^ s;
  const uint32_t u = (uint32_t)(lo >> 32) ^ s;
  const uint64_t V = ((uint64_t)__builtin_amdgcn_alignbit(th, tl, 31) << 32) |
                     __builtin_amdgcn_alignbit(tl, u, 31);
  const int k = V == 0 ? 64 : __builtin_clzll(V);
  if (k == 0)
    return i128w_to_f64((uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi,
                        (uint32_t)((uint64_t)hi >> 32), sh64 - 64);
  const int kk = k < 63 ? k : 63;
  const uint64_t dropped = lo << kk;
  // min(tail, 1) as one instruction (the compiler's compare-and-select form
  // takes two).
  uint32_t sticky;
  asm("v_min_u32 %0, 1, %1" : "=v"(sticky) : "v"((uint32_t)dropped | (uint32_t)(dropped >> 32)));
  const uint64_t top = ((uint64_t)hi << kk) | (lo >> (64 - k)) | sticky;
  return ldexp(i64_to_f64((int64_t)top), sh64 - k);
}

struct ReconCore {
  const int8_t* res8;
  const int32_t* corr;
  const int32_t* res32;   // K-segmented: residue sums, folded here
  const int64_t* corr64;  // K-segmented: correction sum
  double* out;
  const int16_t* sftA;
  const int16_t* sftB;
  const int* bits_eff;
  int64_t M, N, batch, outplane;
  int64_t NB;          // 64-column blocks per padded output row (Np / 64)
  int64_t MBv, NBv;    // 16-row and 64-column blocks covering the valid M, N
  int64_t nblocks;     // batch * MBv * NBv
  FastDiv per_div;     // by MBv * NBv (blocks per member)
  FastDiv nbv_div;     // by NBv
  int ncorr;
  int ksplit;            // S: residue / correction planes per output, summed here
  int P;                 // modulus count
};

// The modulus-count-specialised kernels (the default list) take their
// constants at compile time and no tables, as the extraction's.
template <bool kTab> struct ReconArgs : ReconCore { ModTables tab; };
template <> struct ReconArgs<false> : ReconCore {};

// kSplit: the GEMM ran with a K-split (its own instantiation, so the split
// sums' registers do not weigh on the common path).  kP: the modulus count
// fixed at compile time (0: read from the tables), so the digit loops unroll
// to exactly P steps without guards.  kP > 0 also
// takes the moduli to be the default list's first kP (all odd after 256);
// kP = 0 handles any admissible list.
template <bool kExact, bool kDeep, int kP, bool kSplit>
__global__ void __launch_bounds__(kThreads)
reconstruct_kernel(ReconArgs<kP == 0> a) {
  // Block -> (member, 16-row block, 64-column block): uniform, so every
  // address below is a scalar base plus a 32-bit per-lane offset.
  const uint32_t blk = blockIdx.x;
  const uint32_t b = a.per_div.div(blk);
  const uint32_t rem = blk - b * a.per_div.d;
  const uint32_t mb = a.nbv_div.div(rem);
  const uint32_t nb = rem - mb * a.nbv_div.d;
  const int thr = threadIdx.x;
  const int l = thr >> 2, q4 = thr & 3;
  // This thread's first row in the block: 4 per wave, so uniform per wave
  // (scalar row checks, shift loads and store bases).
  const int row0 = 4 * __builtin_amdgcn_readfirstlane(thr >> 6);
  const int col = 16 * q4 + (l & 15);          // its column in the block
  const int64_t j = (int64_t)nb * 64 + col;
  const int64_t rows_left = a.M - (int64_t)mb * 16;   // valid rows from the block's first
  if (j >= a.N || row0 >= rows_left) return;

  const int P = kP > 0 ? kP : a.P;
  constexpr bool kUsual = kP > 0;
  // Table entries: compile-time constants of the default modulus list in
  // the specialised kernels (no scalar registers held across the kernel and
  // no tables among the arguments), kernel arguments otherwise.
  auto tab_p = [&](int t) {
    if constexpr (kUsual) return kDefaultTab.p[t]; else return a.tab.p[t];
  };
  auto tab_invp = [&](int t) {
    if constexpr (kUsual) return kDefaultTab.invp[t]; else return a.tab.invp[t];
  };
  auto tab_nmp = [&](int i) {
    if constexpr (kUsual) return kDefaultTab.nmp[i]; else return a.tab.nmp[i];
  };
  auto tab_mib = [&](int t) {
    if constexpr (kUsual) return kDefaultTab.mib[t]; else return a.tab.mib[t];
  };
  auto tab_m64 = [&](int g) {
    if constexpr (kUsual) return kDefaultM64[g]; else return a.tab.m64[g];
  };
  // Byte (int8 planes) / element (int32 planes) offset of this block, and
  // the lane's offset inside it.
  const int64_t boff0 = ((int64_t)mb * a.NB + nb) * 1024;
  const uint32_t lane4 = 4u * (uint32_t)thr;
  const int64_t boff = boff0 + lane4;
  // The output scalings, read with the residues (one round trip, instead of
  // a dependent load per element at the end); rows past M read row M - 1.
  // Both shifts grew by bits_eff[1] at the width pick.
  const int cshift = a.bits_eff[0] - 15;
  const int16_t* sftB_blk = a.sftB + (int64_t)b * a.N + (int64_t)nb * 64;
  const int sj = (int)load_at<int16_t>(sftB_blk, 2u * col) + 2 * a.bits_eff[1];
  const int16_t* sftA_blk = a.sftA + (int64_t)b * a.M + (int64_t)mb * 16;
  const int last_row = (int)(rows_left < 16 ? rows_left : 16) - 1;
  int sai[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) sai[e] = (int)load_at<int16_t>(sftA_blk, 2u * min(row0 + e, last_row));
  uint32_t w[kMaxP];
  int64_t cv[4] = {0, 0, 0, 0};
  if (kDeep) {
    // Fold the segment sums (|sum| <= 128 per segment and split) to balanced
    // residues; the S splits' sums add first, and so do their correction
    // sums (S x ncorr int64 planes).
    const int64_t sstride = (int64_t)a.batch * P * a.outplane;
#pragma unroll
    for (int t = 0; t < kMaxP; ++t)
      if (t < P) {
        const int32_t* r = a.res32 + (b * P + t) * a.outplane + boff;
        v4i v = *reinterpret_cast<const v4i*>(r);
        for (int sp = 1; sp < a.ksplit; ++sp) v += *reinterpret_cast<const v4i*>(r + sp * sstride);
        const double ip = tab_invp(t);
        const int negp = -tab_p(t);
        w[t] = pack_bytes(acc_residue(v[0], ip, negp), acc_residue(v[1], ip, negp),
                          acc_residue(v[2], ip, negp), acc_residue(v[3], ip, negp));
      }
    for (int sp = 0; sp < a.ksplit; ++sp)
      for (int cc = 0; cc < a.ncorr; ++cc) {
        const int64_t* c = a.corr64 + (((int64_t)sp * a.batch + b) * a.ncorr + cc) * a.outplane + boff;
#pragma unroll
        for (int e = 0; e < 4; ++e) cv[e] += c[e];
      }
  } else if (!kSplit) {
    const int8_t* rb = a.res8 + (int64_t)b * P * a.outplane + boff0;
#pragma unroll
    for (int t = 0; t < kMaxP; ++t)
      if (t < P) w[t] = load_at<uint32_t>(rb + t * a.outplane, lane4);
  } else {
    // K-split: the S partial residues sum (|sum| <= 128 S) and fold to the
    // residue (any representative serves: each digit reduces mod p again),
    // and the S x ncorr correction parts add up.  Two splits per iteration,
    // residues and corrections together, so the loads share each round trip;
    // for an odd S the last iteration's second split is zeros (a uniform
    // condition), never a read past the S planes.
    int sums[kMaxP][4];
#pragma unroll
    for (int t = 0; t < kMaxP; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e) sums[t][e] = 0;
    for (int sp = 0; sp < a.ksplit; sp += 2) {
      uint32_t u[2][kMaxP];
      v4i cw[2][2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const bool live = h == 0 || sp + 1 < a.ksplit;
#pragma unroll
        for (int t = 0; t < kMaxP; ++t)
          if (t < P)
            u[h][t] = live ? *reinterpret_cast<const uint32_t*>(
                                 a.res8 + (((sp + h) * a.batch + b) * P + t) * a.outplane + boff)
                           : 0u;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
          if (cc < a.ncorr)
            cw[h][cc] = live ? *reinterpret_cast<const v4i*>(
                                   a.corr + (((sp + h) * a.batch + b) * a.ncorr + cc) * a.outplane + boff)
                             : v4i{0, 0, 0, 0};
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int t = 0; t < kMaxP; ++t)
          if (t < P) {
#pragma unroll
            for (int e = 0; e < 4; ++e) sums[t][e] += (int)(int8_t)(uint8_t)(u[h][t] >> (8 * e));
          }
#pragma unroll
        for (int cc = 0; cc < 2; ++cc)
          if (cc < a.ncorr) {
#pragma unroll
            for (int e = 0; e < 4; ++e) cv[e] += cw[h][cc][e];
          }
      }
    }
#pragma unroll
    for (int t = 0; t < kMaxP; ++t)
      if (t < P) {
        const int* sum4 = sums[t];
        const double pd = (double)tab_p(t), ip = tab_invp(t);
        uint32_t u = 0u;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const double vd = (double)sum4[e];
          u |= ((uint32_t)(int)fma(-floor(fma(vd, ip, kHalfUp)), pd, vd) & 0xFFu) << (8 * e);
        }
        w[t] = u;
      }
  }
  if (!kDeep && !kSplit && a.ncorr > 0) {   // (a K-split summed them above)
    const int32_t* cb = a.corr + (int64_t)b * a.ncorr * a.outplane + boff0;
    const v4i c1 = load_at<v4i>(cb, 4 * lane4);
#pragma unroll
    for (int e = 0; e < 4; ++e) cv[e] = c1[e];
    if (a.ncorr == 2) {
      const v4i c2 = load_at<v4i>(cb + a.outplane, 4 * lane4);
#pragma unroll
      for (int e = 0; e < 4; ++e) cv[e] += c2[e];
    }
  }


  // Garner digits, 4 elements in lockstep.
  int dg[4][kMaxP];
  int dp[4][kGarnerWords];
#pragma unroll
  for (int e = 0; e < 4; ++e)
#pragma unroll
    for (int g = 0; g < kGarnerWords; ++g) dp[e][g] = 0;
  if constexpr (kUsual) {
    // The digits of X + M/2, in [0, p_t) (default_digit_offset): digit 0 is
    // r_0 + 128, the residue byte with its top bit flipped; digit t is y mod
    // p_t for y = 128 p_t + r_t minv_t + sum_{u<t} d_u (-M_u minv_t mod p_t),
    // the sum as unsigned dot products of digit bytes and factor bytes in
    // [0, p_t), so 0 < y < 2^21 and its quotient by p_t is one high multiply
    // (mq = ceil(2^32 / p_t): exact below 2^24).
    const uint32_t u0 = w[0] ^ 0x80808080u;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t s0 = u0 >> (8 * e);
      dg[e][0] = (int)(s0 & 0xFFu);
      dp[e][0] = (int)s0;   // bytes 1..3 meet zero factors until digits 1..3 land there
    }
#pragma unroll
    for (int t = 1; t < kMaxP; ++t) {
      if (t >= P) continue;
      const int pt = kDefaultModuli[t];
      const int mib = kDefaultTab.mib[t];
      const uint32_t mq = kDefaultTab.mq[t];
      const int sh = 8 * (t & 3);
      // 128 p_t in one register for the four elements' first dot products
      // (kept opaque: the compiler would otherwise rematerialise it into each
      // chain's accumulator, one move per element).
      uint32_t bias;
      asm volatile("v_mov_b32 %0, %1" : "=v"(bias) : "i"(128 * pt));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // The digits' terms first (from 128 p_t), then r_t minv_t from byte e
        // of the residue word (the factor word holds minv_t at byte e only).
        // (Issuing the residue term first, off the digit-to-digit chain, in
        // the three-operand form with the factor in a scalar register
        // measured 3% slower at 8192^3.)
        uint32_t y = bias;
#pragma unroll
        for (int g = 0; g < kGarnerWords; ++g)
          if (4 * g < t)
            y = __builtin_amdgcn_udot4((uint32_t)dp[e][g], kDefaultTab.ump[t * kGarnerWords + g], y, false);
        y = (uint32_t)__builtin_amdgcn_sdot4((int)w[t], (int)((uint32_t)(uint8_t)(int8_t)mib << (8 * e)),
                                             (int)y, false);
        const int d = __mul24((int)__umulhi(y, mq), -pt) + (int)y;
        dg[e][t] = d;
        dp[e][t >> 2] = (t & 3) == 0 ? d
                                     : (int)__builtin_amdgcn_perm((uint32_t)d, (uint32_t)dp[e][t >> 2],
                                                                   (0x03020100u & ~(0xFFu << sh)) | (0x04u << sh));
      }
    }
  } else {
#pragma unroll
    for (int t = 0; t < kMaxP; ++t) {
      if (t >= P) continue;
      const int pt = tab_p(t);
      if (t == 0) {
        // M_0 = 1: the first digit is the residue.  The GEMM epilogue and the
        // folds above leave it in [-p/2, (p-1)/2] for odd p (nearest quotient)
        // and for p = 256 (any representative's low byte is that range); any
        // other even p is brought there by the floor rule of barrett_bal32.
        const bool norm = !(pt & 1) && pt != 256;
        const double pd0 = (double)pt, ip0 = tab_invp(0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          int d = (int)(int8_t)(uint8_t)(w[0] >> (8 * e));
          if (norm) {
            const double rd = (double)d;
            d = (int)fma(-floor(fma(rd, ip0, kHalfUp)), pd0, rd);
          }
          dg[e][0] = d;
          dp[e][0] = d;   // bytes 1..3 meet zero factors until digits 1..3 land there
        }
        continue;
      }
      const double nip = -tab_invp(t);
      int nmw[kGarnerWords];
#pragma unroll
      for (int g = 0; g < kGarnerWords; ++g) nmw[g] = (4 * g < t) ? tab_nmp(t * kGarnerWords + g) : 0;
      const int mib = tab_mib(t);
      const int sh = 8 * (t & 3);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // y = (r_t - sum_{u<t} d_u M_u) minv_t mod p_t as dot products: r_t
        // minv_t from byte e of the residue word (the factor word holds minv_t
        // at byte e only), then the digits' terms; |y| < 20 * 2^14.
        int y = sdot4_zero(w[t], (uint32_t)(uint8_t)(int8_t)mib << (8 * e));
#pragma unroll
        for (int g = 0; g < kGarnerWords; ++g)
          if (4 * g < t) y = __builtin_amdgcn_sdot4(dp[e][g], nmw[g], y, false);
        // d = y - p q, q the nearest integer to y/p (-q is the low word of the
        // fma rounding -y/p; |q| < 2^19).  Odd p has no ties: d lies in
        // [-(p-1)/2, (p-1)/2].  Even p may give +p/2, barrett_bal32's -p/2.
        int d = __mul24(__double2loint(fma((double)y, nip, kMagic)), pt) + y;
        if (!(pt & 1)) d = d == (pt >> 1) ? -(pt >> 1) : d;
        dg[e][t] = d;
        // Insert the digit's low byte at byte t % 4 of its word.
        dp[e][t >> 2] = (t & 3) == 0 ? d
                                     : (int)__builtin_amdgcn_perm((uint32_t)d, (uint32_t)dp[e][t >> 2],
                                                                   (0x03020100u & ~(0xFFu << sh)) | (0x04u << sh));
      }
    }
  }

  // The wave's output rows from a uniform base; the lane's byte offset is
  // its column's.
  double* const oblk = a.out + ((int64_t)b * a.M + (int64_t)mb * 16 + row0) * a.N + (int64_t)nb * 64;
  const uint32_t olane = 8u * (uint32_t)col;

  // Horner per group of 7 (digits 7g .. 7g+6, high to low), in two 32-bit
  // halves: positions 6..3 give H, positions 2..0 give L (below 2^24), and
  // the group value is H (p_0 p_1 p_2) + L, one 32 x 32 -> 64-bit
  // multiply-add (p_i the group's first three moduli; a group of at most
  // three digits has H = 0).  Every partial H below its last step is below
  // 2^24, so the 24-bit multiplies are exact.  Balanced digits: |H| < 2^31.
  // Default-list digits (in [0, p)): H < p_3 p_4 p_5 p_6 < 2^32 unsigned, and
  // the group's digit offset comes off the 64-bit value.
  long long ag[4][3];
  if constexpr (kUsual) {
    uint32_t h32[4][3], l32[4][3];
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int g = 0; g < 3; ++g) { h32[e][g] = 0u; l32[e][g] = 0u; }
#pragma unroll
    for (int t = kMaxP - 1; t >= 0; --t) {
      if (t >= P) continue;
      const int g = t / 7, pos = t % 7;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (pos >= 3) h32[e][g] = __umul24(h32[e][g], (uint32_t)kDefaultModuli[t]) + (uint32_t)dg[e][t];
        else l32[e][g] = __umul24(l32[e][g], (uint32_t)kDefaultModuli[t]) + (uint32_t)dg[e][t];
      }
    }
#pragma unroll
    for (int g = 0; g < 3; ++g) {
      const int t0 = 7 * g;
      const uint32_t p3 = t0 + 2 < kMaxP ? (uint32_t)(kDefaultModuli[t0] * kDefaultModuli[t0 + 1] *
                                                      kDefaultModuli[t0 + 2]) : 0u;
      const long long off = default_digit_offset(kP, g);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        ag[e][g] = (long long)((unsigned long long)h32[e][g] * p3 + l32[e][g]) - off;
    }
  } else {
    int h32[4][3], l32[4][3];
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int g = 0; g < 3; ++g) { h32[e][g] = 0; l32[e][g] = 0; }
#pragma unroll
    for (int t = kMaxP - 1; t >= 0; --t) {
      if (t >= P) continue;
      const int g = t / 7, pos = t % 7;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (pos >= 3) h32[e][g] = __mul24(h32[e][g], tab_p(t)) + dg[e][t];
        else l32[e][g] = __mul24(l32[e][g], tab_p(t)) + dg[e][t];
      }
    }
#pragma unroll
    for (int g = 0; g < 3; ++g) {
      const int t0 = 7 * g;
      // p_0 p_1 p_2 of group g (< 2^24); moduli past P only meet H = 0.
      const int p3 = t0 + 2 < kMaxP ? tab_p(t0) * tab_p(t0 + 1) * tab_p(t0 + 2) : 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) ag[e][g] = (long long)h32[e][g] * p3 + l32[e][g];
    }
  }

  const int ng = (P + 6) / 7;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (row0 + e >= rows_left) continue;
    // Every group ends on its position-0 digit, an int64 step, so ag holds
    // the group value whatever the group's digit count.
    const long long a0 = ag[e][0], a1 = ag[e][1], a2 = ag[e][2];
    const int sh = -(sai[e] + sj);
    double val;
    if (kExact) {
      // X = a0 + M0 (a1 + M1 a2) as a 128-bit word pair (hi, lo).  The one
      // or two group products of the usual plans (at most 15 moduli: group 2
      // holds at most one digit, so a1 + M1 a2 fits 63 bits) take
      // mul_add_wide's four 32 x 32 -> 64 multiply-adds; longer lists take
      // the general 128-bit product (the true X stays below 2^127, so the
      // products wrap modulo 2^128 harmlessly).
      const uint64_t m0 = (uint64_t)tab_m64(0);
      const uint64_t m1 = (uint64_t)tab_m64(1);
      uint64_t lo;
      int64_t hi;
      if (ng == 1) {
        lo = (uint64_t)a0;
        hi = a0 >> 63;
      } else if (ng == 2 || (kUsual && P == 15)) {
        const int64_t top = ng == 2 ? a1 : (int64_t)((uint64_t)a2 * m1) + a1;
        mul_add_wide(top, m0, a0, lo, hi);
      } else {
        i128 acc = (i128)a2 * (i128)m1 + a1;
        acc = acc * (i128)m0 + a0;
        lo = (uint64_t)acc;
        hi = (int64_t)(acc >> 64);
      }
      // + corr 2^cshift: 1 <= cshift <= 38 (bits_eff in [16, 53]), so the
      // shifted value is the word pair (cv >> (64 - cshift), cv << cshift).
      const unsigned __int128 cw =
          ((unsigned __int128)(uint64_t)(cv[e] >> (64 - cshift)) << 64) | ((uint64_t)cv[e] << cshift);
      const unsigned __int128 u = (((unsigned __int128)(uint64_t)hi << 64) | lo) + cw;
      store_at<double>(oblk + e * a.N, olane, i128_to_f64((int64_t)(u >> 64), (uint64_t)u, 64 + sh));
      continue;
    } else {
      double acc = (double)(ng == 3 ? a2 : (ng == 2 ? a1 : a0));
      if (ng == 3) acc = fma(acc, (double)tab_m64(1), (double)a1);
      if (ng >= 2) acc = fma(acc, (double)tab_m64(0), (double)a0);
      acc = acc + ldexp((double)cv[e], cshift);
      val = acc;
    }
    store_at<double>(oblk + e * a.N, olane, ldexp(val, sh));
  }
}

// bal8's range for an even modulus other than 256 is [-(p/2 - 1), p/2]; the
// GEMM epilogue's nearest quotient leaves ties at -p/2.  This pass turns
// those bytes into +p/2 in every residue plane of that modulus (nplanes
// planes, plane_stride bytes apart).  Default modulus sets never launch it.
__global__ void __launch_bounds__(kThreads)
tie_fix_kernel(int8_t* res8, int64_t outplane, int64_t nplanes, int64_t plane_stride, int p) {
  const int8_t lo = (int8_t)(-(p >> 1)), hi = (int8_t)(p >> 1);
  const int64_t words = outplane / 16, n = nplanes * words;
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads) {
    const int64_t pl = i / words;
    v4i* q = reinterpret_cast<v4i*>(res8 + pl * plane_stride) + (i - pl * words);
    v4i v = *q;
    int8_t* b = reinterpret_cast<int8_t*>(&v);
#pragma unroll
    for (int e = 0; e < 16; ++e) b[e] = b[e] == lo ? hi : b[e];
    *q = v;
  }
}

__global__ void __launch_bounds__(kThreads) fill_zero_kernel(double* out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * kThreads)
    out[i] = 0.0;
}

// ---------------------------------------------------------------------------
// Double-double GEMM for correct-bits measurement (not on the product path):
// per k, the exact product p + e (FMA error-free transform) joins hi by a
// two-sum, the tails collect in lo, and hi/lo renormalise -- the sequence of
// bench/accuracy.py:39-50 of the reference.  16x16 threads per block, 16x16
// operand tiles through LDS.
__device__ __forceinline__ void two_sum(double a, double b, double& s, double& e) {
  s = a + b;
  const double bb = s - a;
  e = (a - (s - bb)) + (b - bb);
}

__global__ void __launch_bounds__(kThreads)
ddgemm_nt_kernel(double* __restrict__ hi, double* __restrict__ lo, const double* __restrict__ A,
                 const double* __restrict__ B, int64_t M, int64_t N, int64_t K) {
  __shared__ double sa[16][17], sb[16][17];
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
  const int64_t i = (int64_t)blockIdx.y * 16 + ty, j = (int64_t)blockIdx.x * 16 + tx;
  double h = 0.0, l = 0.0;
  for (int64_t k0 = 0; k0 < K; k0 += 16) {
    const int64_t ra = (int64_t)blockIdx.y * 16 + ty, rb = (int64_t)blockIdx.x * 16 + ty;
    sa[ty][tx] = (ra < M && k0 + tx < K) ? A[ra * K + k0 + tx] : 0.0;
    sb[ty][tx] = (rb < N && k0 + tx < K) ? B[rb * K + k0 + tx] : 0.0;
    __syncthreads();
    const int kk = (int)min<int64_t>(16, K - k0);
    for (int k = 0; k < kk; ++k) {
      const double x = sa[ty][k], y = sb[tx][k];
      const double p = x * y;
      const double e = fma(x, y, -p);
      double s, t;
      two_sum(h, p, s, t);
      l = l + (t + e);
      two_sum(s, l, h, l);
    }
    __syncthreads();
  }
  if (i < M && j < N) {
    hi[i * N + j] = h;
    lo[i * N + j] = l;
  }
}

// ---------------------------------------------------------------------------
// Ceiling probes (not on the product path): the rates this part attains, for
// the benchmark to set the modular GEMM and the byte phases against.
//
// mfma_probe_kernel<kMode>: the modular GEMM's work-group shape and inner
// loop without its data: 4 waves (one per SIMD, one group per CU), each
// with 8 x 8 accumulator quads, 64 v_mfma_i32_16x16x64_i8 per step in the
// GEMM's serpentine order, on fragments that alternate between two stages
// of the source (A tile, then B tile, 32 KiB each, in the planes' fragment
// order).
//   kMode 0: both stages' fragments stay in registers (no memory traffic).
//   kMode 1: the next step's 16 fragments are read from the GEMM's 4-stage
//            LDS ring as the GEMM reads them (one per 4 MFMAs), with the
//            per-step wait and barrier.
//   kMode 2: kMode 1 plus the GEMM's direct global->LDS copies of the stage
//            three steps ahead (8 of 1 KiB per wave per step) from the 64 KiB
//            source, which every L2 holds: the GEMM's inner loop without
//            HBM or fabric traffic, prologue, epilogue or tail.
// Ring slot q holds stage q mod 2 throughout (the copies rewrite the same
// bytes), so after `steps` steps every accumulator holds the sum of the
// stages' products: the benchmark's source makes stage 1's A tile the
// negation of stage 0's, so an even step count leaves zeros and an odd one
// stage 0's product, which the tests check element by element.  Group 0
// stores its accumulators ([wave][x][y] blocks of 256 int32, lane l's value
// v at 4 l + v).  Thread 0 of each group records s_memtime (shader clock)
// and s_memrealtime (100 MHz) after the first barrier and after the loop.
template <int kMode>
__global__ void __launch_bounds__(kThreads, 1)
mfma_probe_kernel(const int8_t* __restrict__ src, int64_t steps, int32_t* __restrict__ acc_out,
                  unsigned long long* __restrict__ clk) {
  constexpr int kS = 4, kSB = 2 * kTileBytes;
  __shared__ __attribute__((aligned(1024))) int8_t lds[kMode == 0 ? 16 : kS * kSB];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  v4i F0[16], F1[16];
  v4i acc[8][8];
  // Fragment f of stage s: f < 8 is A row block 8 wm + f, else B column
  // block 8 wn + f - 8.
  auto src_frag = [&](int s, int f) -> v4i {
    const v4i* p = reinterpret_cast<const v4i*>(src + s * kSB);
    return f < 8 ? p[(wm * 8 + f) * 64 + lane] : p[kTileBytes / 16 + (wn * 8 + f - 8) * 64 + lane];
  };
  if constexpr (kMode == 0) {
#pragma unroll
    for (int f = 0; f < 16; ++f) {
      F0[f] = src_frag(0, f);
      F1[f] = src_frag(1, f);
    }
  } else {
    // Every ring slot q gets stage q mod 2: 4 x 32 KiB, 512 bytes per thread.
    const v4i* s4 = reinterpret_cast<const v4i*>(src);
    v4i* l4 = reinterpret_cast<v4i*>(lds);
#pragma unroll 4
    for (int i = tid; i < kS * kSB / 16; i += kThreads) l4[i] = s4[i % (2 * kSB / 16)];
    __syncthreads();
    const v4i* sl = reinterpret_cast<const v4i*>(lds);
#pragma unroll
    for (int f = 0; f < 16; ++f)
      F0[f] = f < 8 ? sl[(wm * 8 + f) * 64 + lane] : sl[kTileBytes / 16 + (wn * 8 + f - 8) * 64 + lane];
  }
  __syncthreads();
  unsigned long long t0 = 0, r0 = 0;
  if (tid == 0) {
    t0 = __builtin_amdgcn_s_memtime();
    r0 = __builtin_amdgcn_s_memrealtime();
  }
  const uint32_t goff = (uint32_t)(wave * 4096 + lane * 16);
  // One step: the MFMAs on FC, in modes 1 and 2 the next step's fragments
  // into FN from ring slot (kt + 1) mod 4 and (mode 2) the copies of stage
  // kt + 3 into slot (kt + 3) mod 4, spread as in the GEMM.
  auto step = [&](const int64_t kt, v4i(&FC)[16], v4i(&FN)[16], auto first) {
    if constexpr (kMode != 0) {
      wait_vm_lgkm0<kMode == 2 ? 8 : 0>();
      barrier_lds();
    }
    const v4i* sa = reinterpret_cast<const v4i*>(lds + ((kt + 1) & 3) * kSB);
    const v4i* sb = sa + kTileBytes / 16;
    const int8_t* cg = src + ((kt + 3) & 1) * kSB + goff;
    lds_i8* cl = (lds_i8*)(lds + ((kt + 3) & 3) * kSB + wave * 4096);
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (kMode == 2) {
          const int half = (c >> 1) * kTileBytes;   // chunks 0, 1 copy A; 2, 3 copy B
          if (j == 0 && !(c & 1)) copy_lds16<0>(cg + half, cl + half);
          if (j == 2 && !(c & 1)) copy_lds16<1024>(cg + half, cl + half);
          if (j == 0 && (c & 1)) copy_lds16<2048>(cg + half, cl + half);
          if (j == 2 && (c & 1)) copy_lds16<3072>(cg + half, cl + half);
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (kMode != 0) {
          const int f = c * 4 + j;
          if (f < 8) FN[8 + f] = sb[(wn * 8 + f) * 64 + lane];
          else FN[f - 8] = sa[(wm * 8 + f - 8) * 64 + lane];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int m = 4 * j + u, x = c * 2 + m / 8, y = (m < 8) ? m : 15 - m;
          if constexpr (decltype(first)::value) mma16_init(acc[x][y], FC[x], FC[8 + y]);
          else mma16(acc[x][y], FC[x], FC[8 + y]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
  };
  // Modes 1, 2 read step kt + 1's fragments during step kt; mode 0's second
  // set is stage 1 from the start.
  step(0, F0, F1, std::true_type{});
  int64_t kt = 1;
  for (; kt + 2 <= steps; kt += 2) {
    step(kt, F1, F0, std::false_type{});
    step(kt + 1, F0, F1, std::false_type{});
  }
  if (kt < steps) step(kt, F1, F0, std::false_type{});
  wait_vm_lgkm0<0>();
  mfma_fence();
  if (tid == 0) {
    const unsigned long long t1 = __builtin_amdgcn_s_memtime();
    const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
    unsigned long long* c = clk + (int64_t)blockIdx.x * 4;
    c[0] = t0; c[1] = t1; c[2] = r0; c[3] = r1;
  }
  if (blockIdx.x == 0) {
#pragma unroll
    for (int x = 0; x < 8; ++x)
#pragma unroll
      for (int y = 0; y < 8; ++y) {
        int32_t* d = acc_out + ((wave * 8 + x) * 8 + y) * 256 + lane * 4;
        *reinterpret_cast<v4i*>(d) = v4i{acc_read(acc[x][y][0]), acc_read(acc[x][y][1]),
                                         acc_read(acc[x][y][2]), acc_read(acc[x][y][3])};
      }
  }
}

// stream_probe_kernel<kMode>: HBM streaming over n doubles, each group over
// one contiguous chunk, 16 bytes per lane per access and four accesses in
// flight per lane (contiguous chunks streamed 6.0 / 5.6-6.0 / 5.3 TB/s
// reading / writing / copying 1 GiB, against 5.0 / 4.2-4.7 / 4.3 for a
// grid-stride walk).  kMode 0 reads (each group's sum to dst[group]), 1
// writes dst = v, 2 copies dst = -src (read plus write, the shape of the
// extraction and the reconstruction).
template <int kMode>
__global__ void __launch_bounds__(kThreads)
stream_probe_kernel(double* __restrict__ dst, const double* __restrict__ src, int64_t n2, double v) {
  typedef double v2d __attribute__((ext_vector_type(2)));
  const v2d* s = reinterpret_cast<const v2d*>(src);
  v2d* d = reinterpret_cast<v2d*>(dst);
  const int64_t per = (n2 + gridDim.x - 1) / gridDim.x;
  const int64_t b0 = (int64_t)blockIdx.x * per, b1 = min(b0 + per, n2);
  v2d sum = v2d{0.0, 0.0};
  for (int64_t i = b0 + threadIdx.x; i < b1; i += 4 * kThreads) {
    v2d x[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (kMode != 1 && i + u * kThreads < b1) x[u] = s[i + u * kThreads];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (i + u * kThreads >= b1) continue;
      if constexpr (kMode == 0) sum += x[u];
      else if constexpr (kMode == 1) d[i + u * kThreads] = v2d{v, v};
      else d[i + u * kThreads] = -x[u];
    }
  }
  if constexpr (kMode == 0) {
    __shared__ double red[kThreads];
    red[threadIdx.x] = sum.x + sum.y;
    __syncthreads();
    for (int w = kThreads / 2; w > 0; w >>= 1) {
      if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
      __syncthreads();
    }
    if (threadIdx.x == 0) dst[blockIdx.x] = red[0];
  }
}

// ---------------------------------------------------------------------------
// Host orchestration.  fp64_emu_cuda/fp64_emu.cu:1127-1186, 1220-1270,
// 1343-1407 (the fused slice): sizing -> extraction -> modular GEMMs ->
// reconstruction on one stream, phase events when requested.

struct Call {
  double* out;
  const double* A;
  const double* B;
  int64_t batch, M, N, K;
  bool b_kn;
  const int32_t* primes;
  int P;
  bool exact;
  int bits;
  bool corr;
  void* ws;
  size_t ws_bytes;
  hipStream_t stream;
  hipEvent_t* ev;   // 5 events or nullptr
};

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return FP64EMU_OK;
  return fail(FP64EMU_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

int validate_primes(const int32_t* primes, int P) {
  if (P < 1) return fail(FP64EMU_EINVAL, "nprimes must be >= 1");
  if (P > kMaxP) return fail(FP64EMU_EINVAL, "too many primes");
  if (!primes) return fail(FP64EMU_EINVAL, "primes must not be NULL");
  for (int t = 0; t < P; ++t) {
    if (primes[t] < 2 || primes[t] > 256) return fail(FP64EMU_EINVAL, "moduli must be in [2, 256]");
    for (int u = 0; u < t; ++u)
      if (gcd_int(primes[t], primes[u]) != 1)
        return fail(FP64EMU_EINVAL, "moduli must be pairwise coprime");
  }
  return FP64EMU_OK;
}

// Modulus counts of the planner (plan_config: 14-15; plan: up to 20) get a
// reconstruction compiled for their exact count; others use the generic one.
template <bool kExact, bool kSplit>
void launch_reconstruct_p(int P, unsigned grid, hipStream_t s, const ReconCore& rc,
                          const ModTables& tab) {
  // The specialised kernels carry the default modulus list's constants and
  // take no tables; other lists run the generic one with the tables.
  bool usual = true;
  for (int t = 0; t < P; ++t) usual = usual && tab.p[t] == kDefaultModuli[t];
  ReconArgs<false> rd;
  static_cast<ReconCore&>(rd) = rc;
  switch (usual ? P : 0) {
#define FP64EMU_RECON_CASE(n)                                                                   \
    case n:                                                                                     \
      hipLaunchKernelGGL((reconstruct_kernel<kExact, false, n, kSplit>), dim3(grid),            \
                         dim3(kThreads), 0, s, rd);                                             \
      return;
    FP64EMU_RECON_CASE(12) FP64EMU_RECON_CASE(13) FP64EMU_RECON_CASE(14)
    FP64EMU_RECON_CASE(15) FP64EMU_RECON_CASE(16) FP64EMU_RECON_CASE(17)
    FP64EMU_RECON_CASE(18) FP64EMU_RECON_CASE(19) FP64EMU_RECON_CASE(20)
#undef FP64EMU_RECON_CASE
    default: {
      ReconArgs<true> rg;
      static_cast<ReconCore&>(rg) = rc;
      rg.tab = tab;
      hipLaunchKernelGGL((reconstruct_kernel<kExact, false, 0, kSplit>), dim3(grid), dim3(kThreads),
                         0, s, rg);
    }
  }
}

void launch_reconstruct(bool exact, int P, unsigned grid, hipStream_t s, const ReconCore& rc,
                        const ModTables& tab) {
  const bool split = rc.ksplit > 1;
  if (exact) {
    if (split) launch_reconstruct_p<true, true>(P, grid, s, rc, tab);
    else launch_reconstruct_p<true, false>(P, grid, s, rc, tab);
  } else {
    if (split) launch_reconstruct_p<false, true>(P, grid, s, rc, tab);
    else launch_reconstruct_p<false, false>(P, grid, s, rc, tab);
  }
}

int run(const Call& c) {
  if (int st = validate_primes(c.primes, c.P)) return st;
  if (c.bits < 16 || c.bits > 53) return fail(FP64EMU_EINVAL, "bits must be in [16, 53]");
  if (c.batch < 0 || c.M < 0 || c.N < 0 || c.K < 0)
    return fail(FP64EMU_EINVAL, "shapes must be non-negative");
  if (c.K > kMaxKSingle && (c.b_kn || c.ev))
    return fail(FP64EMU_EINVAL, "K bound for int32 modular GEMM");
  if (c.K > kMaxKDeep) return fail(FP64EMU_EINVAL, "K bound: 128 segments of 65536");
  fp64emu_layout_t L;
  make_layout(c.batch, c.M, c.N, c.K, c.P, c.corr, &L);
  const hipStream_t s = c.stream;
  if (c.ev) {
    if (int st = check_hip(hipEventRecord(c.ev[0], s), "hipEventRecord")) return st;
  }
  const int64_t MF = c.batch * c.M, NF = c.batch * c.N;
  if (MF == 0 || NF == 0) {
    if (c.ev)
      for (int e = 1; e < 5; ++e)
        if (int st = check_hip(hipEventRecord(c.ev[e], s), "hipEventRecord")) return st;
    return FP64EMU_OK;
  }
  if (!c.out) return fail(FP64EMU_EINVAL, "null operand pointer");
  if (c.K == 0) {
    // Empty sums: zeros, written by a kernel (no memset node under capture).
    const int64_t n = MF * c.N;
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)std::min<int64_t>((n + kThreads - 1) / kThreads, 65535)),
                       dim3(kThreads), 0, s, c.out, n);
    if (int st = check_hip(hipGetLastError(), "kernel launch")) return st;
    if (c.ev)
      for (int e = 1; e < 5; ++e)
        if (int st = check_hip(hipEventRecord(c.ev[e], s), "hipEventRecord")) return st;
    return FP64EMU_OK;
  }
  if (!c.A || !c.B) return fail(FP64EMU_EINVAL, "null operand pointer");
  if (!c.ws) return fail(FP64EMU_EWORKSPACE, "workspace too small");
  if (reinterpret_cast<uintptr_t>(c.ws) % kAlign)
    return fail(FP64EMU_EINVAL, "workspace must be 256-byte aligned");
  if (c.ws_bytes < L.total) {
    // Short workspace: the fewest row chunks of A that fit (batch 1, not
    // K-segmented, no phase events).
    bool fits = false;
    if (c.batch == 1 && !L.deep && !c.ev) {
      const int64_t TM = L.Mp / kTileR;
      int64_t last_tiles = TM;
      for (int64_t nc = 2; nc <= TM && !fits; ++nc) {
        const int64_t ct = (TM + nc - 1) / nc;
        if (ct == last_tiles) continue;
        last_tiles = ct;
        fp64emu_layout_t Lc;
        make_layout(c.batch, c.M, c.N, c.K, c.P, c.corr, &Lc, nc);
        if (c.ws_bytes >= Lc.total) { L = Lc; fits = true; }
      }
    }
    if (!fits) return fail(FP64EMU_EWORKSPACE, "workspace too small");
  }
  const ModTables tab = make_tables(c.primes, c.P);
  bool default_moduli = true;
  for (int t = 0; t < c.P; ++t) default_moduli = default_moduli && c.primes[t] == kDefaultModuli[t];

  char* ws = static_cast<char*>(c.ws);
  int16_t* sftA = reinterpret_cast<int16_t*>(ws + L.off_sftA);
  int16_t* sftB = reinterpret_cast<int16_t*>(ws + L.off_sftB);
  float* lgA = reinterpret_cast<float*>(ws + L.off_lgA);
  float* lgB = reinterpret_cast<float*>(ws + L.off_lgB);
  int* bits_eff = reinterpret_cast<int*>(ws + L.off_bits);
  double* pmax = reinterpret_cast<double*>(ws + L.off_pmax);
  double* pss = reinterpret_cast<double*>(ws + L.off_pss);
  int8_t* planesA = reinterpret_cast<int8_t*>(ws + L.off_planesA);
  int8_t* planesB = reinterpret_cast<int8_t*>(ws + L.off_planesB);
  int8_t* res8 = reinterpret_cast<int8_t*>(ws + L.off_res8);
  int32_t* corr = reinterpret_cast<int32_t*>(ws + L.off_corr);

  // The modular GEMM's arguments (its launches follow the sizing).
  GemmArgs ga;
  ga.A = planesA; ga.B = planesB; ga.res8 = res8; ga.corr = corr;
  ga.racc = L.deep ? reinterpret_cast<int32_t*>(res8) : nullptr;
  ga.cacc = L.deep ? reinterpret_cast<int64_t*>(corr) : nullptr;
  ga.memberA = L.memberA_bytes; ga.memberB = L.memberB_bytes;
  ga.planeA = L.planeA_bytes; ga.planeB = L.planeB_bytes;
  ga.outplane = L.outplane_bytes;
  // 128-column (narrow) and 128 x 128 (small) tiles run two groups per CU;
  // their column tiles past N hold only padding and are not launched.
  const bool narrow = L.gemm_tile_cols == 128;
  const bool small = narrow && L.gemm_tile_rows == 128;
  // Wide tiles whose last tile column holds at most 128 columns of N: that
  // column runs 128-column tiles in the same launch.
  const bool mixed = use_mixed_tiles(L);
  ga.TM = small ? (int)((c.M + 127) / 128) : (int)(L.chunk_rows / kTileR);
  ga.TN = narrow ? (int)((c.N + 127) / 128) : (int)(L.Np / kTileR);
  ga.NB = L.Np / 64;
  ga.P = c.P; ga.ncorr = L.ncorr; ga.nslots = c.P + L.ncorr; ga.batch = (int)c.batch;
  ga.ksplit = L.ksplit;
  ga.run = L.gemm_run;
  // One run of every residue slot per tile, and a fused correction slot: the
  // run starts with the correction slot (one group per tile).
  ga.corr_run = (ga.run > 1 && ga.run == c.P && L.ncorr == 1) ? 1 : 0;
  for (int t = 0; t < kMaxP; ++t) { ga.p[t] = tab.p[t]; ga.invp[t] = tab.invp[t]; }
  // Work items per tile: the correction slots, then the residue slots in runs.
  const int64_t vslots = ga.corr_run ? 1 : L.ncorr + (c.P + ga.run - 1) / ga.run;
  ga.total = vslots * c.batch * L.ksplit * ga.TM * ga.TN;
  // Split streams: g.total counts the K-deep units (the correction products
  // as two slots: ncorr is 2), which 256 groups share; extra columns (a last
  // tile column of at most kXMax columns) ride on the last wide tile column.
  ga.xcols = L.gemm_split ? split_extra_cols(L) : 0;
  if (ga.xcols) ga.TN -= 1;
  if (L.gemm_split) ga.total = (int64_t)ga.nslots * c.batch * ga.TM * ga.TN;
  // 256 x 256 tiles one slot per item of at most kStreamMaxSteps k-steps, no
  // K-split, at least two items per CU: groups of kStreamChain items, each
  // run as one stream (modgemm_tile's kStream), instead of one group per item.
  const bool stream = !L.deep && ga.run == 1 && !narrow && !mixed && L.ksplit == 1 &&
                      ga.total >= 2 * kCUs && L.Kp / kTileK <= kStreamMaxSteps;
  ga.chain = kStreamChain;

  {
    // A dispatch holds its grid size in work-items as 32 bits: every launch
    // below, sized as it will be launched, is checked before the first one.
    const int64_t limit = (int64_t)0xFFFFFFFFu / kThreads;
    int64_t kslab; int nslab;
    slab_split(NF, c.K, &kslab, &nslab);
    // (In groups of kThreads; the single column-sizing launch's groups are
    // kSizeThreads wide.)
    const bool group = MF < kRowsGroupBelow;
    const int64_t sizing =
        !c.b_kn ? (MF + NF < kRowsGroupBelow ? MF + NF : (MF + NF + kRowsPerBlock - 1) / kRowsPerBlock)
        : kslab <= kFusedSlabRows
            ? ((group ? (MF + kSizeThreads / 256 - 1) / (kSizeThreads / 256)
                      : (MF + kSizeThreads / 64 - 1) / (kSizeThreads / 64)) +
               (NF + kSizeThreads / nslab - 1) / (kSizeThreads / nslab)) * (kSizeThreads / kThreads)
            : (group ? MF : (MF + kRowsPerBlock - 1) / kRowsPerBlock) + (NF + kThreads - 1) / kThreads * nslab;
    const int64_t extraction = c.batch * (L.ext_rowsA / 64 + L.ext_rowsB / 64) * (L.Kp / kTileK);
    const int64_t recon = c.batch * ((std::min<int64_t>(L.chunk_rows, c.M) + 15) / 16) * ((c.N + 63) / 64);
    for (int64_t gsz : {sizing, extraction, ga.total, recon})
      if (gsz > limit) return fail(FP64EMU_EINVAL, "problem too large for one launch");
  }

  // 1. sizing
  if (!c.b_kn) {
    launch_size_rows(MF + NF, s, c.A, MF, c.B, c.K, c.bits, sftA, lgA, sftB, lgB);
  } else {
    int64_t kslab; int nslab;
    slab_split(NF, c.K, &kslab, &nslab);
    const bool group = MF < kRowsGroupBelow;
    if (kslab <= kFusedSlabRows) {
      // K > 0 here, so 1 <= nslab <= kMaxSlab and a group holds >= 8 columns.
      const int cpw = kSizeThreads / nslab;
      const int64_t ncolgrp = (NF + cpw - 1) / cpw;
      const int64_t nrow = group ? (MF + kSizeThreads / 256 - 1) / (kSizeThreads / 256)
                                 : (MF + kSizeThreads / 64 - 1) / (kSizeThreads / 64);
      const unsigned grid = (unsigned)(nrow + ncolgrp);
      if (group)
        hipLaunchKernelGGL(size_rows_cols_kernel<true>, dim3(grid), dim3(kSizeThreads), 0, s, c.A, MF,
                           ncolgrp, c.K, c.bits, sftA, lgA, c.B, NF, c.N, kslab, nslab, cpw, sftB, lgB);
      else
        hipLaunchKernelGGL(size_rows_cols_kernel<false>, dim3(grid), dim3(kSizeThreads), 0, s, c.A, MF,
                           ncolgrp, c.K, c.bits, sftA, lgA, c.B, NF, c.N, kslab, nslab, cpw, sftB, lgB);
    } else {
      const int64_t gcx = (NF + kThreads - 1) / kThreads;
      const int64_t nrow = group ? MF : (MF + kRowsPerBlock - 1) / kRowsPerBlock;
      const unsigned grid = (unsigned)(nrow + gcx * nslab);
      const int64_t ncol = gcx * nslab;
      if (group)
        hipLaunchKernelGGL(size_rows_slabs_kernel<true>, dim3(grid), dim3(kThreads), 0, s, c.A, MF, ncol,
                           c.K, c.bits, sftA, lgA, c.B, NF, c.N, kslab, gcx, pmax, pss);
      else
        hipLaunchKernelGGL(size_rows_slabs_kernel<false>, dim3(grid), dim3(kThreads), 0, s, c.A, MF, ncol,
                           c.K, c.bits, sftA, lgA, c.B, NF, c.N, kslab, gcx, pmax, pss);
      hipLaunchKernelGGL(size_cols_final_kernel, dim3((unsigned)((NF + kFinalCols - 1) / kFinalCols)),
                         dim3(kThreads), 0, s, pmax, pss, NF, nslab, c.bits, sftB, lgB);
    }
  }
  const float log2M = std::min(tab.log2M, 126.0f);
  const int64_t ext_groups = c.batch * (L.ext_rowsA / 64 + L.ext_rowsB / 64) * (L.Kp / kTileK);
  const bool pick_in_extract = L.nchunk == 1 && L.nseg == 1 && MF + NF <= kPickInExtractMax &&
                               (MF + NF) * (int64_t)sizeof(float) * ext_groups <= kPickInExtractBytes;
  if (!pick_in_extract)
    hipLaunchKernelGGL(pick_width_kernel, dim3(1), dim3(kPickThreads), 0, s, lgA, MF, lgB, NF, log2M,
                       c.bits, bits_eff);

  // 2-4. Per row chunk of A (one unless the workspace is short) and per K
  // segment (one unless deep): extraction (covering the padded planes
  // entirely, so no memset), every modular GEMM in one launch, then the
  // reconstruction of the chunk's rows.  B's planes are extracted once.
  for (int ci = 0; ci < L.nchunk; ++ci) {
    const int64_t m0 = (int64_t)ci * L.chunk_rows;              // 0 unless chunked (batch 1)
    const int64_t Mc = std::min<int64_t>(L.chunk_rows, c.M - m0);
    const bool with_B = L.nchunk == 1 || ci == 0;
    for (int seg = 0; seg < L.nseg; ++seg) {
      const int64_t k0 = (int64_t)seg * L.kseg;
      const int64_t kc = std::min<int64_t>(L.kseg, c.K - k0);
      const int64_t nkt = round_up(kc, kTileK) / kTileK;
      ExtractCore ea;
      ea.A = c.A + m0 * c.K; ea.B = c.B;
      ea.M = Mc; ea.N = c.N; ea.K = kc; ea.batch = c.batch;
      ea.lda = c.K; ea.k0 = k0;
      ea.b_kn = c.b_kn ? 1 : 0;
      ea.use_corr = c.corr ? 1 : 0;
      ea.nkt = nkt;
      ea.planeA = L.planeA_bytes; ea.planeB = L.planeB_bytes;
      ea.memberA = L.memberA_bytes; ea.memberB = L.memberB_bytes;
      ea.rgA = L.ext_rowsA / 64; ea.rgB = with_B ? L.ext_rowsB / 64 : 0;
      ea.rgA_data = (Mc + 63) / 64; ea.rgB_data = with_B ? (c.N + 63) / 64 : 0;
      ea.div_nkt = make_fastdiv(nkt);
      ea.div_rg[0] = make_fastdiv(ea.rgA_data);
      ea.div_rg[1] = make_fastdiv(ea.rgB_data);
      ea.div_rg[2] = make_fastdiv(ea.rgA - ea.rgA_data);
      ea.div_rg[3] = make_fastdiv(ea.rgB - ea.rgB_data);
      ea.sftA = sftA + m0; ea.sftB = sftB; ea.bits_eff = bits_eff;
      ea.pick = pick_in_extract ? 1 : 0; ea.bits = c.bits; ea.log2M = log2M;
      ea.lgA = lgA; ea.lgB = lgB; ea.nlgA = MF; ea.nlgB = NF; ea.bits_out = bits_eff;
      ea.planesA = planesA; ea.planesB = planesB;
      ea.P = c.P;
      const int64_t wg = c.batch * (ea.rgA + ea.rgB) * nkt;
      if (default_moduli) {
        ExtractArgs<false> ed;
        static_cast<ExtractCore&>(ed) = ea;
        hipLaunchKernelGGL(extract_kernel<true>, dim3((unsigned)wg), dim3(kThreads), 0, s, ed);
      } else {
        ExtractArgs<true> eg;
        static_cast<ExtractCore&>(eg) = ea;
        eg.tab = tab;
        hipLaunchKernelGGL(extract_kernel<false>, dim3((unsigned)wg), dim3(kThreads), 0, s, eg);
      }
      if (c.ev) {
        if (int st = check_hip(hipEventRecord(c.ev[1], s), "hipEventRecord")) return st;
      }
      ga.nkt = (int)nkt;
      ga.first = seg == 0 ? 1 : 0;
      if (L.deep)
        hipLaunchKernelGGL((modgemm_kernel<true, 8, 8>), dim3((unsigned)ga.total), dim3(kThreads), 0, s, ga);
      else if (L.gemm_split && ga.xcols == 1)   // 256 x 256 tiles, K-split 2 (use_split_streams)
        hipLaunchKernelGGL(modgemm_split_x_kernel<1>, dim3(kCUs), dim3(kThreads), 0, s, ga);
      else if (L.gemm_split && ga.xcols == 2)
        hipLaunchKernelGGL(modgemm_split_x_kernel<2>, dim3(kCUs), dim3(kThreads), 0, s, ga);
      else if (L.gemm_split)
        hipLaunchKernelGGL(modgemm_split_kernel, dim3(kCUs), dim3(kThreads), 0, s, ga);
      else if (ga.run > 1)   // 256 x 256 tiles only (use_slot_runs)
        hipLaunchKernelGGL((modgemm_kernel<false, 8, 8, true>), dim3((unsigned)ga.total), dim3(kThreads), 0, s, ga);
      else if (small)
        hipLaunchKernelGGL((modgemm_kernel<false, 4, 4>), dim3((unsigned)ga.total), dim3(kThreads), 0, s, ga);
      else if (narrow)
        hipLaunchKernelGGL((modgemm_kernel<false, 8, 4>), dim3((unsigned)ga.total), dim3(kThreads), 0, s, ga);
      else if (mixed)
        hipLaunchKernelGGL(modgemm_mixed_kernel, dim3((unsigned)ga.total), dim3(kThreads), 0, s, ga);
      else if (stream)   // groups of ga.chain items, each run as one stream
        hipLaunchKernelGGL((modgemm_kernel<false, 8, 8, false, true>),
                           dim3((unsigned)((ga.total + 256 * ga.chain - 1) / (256 * ga.chain) * 256)),
                           dim3(kThreads), 0, s, ga);
      else
        hipLaunchKernelGGL((modgemm_kernel<false, 8, 8>), dim3((unsigned)ga.total), dim3(kThreads), 0, s, ga);
      for (int t = 0; t < c.P && !L.deep; ++t) {
        if ((tab.p[t] & 1) || tab.p[t] == 256) continue;
        const int64_t np = (int64_t)L.ksplit * c.batch;
        const int64_t n = np * (L.outplane_bytes / 16);
        hipLaunchKernelGGL(tie_fix_kernel, dim3((unsigned)std::min<int64_t>((n + kThreads - 1) / kThreads, 4096)),
                           dim3(kThreads), 0, s, res8 + t * L.outplane_bytes, L.outplane_bytes, np,
                           (int64_t)c.P * L.outplane_bytes, tab.p[t]);
      }
    }
    if (c.ev) {
      if (int st = check_hip(hipEventRecord(c.ev[2], s), "hipEventRecord")) return st;
      if (int st = check_hip(hipEventRecord(c.ev[3], s), "hipEventRecord")) return st;
    }

    ReconCore ra;
    ra.res8 = res8; ra.corr = corr;
    ra.res32 = reinterpret_cast<const int32_t*>(res8);
    ra.corr64 = reinterpret_cast<const int64_t*>(corr);
    ra.out = c.out + m0 * c.N;
    ra.sftA = sftA + m0; ra.sftB = sftB; ra.bits_eff = bits_eff;
    ra.M = Mc; ra.N = c.N; ra.batch = c.batch; ra.outplane = L.outplane_bytes;
    ra.NB = L.Np / 64;
    ra.MBv = (Mc + 15) / 16; ra.NBv = (c.N + 63) / 64;
    ra.nblocks = c.batch * ra.MBv * ra.NBv;
    ra.per_div = make_fastdiv(ra.MBv * ra.NBv);
    ra.nbv_div = make_fastdiv(ra.NBv);
    ra.ncorr = L.ncorr;
    ra.ksplit = L.ksplit;
    ra.P = c.P;
    const unsigned grid = (unsigned)ra.nblocks;
    if (L.deep) {
      ReconArgs<true> rg;
      static_cast<ReconCore&>(rg) = ra;
      rg.tab = tab;
      if (c.exact)
        hipLaunchKernelGGL((reconstruct_kernel<true, true, 0, false>), dim3(grid), dim3(kThreads), 0, s, rg);
      else
        hipLaunchKernelGGL((reconstruct_kernel<false, true, 0, false>), dim3(grid), dim3(kThreads), 0, s, rg);
    } else {
      launch_reconstruct(c.exact, c.P, grid, s, ra, tab);
    }
  }
  if (int st = check_hip(hipGetLastError(), "kernel launch")) return st;
  if (c.ev) {
    if (int st = check_hip(hipEventRecord(c.ev[4], s), "hipEventRecord")) return st;
  }
  return FP64EMU_OK;
}

Call make_call(double* out, const double* A, const double* B, int64_t batch, int64_t M,
               int64_t N, int64_t K, bool b_kn, const int32_t* primes, int nprimes, int exact,
               int64_t bits, int use_corr, void* ws, size_t ws_bytes, fp64emu_stream_t stream) {
  Call c;
  c.out = out; c.A = A; c.B = B;
  c.batch = batch; c.M = M; c.N = N; c.K = K;
  c.b_kn = b_kn;
  c.primes = primes; c.P = nprimes;
  c.exact = exact != 0;
  c.bits = (bits < 0 || bits > 1000) ? -1 : (int)bits;
  c.corr = use_corr != 0;
  c.ws = ws; c.ws_bytes = ws_bytes;
  c.stream = reinterpret_cast<hipStream_t>(stream);
  c.ev = nullptr;
  return c;
}

}  // namespace

// ---------------------------------------------------------------------------
// Static scratch of fp64emu_mm_nt_noalloc: each GPU holds its own copy of
// this array for the life of the process.  In host code `scratch` names a
// host-side stand-in, not the device memory: the device address comes from
// hipGetSymbolAddress, once per device (with that device current), and only
// that address is ever passed to kernels.
static __device__ __align__(256) unsigned char scratch[FP64EMU_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

// The current device's address of `scratch` (looked up on its first use).
int scratch_address(void** out) {
  int dev = -1;
  if (int st = check_hip(hipGetDevice(&dev), "hipGetDevice")) return st;
  if (dev < 0 || dev >= kMaxDevices) return fail(FP64EMU_EHIP, "device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    if (int st = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress"))
      return st;
    if (!p) return fail(FP64EMU_EHIP, "hipGetSymbolAddress: null scratch address");
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return FP64EMU_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI

extern "C" {

int fp64emu_maxp(void) { return kMaxP; }

const char* fp64emu_last_error(void) { return g_err.c_str(); }

size_t fp64emu_workspace_size(int64_t batch, int64_t M, int64_t N, int64_t K, int nprimes,
                              int use_corr) {
  if (batch < 0 || M < 0 || N < 0 || K < 0 || nprimes < 1 || nprimes > kMaxP) return 0;
  fp64emu_layout_t L;
  make_layout(batch, M, N, K, nprimes, use_corr != 0, &L);
  return L.total;
}

size_t fp64emu_workspace_size_min(int64_t batch, int64_t M, int64_t N, int64_t K, int nprimes,
                                  int use_corr) {
  if (batch < 0 || M < 0 || N < 0 || K < 0 || nprimes < 1 || nprimes > kMaxP) return 0;
  fp64emu_layout_t L;
  make_layout(batch, M, N, K, nprimes, use_corr != 0, &L, round_up(std::max<int64_t>(M, 1), kTileR) / kTileR);
  return L.total;
}

int fp64emu_layout(int64_t batch, int64_t M, int64_t N, int64_t K, int nprimes, int use_corr,
                   fp64emu_layout_t* out) {
  g_err.clear();
  if (!out) return fail(FP64EMU_EINVAL, "layout output must not be NULL");
  if (batch < 0 || M < 0 || N < 0 || K < 0) return fail(FP64EMU_EINVAL, "shapes must be non-negative");
  if (nprimes < 1 || nprimes > kMaxP) return fail(FP64EMU_EINVAL, "too many primes");
  make_layout(batch, M, N, K, nprimes, use_corr != 0, out);
  return FP64EMU_OK;
}

int fp64emu_mm(double* out, const double* A, const double* B, int64_t M, int64_t N, int64_t K,
               const int32_t* primes, const int32_t* inv, const int64_t* mu, int nprimes,
               int exact, int64_t bits, int use_corr, void* workspace, size_t workspace_bytes,
               fp64emu_stream_t stream) {
  (void)inv; (void)mu;
  g_err.clear();
  return run(make_call(out, A, B, 1, M, N, K, false, primes, nprimes, exact, bits, use_corr,
                       workspace, workspace_bytes, stream));
}

int fp64emu_mm_nt(double* out, const double* A, const double* Bt, int64_t M, int64_t N, int64_t K,
                  const int32_t* primes, const int32_t* inv, const int64_t* mu, int nprimes,
                  int exact, int64_t bits, int use_corr, void* workspace, size_t workspace_bytes,
                  fp64emu_stream_t stream) {
  (void)inv; (void)mu;
  g_err.clear();
  return run(make_call(out, A, Bt, 1, M, N, K, true, primes, nprimes, exact, bits, use_corr,
                       workspace, workspace_bytes, stream));
}

int fp64emu_bmm(double* out, const double* A, const double* B, int64_t batch, int64_t M, int64_t N,
                int64_t K, const int32_t* primes, const int32_t* inv, const int64_t* mu,
                int nprimes, int exact, int64_t bits, int use_corr, void* workspace,
                size_t workspace_bytes, fp64emu_stream_t stream) {
  (void)inv; (void)mu;
  g_err.clear();
  return run(make_call(out, A, B, batch, M, N, K, false, primes, nprimes, exact, bits, use_corr,
                       workspace, workspace_bytes, stream));
}

int fp64emu_bmm_nt(double* out, const double* A, const double* Bt, int64_t batch, int64_t M,
                   int64_t N, int64_t K, const int32_t* primes, const int32_t* inv,
                   const int64_t* mu, int nprimes, int exact, int64_t bits, int use_corr,
                   void* workspace, size_t workspace_bytes, fp64emu_stream_t stream) {
  (void)inv; (void)mu;
  g_err.clear();
  return run(make_call(out, A, Bt, batch, M, N, K, true, primes, nprimes, exact, bits, use_corr,
                       workspace, workspace_bytes, stream));
}

int fp64emu_mm_timed(double* out, float* times, const double* A, const double* B, int64_t M,
                     int64_t N, int64_t K, const int32_t* primes, const int32_t* inv,
                     const int64_t* mu, int nprimes, int exact, int64_t bits, int use_corr,
                     void* workspace, size_t workspace_bytes, fp64emu_stream_t stream) {
  (void)inv; (void)mu;
  g_err.clear();
  if (!times) return fail(FP64EMU_EINVAL, "times must not be NULL");
  Call c = make_call(out, A, B, 1, M, N, K, false, primes, nprimes, exact, bits, use_corr,
                     workspace, workspace_bytes, stream);
  hipEvent_t ev[5];
  int created = 0;
  int st = FP64EMU_OK;
  for (; created < 5; ++created) {
    // Timing-only events: no system-scope fence (cache writeback) on record.
    st = check_hip(hipEventCreateWithFlags(&ev[created], hipEventDisableSystemFence),
                   "hipEventCreate");
    if (st) break;
  }
  if (!st) {
    c.ev = ev;
    st = run(c);
  }
  if (!st) st = check_hip(hipEventSynchronize(ev[4]), "hipEventSynchronize");
  if (!st) {
    for (int i = 0; i < 4 && !st; ++i)
      st = check_hip(hipEventElapsedTime(&times[i], ev[i], ev[i + 1]), "hipEventElapsedTime");
  }
  for (int i = 0; i < created; ++i) (void)hipEventDestroy(ev[i]);
  return st;
}

int fp64emu_mm_nt_events(double* out, const double* A, const double* Bt, int64_t M, int64_t N,
                         int64_t K, const int32_t* primes, const int32_t* inv, const int64_t* mu,
                         int nprimes, int exact, int64_t bits, int use_corr, void* workspace,
                         size_t workspace_bytes, fp64emu_stream_t stream,
                         const fp64emu_event_t* events) {
  (void)inv; (void)mu;
  g_err.clear();
  if (!events) return fail(FP64EMU_EINVAL, "events must not be NULL");
  hipEvent_t ev[5];
  for (int i = 0; i < 5; ++i) {
    if (!events[i]) return fail(FP64EMU_EINVAL, "events must not be NULL");
    ev[i] = reinterpret_cast<hipEvent_t>(events[i]);
  }
  Call c = make_call(out, A, Bt, 1, M, N, K, true, primes, nprimes, exact, bits, use_corr,
                     workspace, workspace_bytes, stream);
  c.ev = ev;
  return run(c);
}

int fp64emu_bmm_nt_events(double* out, const double* A, const double* Bt, int64_t batch, int64_t M,
                          int64_t N, int64_t K, const int32_t* primes, const int32_t* inv,
                          const int64_t* mu, int nprimes, int exact, int64_t bits, int use_corr,
                          void* workspace, size_t workspace_bytes, fp64emu_stream_t stream,
                          const fp64emu_event_t* events) {
  (void)inv; (void)mu;
  g_err.clear();
  if (!events) return fail(FP64EMU_EINVAL, "events must not be NULL");
  hipEvent_t ev[5];
  for (int i = 0; i < 5; ++i) {
    if (!events[i]) return fail(FP64EMU_EINVAL, "events must not be NULL");
    ev[i] = reinterpret_cast<hipEvent_t>(events[i]);
  }
  Call c = make_call(out, A, Bt, batch, M, N, K, true, primes, nprimes, exact, bits, use_corr,
                     workspace, workspace_bytes, stream);
  c.ev = ev;
  return run(c);
}

int fp64emu_mm_nt_noalloc(double* out, const double* A, const double* Bt, int64_t M, int64_t N,
                          int64_t K, const int32_t* primes, const int32_t* inv,
                          const int64_t* mu, int nprimes, int exact, int64_t bits,
                          int use_corr, fp64emu_stream_t stream) {
  (void)inv; (void)mu;
  g_err.clear();
  // Argument checks first, then the size check, both before any HIP call.
  if (int st = validate_primes(primes, nprimes)) return st;
  if (bits < 16 || bits > 53) return fail(FP64EMU_EINVAL, "bits must be in [16, 53]");
  if (M < 0 || N < 0 || K < 0) return fail(FP64EMU_EINVAL, "shapes must be non-negative");
  if (K > kMaxKSingle) return fail(FP64EMU_EINVAL, "K bound for int32 modular GEMM");
  const size_t need = fp64emu_workspace_size_min(1, M, N, K, nprimes, use_corr);
  if (need > FP64EMU_NOALLOC_SCRATCH_BYTES)
    return fail(FP64EMU_EWORKSPACE,
                "problem too large for the static scratch of fp64emu_mm_nt_noalloc: needs " +
                    std::to_string(need) + " bytes, holds " +
                    std::to_string((unsigned long long)FP64EMU_NOALLOC_SCRATCH_BYTES));
  if (M == 0 || N == 0 || K == 0)   // no workspace use: the ordinary entry point's path
    return run(make_call(out, A, Bt, 1, M, N, K, true, primes, nprimes, exact, bits, use_corr,
                         nullptr, 0, stream));
  void* ws = nullptr;
  if (int st = scratch_address(&ws)) return st;
  return run(make_call(out, A, Bt, 1, M, N, K, true, primes, nprimes, exact, bits, use_corr, ws,
                       FP64EMU_NOALLOC_SCRATCH_BYTES, stream));
}

int fp64emu_ddgemm_nt(double* hi, double* lo, const double* A, const double* B, int64_t M,
                      int64_t N, int64_t K, fp64emu_stream_t stream) {
  g_err.clear();
  if (M < 0 || N < 0 || K < 0) return fail(FP64EMU_EINVAL, "shapes must be non-negative");
  if (M == 0 || N == 0) return FP64EMU_OK;
  if (!hi || !lo || !A || !B) return fail(FP64EMU_EINVAL, "null operand pointer");
  const dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16));
  hipLaunchKernelGGL(ddgemm_nt_kernel, grid, dim3(kThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), hi, lo, A, B, M, N, K);
  return check_hip(hipGetLastError(), "ddgemm launch");
}

int fp64emu_probe_mfma(int32_t* acc_out, unsigned long long* clocks, const int8_t* src,
                       int64_t groups, int64_t steps, int mode, fp64emu_stream_t stream) {
  g_err.clear();
  if (!acc_out || !clocks || !src) return fail(FP64EMU_EINVAL, "null probe pointer");
  if (groups < 1 || groups > 65536) return fail(FP64EMU_EINVAL, "probe groups must be in [1, 65536]");
  if (steps < 1) return fail(FP64EMU_EINVAL, "probe steps must be >= 1");
  if (reinterpret_cast<uintptr_t>(src) % 16 || reinterpret_cast<uintptr_t>(acc_out) % 16)
    return fail(FP64EMU_EINVAL, "probe buffers must be 16-byte aligned");
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)groups);
  switch (mode) {
    case 0: hipLaunchKernelGGL(mfma_probe_kernel<0>, grid, dim3(kThreads), 0, s, src, steps, acc_out, clocks); break;
    case 1: hipLaunchKernelGGL(mfma_probe_kernel<1>, grid, dim3(kThreads), 0, s, src, steps, acc_out, clocks); break;
    case 2: hipLaunchKernelGGL(mfma_probe_kernel<2>, grid, dim3(kThreads), 0, s, src, steps, acc_out, clocks); break;
    default: return fail(FP64EMU_EINVAL, "probe mode must be 0, 1 or 2");
  }
  return check_hip(hipGetLastError(), "probe launch");
}

int fp64emu_probe_stream(double* dst, const double* src, int64_t n, int mode,
                         fp64emu_stream_t stream) {
  g_err.clear();
  if (mode < 0 || mode > 2) return fail(FP64EMU_EINVAL, "probe mode must be 0, 1 or 2");
  if (n < 2048 || n % 2) return fail(FP64EMU_EINVAL, "probe length must be even and >= 2048");
  if (!dst || (mode != 1 && !src)) return fail(FP64EMU_EINVAL, "null probe pointer");
  if (reinterpret_cast<uintptr_t>(dst) % 16 || reinterpret_cast<uintptr_t>(src) % 16)
    return fail(FP64EMU_EINVAL, "probe buffers must be 16-byte aligned");
  const int64_t n2 = n / 2;
  // n >= 2048 groups' worth: a read's per-group sums fit in dst.
  const dim3 grid((unsigned)std::min<int64_t>(std::max<int64_t>(n2 / 1024, 1), 4096));
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (mode == 0) hipLaunchKernelGGL(stream_probe_kernel<0>, grid, dim3(kThreads), 0, s, dst, src, n2, 0.0);
  else if (mode == 1) hipLaunchKernelGGL(stream_probe_kernel<1>, grid, dim3(kThreads), 0, s, dst, src, n2, 1.0);
  else hipLaunchKernelGGL(stream_probe_kernel<2>, grid, dim3(kThreads), 0, s, dst, src, n2, 0.0);
  return check_hip(hipGetLastError(), "probe launch");
}

}  // extern "C"
