// gossmx oracle: CPU restatement of gpt-oss-rs's MXFP4 mixture-of-experts path.
//
// TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP path: only
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it. The
// product library (gpt-oss-rs_amd/csrc) never links, loads or calls it.
//
// Every function restates the scalar reference semantics of
// /root/reference/crates/gpt-oss-cpu-kernels and
// /root/reference/crates/gpt-oss-model-runner/src/cpu_runner.rs, with the
// file:line it follows. Compile with -ffp-contract=off and without fast-math:
// the reference's float chains are order-defined and unfused.
//
// Pinning (what checks each function; see tests/test_oracle.py):
//   matmul / layouts / fixtures  - the 12 golden SHA-256 vectors of
//       docs/research/evidence/v0.1.0/mxfp4-{gate-up,down}.json
//   block dots, e8m0, codes, split packing, quantizers - the lib.rs KATs
//   swiglu, stable_top_k, grouping, route_top_k - the cpu_runner.rs and
//       gpt-oss-moe-semantics KATs
//   expf restatement - exhaustive comparison against the host glibc expf
//   bf16 rounding - half 2.7.1 KAT bits (exact-BF16 lane KAT, lib.rs:1834)
//   moe_batch composition - brute-force checks against the pieces above and
//       closed-form invariants (top_k == experts, one-hot routing)
//   x8 AVX2 GEMV baseline lane - bit-identical to the scalar matmul on the
//       golden fixtures
//   dense path (attention, YaRN, KV window, greedy token, model step) - the
//       cpu_runner.rs attention / sink / window / cache / YaRN KATs and the
//       step invariants in tests/test_dense.py (chunked prefill == one step,
//       a covering window == full attention, thread-count independence)
#include <cmath>
#include <cstdint>
#include <cstring>
#include <cstdlib>
#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>
#include <immintrin.h>

namespace {

constexpr int kBlock = 32;        // QUANT_BLOCK_SIZE, lib.rs:33
constexpr int kPacked = 16;       // MXFP4_PACKED_BYTES, lib.rs:34
constexpr int kRecord = 17;       // scale byte + 16 packed bytes, lib.rs:781

enum Status : int {
  OK = 0,
  INVALID_DIMENSIONS = 3,
  NON_FINITE_INPUT = 4,
  UNAVAILABLE_BACKEND = 5,
  NON_FINITE_LOGITS = 8,
};

inline uint32_t f2u(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float u2f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint64_t d2u(double d) { uint64_t u; std::memcpy(&u, &d, 8); return u; }
inline double u2d(uint64_t u) { double d; std::memcpy(&d, &u, 8); return d; }

// half 2.7.1 bf16::from_f32 (round to nearest even; NaN keeps the high
// mantissa bits and is quieted). Used by fp32_to_bf16_roundtrip,
// cpu_runner.rs:3740-3744.
inline uint16_t bf16_bits(float f) {
  uint32_t x = f2u(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
  const uint32_t round_bit = 0x8000u;
  if ((x & round_bit) != 0 && (x & (3 * round_bit - 1)) != 0) return (uint16_t)((x >> 16) + 1);
  return (uint16_t)(x >> 16);
}
inline float bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }
inline float bf16_round(float f) { return bf16_to_f32(bf16_bits(f)); }

// e8m0_scale, lib.rs:957-963.
inline float e8m0_scale(uint8_t s) {
  if (s == 0) return u2f(0x00400000u);
  if (s == 0xff) return u2f(0x7fc00000u);  // f32::NAN
  return u2f((uint32_t)s << 23);
}

// mxfp4_integer, lib.rs:1067-1074: E2M1 values doubled so 0.5 stays integral.
const int8_t kLut2[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
// MXFP4_VALUES, lib.rs:37-39.
const float kE2M1[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                         -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

struct Q8Block { float scale; int8_t values[kBlock]; };            // lib.rs:732-736
struct ResidualQ8Block { Q8Block primary; Q8Block residual; };      // lib.rs:738-742
static_assert(sizeof(Q8Block) == 36, "Q8Block is 36 bytes");
static_assert(sizeof(ResidualQ8Block) == 72, "ResidualQ8Block is 72 bytes");

struct Mxfp4Block { uint8_t scale; uint8_t packed[kPacked]; };      // lib.rs:744-750

// Mxfp4Block::unpack, lib.rs:754-761 (adjacent packing, low nibble first).
inline void unpack(const Mxfp4Block& b, int8_t out[kBlock]) {
  for (int i = 0; i < kPacked; ++i) {
    out[2 * i] = kLut2[b.packed[i] & 0x0f];
    out[2 * i + 1] = kLut2[b.packed[i] >> 4];
  }
}

// mxfp4_adjacent_to_split / mxfp4_split_to_adjacent, lib.rs:906-928.
inline uint8_t adj_code(const uint8_t* adj, int i) { return (i & 1) ? (adj[i / 2] >> 4) : (adj[i / 2] & 0x0f); }
void adjacent_to_split(const uint8_t adj[16], uint8_t split[16]) {
  for (int i = 0; i < 16; ++i) split[i] = (uint8_t)(adj_code(adj, i) | (adj_code(adj, i + 16) << 4));
}
inline uint8_t split_code(const uint8_t* split, int i) { return i < 16 ? (split[i] & 0x0f) : (split[i - 16] >> 4); }
void split_to_adjacent(const uint8_t split[16], uint8_t adj[16]) {
  for (int i = 0; i < 16; ++i) adj[i] = (uint8_t)(split_code(split, 2 * i) | (split_code(split, 2 * i + 1) << 4));
}

// Mxfp4MatrixView::block, lib.rs:810-851. layout 1 = CanonicalAdjacentV1,
// layout 2 = InterleavedSplitX8V2 (complete 8-row groups of 136-byte records,
// rows % 8 tail kept canonical after them).
bool view_block(const uint8_t* data, size_t rows, size_t blocks, int layout, size_t row, size_t block,
                Mxfp4Block* out) {
  if (row >= rows || block >= blocks) return false;
  if (layout == 1) {
    const uint8_t* p = data + (row * blocks + block) * kRecord;
    out->scale = p[0];
    std::memcpy(out->packed, p + 1, kPacked);
    return true;
  }
  if (layout != 2) return false;
  const size_t complete_rows = rows / 8 * 8;
  if (row < complete_rows) {
    const size_t group = row / 8, lane = row % 8;
    const uint8_t* x8 = data + (group * blocks + block) * 136;
    uint8_t split[16];
    for (int i = 0; i < 16; ++i) split[i] = x8[8 + (i / 8) * 64 + lane * 8 + i % 8];
    out->scale = x8[lane];
    split_to_adjacent(split, out->packed);
    return true;
  }
  const size_t tail_row = row - complete_rows;
  const uint8_t* p = data + (rows / 8) * blocks * 136 + (tail_row * blocks + block) * kRecord;
  out->scale = p[0];
  std::memcpy(out->packed, p + 1, kPacked);
  return true;
}

// scalar_max_abs, lib.rs:1045-1049.
float max_abs(const float* v, int n) {
  float m = 0.0f;
  for (int i = 0; i < n; ++i) m = std::fmax(m, std::fabs(v[i]));
  return m;
}

// quantize_q8_block, lib.rs:1051-1065.
Q8Block quantize_q8_block(const float* v, float mx) {
  Q8Block b;
  const float scale = mx / 127.0f;
  const float inv = scale == 0.0f ? 0.0f : 1.0f / scale;
  for (int i = 0; i < kBlock; ++i) {
    float q = std::round(v[i] * inv);
    q = std::min(std::max(q, -127.0f), 127.0f);
    b.values[i] = (int8_t)q;
  }
  b.scale = scale;
  return b;
}

// Kernels::quantize_residual_q8, lib.rs:382-409.
int quantize_residual_q8(const float* in, size_t n, ResidualQ8Block* out) {
  if (n % kBlock) return INVALID_DIMENSIONS;
  for (size_t i = 0; i < n; ++i)
    if (!std::isfinite(in[i])) return NON_FINITE_INPUT;
  for (size_t b = 0; b < n / kBlock; ++b) {
    const float* blk = in + b * kBlock;
    Q8Block primary = quantize_q8_block(blk, max_abs(blk, kBlock));
    float residual[kBlock];
    for (int i = 0; i < kBlock; ++i) residual[i] = blk[i] - (float)primary.values[i] * primary.scale;
    out[b].primary = primary;
    out[b].residual = quantize_q8_block(residual, max_abs(residual, kBlock));
  }
  return OK;
}

// Kernels::quantize_q8, lib.rs:347-378.
int quantize_q8(const float* in, size_t n, Q8Block* out) {
  if (n % kBlock) return INVALID_DIMENSIONS;
  for (size_t i = 0; i < n; ++i)
    if (!std::isfinite(in[i])) return NON_FINITE_INPUT;
  for (size_t b = 0; b < n / kBlock; ++b) out[b] = quantize_q8_block(in + b * kBlock, max_abs(in + b * kBlock, kBlock));
  return OK;
}

// scalar_bf16_dot, lib.rs:1007-1029: 16 fixed reduction lanes, mul then add,
// lanes folded 0..15 in order.
float bf16_dot(const uint16_t* a, const uint16_t* b, size_t n) {
  float lanes[16] = {0};
  size_t i = 0;
  for (; i + 16 <= n; i += 16)
    for (int l = 0; l < 16; ++l) lanes[l] += bf16_to_f32(a[i + l]) * bf16_to_f32(b[i + l]);
  for (int l = 0; i < n; ++i, ++l) lanes[l] += bf16_to_f32(a[i]) * bf16_to_f32(b[i]);
  float s = -0.0f;
  for (int l = 0; l < 16; ++l) s += lanes[l];
  return s;
}

// scalar_sum_squares + Kernels::rms_norm, lib.rs:699-730, 1031-1043.
void rms_norm(const float* in, const float* w, size_t n, float eps, float* out) {
  float lanes[16] = {0};
  size_t i = 0;
  for (; i + 16 <= n; i += 16)
    for (int l = 0; l < 16; ++l) lanes[l] += in[i + l] * in[i + l];
  for (int l = 0; i < n; ++i, ++l) lanes[l] += in[i] * in[i];
  float ss = -0.0f;
  for (int l = 0; l < 16; ++l) ss += lanes[l];
  const float inv = 1.0f / std::sqrt(ss / (float)n + eps);
  for (size_t k = 0; k < n; ++k) out[k] = in[k] * inv * w[k];
}

// Restatement of glibc 2.35 expf (sysdeps/ieee754/flt-32/e_expf.c, the
// ARM optimized-routines algorithm by Szabolcs Nagy: N=32 table of 2^(i/N)
// in double, degree-3 polynomial, round-to-int by the 0x1.8p52 shift), as
// built by the x86_64 FMA multiarch variant (the one selected on every host
// with FMA). The table is 2^(i/32) rounded to double, stored with i<<47
// subtracted from its bits. Pinned against the host glibc expf on all 2^32
// inputs (tests/test_oracle.py::test_expf_restatement_matches_glibc).
struct ExpfTable {
  uint64_t t[32];
  ExpfTable() {
    for (int i = 0; i < 32; ++i) {
      long double v = exp2l((long double)i / 32.0L);
      t[i] = d2u((double)v) - ((uint64_t)i << 47);
    }
  }
};
const ExpfTable kExpfTable;

float expf_restated(float x) {
  const uint32_t abstop = (f2u(x) >> 20) & 0x7ff;
  if (abstop >= ((f2u(88.0f) >> 20) & 0x7ff)) {
    if (f2u(x) == f2u(-INFINITY)) return 0.0f;
    if (abstop >= ((f2u(INFINITY) >> 20) & 0x7ff)) return x + x;
    if (x > 0x1.62e42ep6f) return INFINITY;
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double inv_ln2_n = 0x1.71547652b82fep+0 * 32;
  const double shift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
  const double xd = (double)x;
  double kd = std::fma(inv_ln2_n, xd, shift);
  const uint64_t ki = d2u(kd);
  kd -= shift;
  const double r = std::fma(inv_ln2_n, xd, -kd);
  const uint64_t t = kExpfTable.t[ki % 32] + (ki << 47);
  const double s = u2d(t);
  const double z = std::fma(c0, r, c1);
  const double r2 = r * r;
  double y = std::fma(c2, r, 1.0);
  y = std::fma(z, r2, y);
  y = y * s;
  return (float)y;
}

// gpt_oss_swiglu, cpu_runner.rs:3797-3826. Uses the host libm expf, which is
// what Rust's f32::exp lowers to on x86_64 Linux.
float swiglu_one(float g, float u, float alpha, float limit) {
  const float gate = std::fmin(g, limit);  // f32::min ignores NaN like fminf
  float up = u;                            // f32::clamp keeps NaN
  if (up < -limit) up = -limit;
  if (up > limit) up = limit;
  const float scaled = bf16_round(gate * alpha);
  const float sig = bf16_round(1.0f / (1.0f + expf(-scaled)));
  const float glu = bf16_round(gate * sig);
  const float lin = bf16_round(up + 1.0f);
  return bf16_round(glu * lin);
}

// stable_top_k, cpu_runner.rs:3768-3778 (descending by value, ties to the
// lower index). Non-finite values are rejected by the caller first.
void stable_top_k(const float* v, size_t n, size_t k, uint32_t* out) {
  std::vector<uint32_t> idx(n);
  for (size_t i = 0; i < n; ++i) idx[i] = (uint32_t)i;
  std::stable_sort(idx.begin(), idx.end(), [&](uint32_t a, uint32_t b) {
    if (v[a] > v[b]) return true;
    if (v[a] < v[b]) return false;
    return a < b;
  });
  for (size_t i = 0; i < std::min(k, n); ++i) out[i] = idx[i];
}

// softmax, cpu_runner.rs:3784-3795.
void softmax(const float* v, size_t n, float* out) {
  float mx = -INFINITY;
  for (size_t i = 0; i < n; ++i) mx = std::fmax(mx, v[i]);
  float denom = -0.0f;
  for (size_t i = 0; i < n; ++i) { out[i] = expf(v[i] - mx); denom += out[i]; }
  for (size_t i = 0; i < n; ++i) out[i] = out[i] / denom;
}

// scalar_matmul_range, matmul.rs:529-578 (also the M==1 gemv float contract of
// mxfp4_residual_q8_gemv_rows, lib.rs:673-696: bias, then per block the
// primary term then the residual term).
struct MatmulArgs {
  const uint8_t* weights; size_t rows; size_t blocks; int layout;
  int kind;  // 1 = Q8, 2 = ResidualQ8
  const void* act; size_t m; size_t act_stride;
  const float* bias;
  float* out; size_t out_stride;
};

void scalar_matmul_rows(const MatmulArgs& a, size_t in_lo, size_t in_hi, size_t out_lo, size_t out_hi) {
  int8_t w[kBlock];
  for (size_t r = in_lo; r < in_hi; ++r) {
    for (size_t o = out_lo; o < out_hi; ++o) {
      float total = a.bias ? a.bias[o] : 0.0f;
      for (size_t b = 0; b < a.blocks; ++b) {
        Mxfp4Block blk;
        view_block(a.weights, a.rows, a.blocks, a.layout, o, b, &blk);
        unpack(blk, w);
        if (a.kind == 1) {
          const Q8Block& q = static_cast<const Q8Block*>(a.act)[r * a.act_stride + b];
          int32_t s = 0;
          for (int k = 0; k < kBlock; ++k) s += (int32_t)w[k] * (int32_t)q.values[k];
          total += (float)s * 0.5f * e8m0_scale(blk.scale) * q.scale;
        } else {
          const ResidualQ8Block& q = static_cast<const ResidualQ8Block*>(a.act)[r * a.act_stride + b];
          int32_t p = 0, e = 0;
          for (int k = 0; k < kBlock; ++k) {
            p += (int32_t)w[k] * (int32_t)q.primary.values[k];
            e += (int32_t)w[k] * (int32_t)q.residual.values[k];
          }
          const float ws = 0.5f * e8m0_scale(blk.scale);
          total += (float)p * ws * q.primary.scale;
          total += (float)e * ws * q.residual.scale;
        }
      }
      a.out[r * a.out_stride + o] = total;
    }
  }
}

// Mxfp4MatmulProblem::new validation, matmul.rs:339-369, plus the view
// checks of Mxfp4MatrixView::new (lib.rs:774-796) and
// validate_activation_extent (matmul.rs:245-267).
int validate_matmul(size_t data_len, size_t rows, size_t blocks, int layout, int kind, size_t act_len, size_t m,
                    size_t act_bpr, size_t act_stride, size_t bias_len, bool has_bias, size_t out_len,
                    size_t out_stride) {
  if (rows == 0 || blocks == 0 || data_len != rows * blocks * kRecord) return INVALID_DIMENSIONS;
  if (layout != 1 && layout != 2) return INVALID_DIMENSIONS;
  if (kind != 1 && kind != 2) return INVALID_DIMENSIONS;
  if (m == 0 || act_bpr == 0 || act_stride < act_bpr || (m - 1) * act_stride + act_bpr > act_len)
    return INVALID_DIMENSIONS;
  if (act_bpr != blocks || out_stride < rows || (m - 1) * out_stride + rows > out_len) return INVALID_DIMENSIONS;
  if (has_bias && bias_len != rows) return INVALID_DIMENSIONS;
  return OK;
}

// ---------------------------------------------------------------------------
// Baseline lane: the reference's Auto path for M == 1 on AVX2 hosts, the x8
// residual-Q8 GEMV (x86.rs:332-370 over pack_x8 weights, dispatch at
// lib.rs:236-295 and matmul.rs:429-455). Written from the algorithm: per
// 8-row group and K block, the eight exact integer dots, then the float chain
// ((int * 0.5) * e8m0) * act_scale added to an 8-wide accumulator seeded with
// the bias, primary then residual. Bit-identical to the scalar chain.
__attribute__((target("avx2")))
void x8_dots_avx2(const uint8_t* x8, const int8_t* primary, const int8_t* residual, int32_t pd[8], int32_t rd[8]) {
  // x8 record: 8 scales, then chunk c (0..1) x lane (0..7) x 8 split bytes.
  // split byte i holds code(i) in the low nibble and code(i + 16) high.
  const __m128i lut = _mm_setr_epi8(0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12);
  const __m128i mask = _mm_set1_epi8(0x0f);
  for (int lane = 0; lane < 8; ++lane) {
    // Gather this row's 16 split bytes (8 from each chunk).
    const __m128i lo8 = _mm_loadl_epi64((const __m128i*)(x8 + 8 + lane * 8));
    const __m128i hi8 = _mm_loadl_epi64((const __m128i*)(x8 + 8 + 64 + lane * 8));
    const __m128i split = _mm_unpacklo_epi64(lo8, hi8);
    const __m128i first = _mm_shuffle_epi8(lut, _mm_and_si128(split, mask));                      // codes 0..15
    const __m128i second = _mm_shuffle_epi8(lut, _mm_and_si128(_mm_srli_epi16(split, 4), mask));  // codes 16..31
    const __m256i w = _mm256_set_m128i(second, first);
    const __m256i w_lo = _mm256_cvtepi8_epi16(_mm256_castsi256_si128(w));
    const __m256i w_hi = _mm256_cvtepi8_epi16(_mm256_extracti128_si256(w, 1));
    const __m256i p = _mm256_loadu_si256((const __m256i*)primary);
    __m256i acc = _mm256_add_epi32(_mm256_madd_epi16(w_lo, _mm256_cvtepi8_epi16(_mm256_castsi256_si128(p))),
                                   _mm256_madd_epi16(w_hi, _mm256_cvtepi8_epi16(_mm256_extracti128_si256(p, 1))));
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(acc), _mm256_extracti128_si256(acc, 1));
    s = _mm_hadd_epi32(s, s);
    s = _mm_hadd_epi32(s, s);
    pd[lane] = _mm_cvtsi128_si32(s);
    if (residual) {
      const __m256i r = _mm256_loadu_si256((const __m256i*)residual);
      acc = _mm256_add_epi32(_mm256_madd_epi16(w_lo, _mm256_cvtepi8_epi16(_mm256_castsi256_si128(r))),
                             _mm256_madd_epi16(w_hi, _mm256_cvtepi8_epi16(_mm256_extracti128_si256(r, 1))));
      s = _mm_add_epi32(_mm256_castsi256_si128(acc), _mm256_extracti128_si256(acc, 1));
      s = _mm_hadd_epi32(s, s);
      s = _mm_hadd_epi32(s, s);
      rd[lane] = _mm_cvtsi128_si32(s);
    }
  }
}

__attribute__((target("avx2")))
void x8_gemv_group_avx2(const uint8_t* x8_data, size_t blocks, size_t group, const ResidualQ8Block* act,
                        const float* bias8, float* out8) {
  __m256 accum = _mm256_loadu_ps(bias8);
  const __m256 half = _mm256_set1_ps(0.5f);
  for (size_t b = 0; b < blocks; ++b) {
    const uint8_t* rec = x8_data + (group * blocks + b) * 136;
    int32_t pd[8], rd[8];
    x8_dots_avx2(rec, act[b].primary.values, act[b].residual.values, pd, rd);
    float sc[8];
    for (int l = 0; l < 8; ++l) sc[l] = e8m0_scale(rec[l]);
    const __m256 ws = _mm256_loadu_ps(sc);
    __m256 c = _mm256_cvtepi32_ps(_mm256_loadu_si256((const __m256i*)pd));
    c = _mm256_mul_ps(_mm256_mul_ps(_mm256_mul_ps(c, half), ws), _mm256_set1_ps(act[b].primary.scale));
    accum = _mm256_add_ps(accum, c);
    c = _mm256_cvtepi32_ps(_mm256_loadu_si256((const __m256i*)rd));
    c = _mm256_mul_ps(_mm256_mul_ps(_mm256_mul_ps(c, half), ws), _mm256_set1_ps(act[b].residual.scale));
    accum = _mm256_add_ps(accum, c);
  }
  _mm256_storeu_ps(out8, accum);
}

bool host_has_avx2() { return __builtin_cpu_supports("avx2"); }

// Auto lane for one residual-Q8 problem (matmul.rs:398-414 with
// resolved_for_rows, matmul.rs:51-57): M == 1 with a bias on x8 weights takes
// the x8 GEMV for complete groups and the scalar rows for the tail; otherwise
// the scalar matmul. `threads` > 1 spreads 8-row tiles over threads the way
// project_mxfp4 spreads them over rayon (cpu_runner.rs:3465-3496).
void auto_matmul(const MatmulArgs& a, int threads) {
  const bool gemv = a.m == 1 && a.bias && a.layout == 2 && a.kind == 2 && host_has_avx2();
  const size_t groups = a.rows / 8;
  auto work = [&](size_t g_lo, size_t g_hi) {
    for (size_t g = g_lo; g < g_hi; ++g) {
      if (gemv)
        x8_gemv_group_avx2(a.weights, a.blocks, g, static_cast<const ResidualQ8Block*>(a.act), a.bias + g * 8,
                           a.out + g * 8);
      else
        scalar_matmul_rows(a, 0, a.m, g * 8, g * 8 + 8);
    }
  };
  if (threads <= 1 || groups < 2) {
    work(0, groups);
  } else {
    std::vector<std::thread> pool;
    std::atomic<size_t> next{0};
    for (int t = 0; t < threads; ++t)
      pool.emplace_back([&] {
        for (;;) {
          size_t g = next.fetch_add(1);
          if (g >= groups) break;
          work(g, g + 1);
        }
      });
    for (auto& th : pool) th.join();
  }
  if (groups * 8 != a.rows) scalar_matmul_rows(a, 0, a.m, groups * 8, a.rows);
}

// ---------------------------------------------------------------------------
// The reference's forced multi-row lanes (Mxfp4MatmulBackend::Avx2 and
// ::Avx512Vnni): avx2_matmul / avx512_vnni_matmul (matmul.rs:829-961) over
// mxfp4_matmul_x8_avx2 / _avx512_vnni (x86.rs:449-520, 660-732). Input rows
// go in panels of P (4 for AVX2, 8 for AVX-512); per complete 8-output x8
// group the panel rows start from the bias (or +0.0), and per K block the
// eight exact integer dots of every panel row are taken from the block's
// decoded weights, then each row adds ((dot * 0.5) * e8m0) * act_scale,
// primary then residual. The output-row tail (n % 8) takes the scalar rows.
// Integer dots are exact in any order, so the dots here are this restatement's
// own: the block's eight weight rows are widened to 16 bits once and reused
// by every panel row (the reference decodes each x8 chunk once per panel too),
// then 16-bit multiply-adds (256-bit on the AVX2 lane, 512-bit on the
// AVX-512 lane; the reference's AVX-512 lane uses VNNI); the float chain is
// the reference's.

// The 32 LUT integers (2 x E2M1) of each of the eight rows of an x8 record:
// w[row][k], codes k = 0..31 of the block.
void x8_decode(const uint8_t* rec, int16_t w[8][32]) {
  static const int16_t lut[16] = {0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
  for (int lane = 0; lane < 8; ++lane)
    for (int c = 0; c < 2; ++c)
      for (int i = 0; i < 8; ++i) {
        const uint8_t b = rec[8 + c * 64 + lane * 8 + i];  // split byte 8c + i: code(8c + i) | code(8c + i + 16) << 4
        w[lane][8 * c + i] = lut[b & 0x0f];
        w[lane][8 * c + i + 16] = lut[b >> 4];
      }
}

// The eight 8-lane partial-sum vectors s[o] reduced to one vector of eight sums.
__attribute__((target("avx2")))
inline __m256i reduce8(const __m256i s[8]) {
  const __m256i s01 = _mm256_hadd_epi32(s[0], s[1]), s23 = _mm256_hadd_epi32(s[2], s[3]);
  const __m256i s45 = _mm256_hadd_epi32(s[4], s[5]), s67 = _mm256_hadd_epi32(s[6], s[7]);
  const __m256i s0123 = _mm256_hadd_epi32(s01, s23), s4567 = _mm256_hadd_epi32(s45, s67);
  return _mm256_add_epi32(_mm256_permute2x128_si256(s0123, s4567, 0x20),
                          _mm256_permute2x128_si256(s0123, s4567, 0x31));
}

__attribute__((target("avx2")))
void panel_dots_avx2(const int16_t w[8][32], const int8_t* act, int32_t d[8]) {
  const __m256i a = _mm256_loadu_si256((const __m256i*)act);
  const __m256i a_lo = _mm256_cvtepi8_epi16(_mm256_castsi256_si128(a));
  const __m256i a_hi = _mm256_cvtepi8_epi16(_mm256_extracti128_si256(a, 1));
  __m256i sums[8];
  for (int o = 0; o < 8; ++o)
    sums[o] = _mm256_add_epi32(_mm256_madd_epi16(_mm256_loadu_si256((const __m256i*)w[o]), a_lo),
                               _mm256_madd_epi16(_mm256_loadu_si256((const __m256i*)(w[o] + 16)), a_hi));
  _mm256_storeu_si256((__m256i*)d, reduce8(sums));
}

__attribute__((target("avx2,avx512f,avx512bw,avx512vl")))
void panel_dots_avx512(const int16_t w[8][32], const int8_t* act, int32_t d[8]) {
  const __m512i a = _mm512_cvtepi8_epi16(_mm256_loadu_si256((const __m256i*)act));
  __m256i sums[8];
  for (int o = 0; o < 8; ++o) {
    const __m512i p = _mm512_madd_epi16(_mm512_loadu_si512(w[o]), a);
    sums[o] = _mm256_add_epi32(_mm512_castsi512_si256(p), _mm512_extracti64x4_epi64(p, 1));
  }
  _mm256_storeu_si256((__m256i*)d, reduce8(sums));
}

bool host_has_avx512_vnni() {
  return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
         __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512vnni");
}

// One 8-output group of the panel lane for panel rows [r0, r0 + rows).
void panel_group(const MatmulArgs& a, size_t group, size_t r0, size_t rows, bool avx512) {
  const bool residual = a.kind == 2;
  float acc[8][8];
  for (size_t r = 0; r < rows; ++r)
    for (int o = 0; o < 8; ++o) acc[r][o] = a.bias ? a.bias[group * 8 + o] : 0.0f;
  alignas(64) int16_t w[8][32];
  for (size_t b = 0; b < a.blocks; ++b) {
    const uint8_t* rec = a.weights + (group * a.blocks + b) * 136;
    x8_decode(rec, w);
    float ws[8];
    for (int o = 0; o < 8; ++o) ws[o] = e8m0_scale(rec[o]);
    for (size_t r = 0; r < rows; ++r) {
      const size_t i = (r0 + r) * a.act_stride + b;
      const int8_t* pv;
      float ps;
      const int8_t* rv = nullptr;
      float rs = 0.0f;
      if (residual) {
        const ResidualQ8Block& blk = static_cast<const ResidualQ8Block*>(a.act)[i];
        pv = blk.primary.values;
        ps = blk.primary.scale;
        rv = blk.residual.values;
        rs = blk.residual.scale;
      } else {
        const Q8Block& blk = static_cast<const Q8Block*>(a.act)[i];
        pv = blk.values;
        ps = blk.scale;
      }
      int32_t pd[8], rd[8];
      if (avx512) panel_dots_avx512(w, pv, pd);
      else panel_dots_avx2(w, pv, pd);
      if (residual) {
        if (avx512) panel_dots_avx512(w, rv, rd);
        else panel_dots_avx2(w, rv, rd);
      }
      for (int o = 0; o < 8; ++o) {
        float c = (((float)pd[o] * 0.5f) * ws[o]) * ps;
        acc[r][o] = acc[r][o] + c;
        if (residual) {
          c = (((float)rd[o] * 0.5f) * ws[o]) * rs;
          acc[r][o] = acc[r][o] + c;
        }
      }
    }
  }
  for (size_t r = 0; r < rows; ++r)
    for (int o = 0; o < 8; ++o) a.out[(r0 + r) * a.out_stride + group * 8 + o] = acc[r][o];
}

// lane 4: AVX2 4x8 panels; lane 8: AVX-512/VNNI 8x8 panels. x8 layout only.
// threads > 1 spreads (panel, group) units over threads (the forced lanes of
// the reference run one thread per problem).
void panel_matmul(const MatmulArgs& a, int lane, int threads) {
  const size_t P = lane == 8 ? 8 : 4, groups = a.rows / 8, panels = (a.m + P - 1) / P;
  const bool avx512 = lane == 8;
  auto unit = [&](size_t u) {
    const size_t panel = u / std::max<size_t>(groups, 1), g = u % std::max<size_t>(groups, 1);
    const size_t r0 = panel * P, rows = std::min(P, a.m - r0);
    panel_group(a, g, r0, rows, avx512);
  };
  const size_t units = panels * groups;
  if (threads <= 1 || units < 2) {
    for (size_t u = 0; u < units; ++u) unit(u);
  } else {
    std::vector<std::thread> pool;
    std::atomic<size_t> next{0};
    for (int t = 0; t < threads; ++t)
      pool.emplace_back([&] {
        for (;;) {
          const size_t u = next.fetch_add(1);
          if (u >= units) break;
          unit(u);
        }
      });
    for (auto& th : pool) th.join();
  }
  if (groups * 8 != a.rows) scalar_matmul_rows(a, 0, a.m, groups * 8, a.rows);
}

// ---------------------------------------------------------------------------
// Deterministic synthetic data (shared with the GPU library's generator).
inline uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
inline uint64_t stream_hash(uint64_t seed, uint64_t stream, uint64_t index) {
  return splitmix64(splitmix64(seed ^ (stream * 0xD1B54A32D192ED03ull)) + index);
}

}  // namespace

// ===========================================================================
// C ABI for the Python test harness (ctypes).
extern "C" {

uint16_t oracle_bf16_bits(float f) { return bf16_bits(f); }
float oracle_e8m0_scale(uint8_t s) { return e8m0_scale(s); }
float oracle_decode_mxfp4(uint8_t code) { return kE2M1[code & 0x0f]; }
int32_t oracle_mxfp4_integer(uint8_t code) { return kLut2[code & 0x0f]; }
float oracle_expf_glibc(float x) { return expf(x); }
float oracle_expf_restated(float x) { return expf_restated(x); }

void oracle_adjacent_to_split(const uint8_t* adj, uint8_t* split) { adjacent_to_split(adj, split); }
void oracle_split_to_adjacent(const uint8_t* split, uint8_t* adj) { split_to_adjacent(split, adj); }

// Exhaustive check of expf_restated against the host glibc expf over the
// float bit patterns [lo, hi]; returns the number of mismatching inputs
// (NaN inputs skipped) and the first one in *first.
uint64_t oracle_expf_check(uint32_t lo, uint32_t hi, int threads, uint32_t* first) {
  if (threads < 1) threads = 1;
  std::vector<uint64_t> bad(threads, 0);
  std::vector<uint32_t> fst(threads, 0);
  std::vector<std::thread> pool;
  const uint64_t n = (uint64_t)hi - lo + 1;
  for (int t = 0; t < threads; ++t)
    pool.emplace_back([&, t] {
      const uint64_t a = lo + n * t / threads, b = lo + n * (t + 1) / threads;
      for (uint64_t u = a; u < b; ++u) {
        const float x = u2f((uint32_t)u);
        if (std::isnan(x)) continue;
        if (f2u(expf(x)) != f2u(expf_restated(x))) {
          if (!bad[t]) fst[t] = (uint32_t)u;
          ++bad[t];
        }
      }
    });
  for (auto& th : pool) th.join();
  uint64_t total = 0;
  *first = 0;
  for (int t = 0; t < threads; ++t) {
    if (bad[t] && !total) *first = fst[t];
    total += bad[t];
  }
  return total;
}

int oracle_quantize_residual_q8(const float* in, size_t n, void* out) {
  return quantize_residual_q8(in, n, static_cast<ResidualQ8Block*>(out));
}
int oracle_quantize_q8(const float* in, size_t n, void* out) { return quantize_q8(in, n, static_cast<Q8Block*>(out)); }

// Exact integer block dots (scalar_mxfp4_residual_q8_dot_i32, lib.rs:1085-1098)
// for every (row, block) of a canonical matrix against one activation row.
void oracle_block_dots(const uint8_t* canonical, size_t rows, size_t blocks, const void* act, int32_t* out) {
  const ResidualQ8Block* q = static_cast<const ResidualQ8Block*>(act);
  int8_t w[kBlock];
  for (size_t r = 0; r < rows; ++r)
    for (size_t b = 0; b < blocks; ++b) {
      Mxfp4Block blk;
      view_block(canonical, rows, blocks, 1, r, b, &blk);
      unpack(blk, w);
      int32_t p = 0, e = 0;
      for (int k = 0; k < kBlock; ++k) {
        p += (int32_t)w[k] * q[b].primary.values[k];
        e += (int32_t)w[k] * q[b].residual.values[k];
      }
      out[(r * blocks + b) * 2] = p;
      out[(r * blocks + b) * 2 + 1] = e;
    }
}

// Kernels::mxfp4_matmul with the Scalar backend (matmul.rs:398-414,
// 529-578). Validation failures leave the output untouched.
int oracle_mxfp4_matmul(const uint8_t* data, size_t data_len, size_t rows, size_t blocks, int layout, int kind,
                        const void* act, size_t act_len, size_t m, size_t act_bpr, size_t act_stride,
                        const float* bias, size_t bias_len, float* out, size_t out_len, size_t out_stride) {
  int st = validate_matmul(data_len, rows, blocks, layout, kind, act_len, m, act_bpr, act_stride, bias_len,
                           bias != nullptr, out_len, out_stride);
  if (st) return st;
  MatmulArgs a{data, rows, blocks, layout, kind, act, m, act_stride, bias, out, out_stride};
  scalar_matmul_rows(a, 0, m, 0, rows);
  return OK;
}

// The Auto lane (x8 GEMV for M == 1, scalar otherwise), optionally spread over
// threads. Residual-Q8 only (the serving default, cpu_runner.rs:49-90).
int oracle_mxfp4_matmul_auto(const uint8_t* data, size_t rows, size_t blocks, int layout, const void* act, size_t m,
                             const float* bias, float* out, size_t out_stride, int threads) {
  MatmulArgs a{data, rows, blocks, layout, 2, act, m, blocks, bias, out, out_stride};
  auto_matmul(a, threads);
  return OK;
}

int oracle_has_avx2() { return host_has_avx2() ? 1 : 0; }
int oracle_has_avx512_vnni() { return host_has_avx512_vnni() ? 1 : 0; }

// The forced panel lanes on x8 weights: lane 4 (AVX2 4x8) or 8 (AVX-512/VNNI
// 8x8); kind 1 (Q8) or 2 (residual-Q8).
int oracle_mxfp4_matmul_lane(const uint8_t* data, size_t rows, size_t blocks, int kind, const void* act, size_t m,
                             const float* bias, float* out, size_t out_stride, int lane, int threads) {
  if ((lane != 4 && lane != 8) || (kind != 1 && kind != 2)) return INVALID_DIMENSIONS;
  if (lane == 4 && !host_has_avx2()) return UNAVAILABLE_BACKEND;
  if (lane == 8 && !host_has_avx512_vnni()) return UNAVAILABLE_BACKEND;
  MatmulArgs a{data, rows, blocks, 2, kind, act, m, blocks, bias, out, out_stride};
  panel_matmul(a, lane, threads);
  return OK;
}

// Fixture generators of mxfp4_matrix_bench.rs:524-570 (make_weights, make_q8,
// make_residual, make_bias) and pack_x8 (:572-597).
void oracle_bench_weights(size_t rows, size_t blocks, uint8_t* canonical) {
  for (size_t index = 0; index < rows * blocks; ++index) {
    uint8_t* rec = canonical + index * kRecord;
    rec[0] = index % 127 == 0 ? 0 : (uint8_t)(124 + index % 7);
    for (size_t byte = 0; byte < kPacked; ++byte)
      rec[1 + byte] = (uint8_t)(((index * 13 + byte * 7) & 0x0f) | (((index * 5 + byte * 11 + 3) & 0x0f) << 4));
  }
}
void oracle_bench_residual(size_t rows, size_t blocks, void* out) {
  ResidualQ8Block* q = static_cast<ResidualQ8Block*>(out);
  for (size_t index = 0; index < rows * blocks; ++index) {
    Q8Block p;
    p.scale = 0.0005f + (float)(index % 251) * 0.000001f;
    for (size_t lane = 0; lane < kBlock; ++lane) p.values[lane] = (int8_t)((int)((index * 31 + lane * 17) % 255) - 127);
    Q8Block r;
    r.scale = p.scale / 127.0f;
    for (size_t lane = 0; lane < kBlock; ++lane) r.values[lane] = (int8_t)((int)((index + lane * 3) % 15) - 7);
    q[index].primary = p;
    q[index].residual = r;
  }
}
void oracle_bench_bias(size_t rows, float* bias) {
  for (size_t i = 0; i < rows; ++i) bias[i] = (float)i * 0.00003125f - 0.25f;
}
void pack_x8_groups(const uint8_t* canonical, size_t blocks, uint8_t* out, size_t g_lo, size_t g_hi) {
  for (size_t g = g_lo; g < g_hi; ++g)
    for (size_t b = 0; b < blocks; ++b) {
      uint8_t* p = out + (g * blocks + b) * 136;
      for (size_t lane = 0; lane < 8; ++lane) *p++ = canonical[((g * 8 + lane) * blocks + b) * kRecord];
      uint8_t split[8][16];
      for (size_t lane = 0; lane < 8; ++lane)
        adjacent_to_split(canonical + ((g * 8 + lane) * blocks + b) * kRecord + 1, split[lane]);
      for (int chunk = 0; chunk < 2; ++chunk)
        for (size_t lane = 0; lane < 8; ++lane) {
          std::memcpy(p, split[lane] + chunk * 8, 8);
          p += 8;
        }
    }
}

// pack_x8 with the complete groups spread over threads (same bytes).
void pack_x8_threaded(const uint8_t* canonical, size_t rows, size_t blocks, uint8_t* out, int threads) {
  const size_t groups = rows / 8;
  if (threads <= 1 || groups < 64) {
    pack_x8_groups(canonical, blocks, out, 0, groups);
  } else {
    std::vector<std::thread> pool;
    const size_t per = (groups + threads - 1) / threads;
    for (int t = 0; t < threads; ++t) {
      const size_t lo = std::min(groups, t * per), hi = std::min(groups, lo + per);
      pool.emplace_back([=] { pack_x8_groups(canonical, blocks, out, lo, hi); });
    }
    for (auto& th : pool) th.join();
  }
  uint8_t* p = out + groups * blocks * 136;
  for (size_t r = groups * 8; r < rows; ++r)
    for (size_t b = 0; b < blocks; ++b) {
      std::memcpy(p, canonical + (r * blocks + b) * kRecord, kRecord);
      p += kRecord;
    }
}

void oracle_pack_x8(const uint8_t* canonical, size_t rows, size_t blocks, uint8_t* out) {
  uint8_t* p = out;
  for (size_t g = 0; g < rows / 8; ++g)
    for (size_t b = 0; b < blocks; ++b) {
      for (size_t lane = 0; lane < 8; ++lane) *p++ = canonical[((g * 8 + lane) * blocks + b) * kRecord];
      uint8_t split[8][16];
      for (size_t lane = 0; lane < 8; ++lane)
        adjacent_to_split(canonical + ((g * 8 + lane) * blocks + b) * kRecord + 1, split[lane]);
      for (int chunk = 0; chunk < 2; ++chunk)
        for (size_t lane = 0; lane < 8; ++lane) {
          std::memcpy(p, split[lane] + chunk * 8, 8);
          p += 8;
        }
    }
  for (size_t r = rows / 8 * 8; r < rows; ++r)
    for (size_t b = 0; b < blocks; ++b) {
      std::memcpy(p, canonical + (r * blocks + b) * kRecord, kRecord);
      p += kRecord;
    }
}

// accumulate_mxfp4_bf16_block, lib.rs:932-945 (the exact-BF16 projection
// lane contract); here it pins bf16_bits against the reference's lane-bit KAT.
void oracle_accumulate_mxfp4_bf16_block(const uint8_t* record17, const uint16_t* activation, float* lanes16) {
  const float scale = e8m0_scale(record17[0]);
  for (int i = 0; i < kPacked; ++i) {
    const uint8_t packed = record17[1 + i];
    const float low = bf16_round(kE2M1[packed & 0x0f] * scale);
    const float high = bf16_round(kE2M1[packed >> 4] * scale);
    lanes16[(2 * i) % 16] += low * bf16_to_f32(activation[2 * i]);
    lanes16[(2 * i + 1) % 16] += high * bf16_to_f32(activation[2 * i + 1]);
  }
}

void oracle_bf16_matvec(const uint16_t* w, size_t rows, size_t cols, const uint16_t* x, float* out) {
  for (size_t r = 0; r < rows; ++r) out[r] = bf16_dot(w + r * cols, x, cols);
}
void oracle_rms_norm(const float* in, const float* w, size_t n, float eps, float* out) { rms_norm(in, w, n, eps, out); }
// norm_boundary, cpu_runner.rs:2680-2687: bf16 -> f32, rms_norm, -> bf16.
void oracle_norm_boundary(const uint16_t* x, const float* w, size_t n, float eps, uint16_t* out) {
  std::vector<float> in(n), o(n);
  for (size_t i = 0; i < n; ++i) in[i] = bf16_to_f32(x[i]);
  rms_norm(in.data(), w, n, eps, o.data());
  for (size_t i = 0; i < n; ++i) out[i] = bf16_bits(o[i]);
}
// add_residual, cpu_runner.rs:3732-3738: bf16(residual.to_f32() + update).
void oracle_add_residual(const uint16_t* residual, const float* update, size_t n, uint16_t* out) {
  for (size_t i = 0; i < n; ++i) out[i] = bf16_bits(bf16_to_f32(residual[i]) + update[i]);
}

int oracle_swiglu(const float* gate_up, size_t intermediate, float alpha, float limit, float* out) {
  for (size_t i = 0; i < intermediate; ++i) out[i] = swiglu_one(gate_up[2 * i], gate_up[2 * i + 1], alpha, limit);
  return OK;
}
void oracle_stable_top_k(const float* v, size_t n, size_t k, uint32_t* out) { stable_top_k(v, n, k, out); }
void oracle_softmax(const float* v, size_t n, float* out) { softmax(v, n, out); }
void combine_rows(const float* y, const float* w, size_t m, size_t K, size_t H, float* out, float* unrounded);
void oracle_combine(const float* y, const float* w, size_t m, size_t k, size_t h, float* out) {
  combine_rows(y, w, m, k, h, out, nullptr);
}

// The MoE block, CpuModel::moe_batch (cpu_runner.rs:2794-3013), with the
// residual-Q8 expert projection (the default, cpu_runner.rs:49-90).
// Weights are canonical v1 [E][rows][blocks][17] for gate_up and down.
struct OracleLayer {
  const uint16_t* router_weight;  // bf16 [E][H]
  const float* router_bias;       // [E]
  const uint8_t* gate_up;         // canonical [E][2I][H/32][17]
  const float* gate_up_bias;      // [E][2I]
  const uint8_t* down;            // canonical [E][H][I/32][17]
  const float* down_bias;         // [E][H]
  size_t experts, hidden, intermediate, top_k;
  float alpha, limit;
};

// Weighted combine by source row and rank, then bf16 (cpu_runner.rs:2959-2999):
// per row, output = 0.0; for rank 0..K-1 in order: weighted = y * weight (one
// rounding), output += weighted (one rounding); then fp32_to_bf16_roundtrip.
// y is [m][K][H] by (row, rank) slot, w [m][K]. unrounded (nullable)
// receives the sum before the round trip.
void combine_rows(const float* y, const float* w, size_t m, size_t K, size_t H, float* out, float* unrounded) {
  for (size_t r = 0; r < m; ++r) {
    for (size_t h = 0; h < H; ++h) {
      float acc = 0.0f;
      for (size_t k = 0; k < K; ++k) {
        const float weighted = y[(r * K + k) * H + h] * w[r * K + k];
        acc = acc + weighted;
      }
      if (unrounded) unrounded[r * H + h] = acc;
      out[r * H + h] = bf16_round(acc);
    }
  }
}

// Outputs mirror CpuMoeStep (cpu_runner.rs:569-575); trace arrays mirror
// CpuExpertTrace for every (row, rank) when non-null:
// gate_up [M][k][2I], swiglu [M][k][I], down [M][k][H].
// route_order receives the stable_group_routes order as (row * k + rank).
// injected_logits (nullable) replaces the router projection output before the
// bf16 round trip. `threads` > 1 and `auto_lane` select the baseline lanes for
// the expert projections (1/false is the scalar oracle).
// The exact-BF16 projection of one row (project_mxfp4, cpu_runner.rs:3497-3519):
// total = bias; 16 lanes fed by accumulate_mxfp4_bf16_block block after block
// (lib.rs:932-945); total += the lanes summed 0..15 from -0.0.
void exact_bf16_project(const uint8_t* canonical, size_t rows, size_t blocks, const uint16_t* x, const float* bias,
                        float* out) {
  for (size_t r = 0; r < rows; ++r) {
    float lanes[16] = {0};
    for (size_t b = 0; b < blocks; ++b)
      oracle_accumulate_mxfp4_bf16_block(canonical + (r * blocks + b) * kRecord, x + b * kBlock, lanes);
    float sum = -0.0f;
    for (int l = 0; l < 16; ++l) sum = sum + lanes[l];
    out[r] = bias[r] + sum;
  }
}

int oracle_moe_batch_ex(const OracleLayer* L, const uint16_t* x, size_t m, const float* injected_logits,
                        float* logits, uint32_t* selected, float* weights, float* output, uint32_t* route_order,
                        float* trace_gate_up, float* trace_swiglu, float* trace_down, int auto_lane, int threads,
                        int projection);
int oracle_moe_batch_full(const OracleLayer* L, const uint16_t* x, size_t m, const float* injected_logits,
                          float* logits, uint32_t* selected, float* weights, float* output, uint32_t* route_order,
                          float* trace_gate_up, float* trace_swiglu, float* trace_down, int auto_lane, int threads,
                          int projection, float* output_unrounded);

int oracle_moe_batch(const OracleLayer* L, const uint16_t* x, size_t m, const float* injected_logits, float* logits,
                     uint32_t* selected, float* weights, float* output, uint32_t* route_order, float* trace_gate_up,
                     float* trace_swiglu, float* trace_down, int auto_lane, int threads) {
  return oracle_moe_batch_ex(L, x, m, injected_logits, logits, selected, weights, output, route_order, trace_gate_up,
                             trace_swiglu, trace_down, auto_lane, threads, 0);
}

// lane: 0 the scalar matmul, 1 the faithful Auto lane (x8 GEMV for single-row
// buckets), 4 / 8 the forced AVX2 4x8 / AVX-512 8x8 panel lanes; threads
// spread a bucket's work (1 is the reference's one thread per bucket).
// projection: 0 residual-Q8 (the serving default), 1 Q8, 2 exact-BF16
// (CpuExpertProjection, cpu_runner.rs:49-90; prepare_expert_input and
// project_mxfp4_batch, :3092-3440).
int oracle_moe_batch_ex(const OracleLayer* L, const uint16_t* x, size_t m, const float* injected_logits,
                        float* logits, uint32_t* selected, float* weights, float* output, uint32_t* route_order,
                        float* trace_gate_up, float* trace_swiglu, float* trace_down, int auto_lane, int threads,
                        int projection) {
  return oracle_moe_batch_full(L, x, m, injected_logits, logits, selected, weights, output, route_order,
                               trace_gate_up, trace_swiglu, trace_down, auto_lane, threads, projection, nullptr);
}

// oracle_moe_batch_ex with the combine's sum before fp32_to_bf16_roundtrip
// (cpu_runner.rs:2991) in output_unrounded (nullable).
int oracle_moe_batch_full(const OracleLayer* L, const uint16_t* x, size_t m, const float* injected_logits,
                          float* logits, uint32_t* selected, float* weights, float* output, uint32_t* route_order,
                          float* trace_gate_up, float* trace_swiglu, float* trace_down, int auto_lane, int threads,
                          int projection, float* output_unrounded) {
  if (projection < 0 || projection > 2) return INVALID_DIMENSIONS;
  if ((auto_lane == 4 && !host_has_avx2()) || (auto_lane == 8 && !host_has_avx512_vnni())) return UNAVAILABLE_BACKEND;
  const size_t E = L->experts, H = L->hidden, I = L->intermediate, K = L->top_k;
  if (m == 0 || K == 0 || K > E || H % kBlock || I % kBlock) return INVALID_DIMENSIONS;
  const size_t N1 = 2 * I, B1 = H / kBlock, N2 = H, B2 = I / kBlock;
  // Router: project_bf16_batch then += bias (cpu_runner.rs:2689-2792).
  std::vector<float> lg(m * E);
  for (size_t r = 0; r < m; ++r)
    for (size_t e = 0; e < E; ++e) {
      float v = injected_logits ? injected_logits[r * E + e] : bf16_dot(L->router_weight + e * H, x + r * H, H);
      if (!injected_logits) v += L->router_bias[e];
      lg[r * E + e] = bf16_round(v);
    }
  for (float v : lg)
    if (!std::isfinite(v)) return NON_FINITE_LOGITS;
  struct Route { uint32_t expert, row, rank; float weight; };
  std::vector<Route> routes;
  std::vector<uint32_t> sel(m * K);
  std::vector<float> wts(m * K);
  for (size_t r = 0; r < m; ++r) {
    stable_top_k(&lg[r * E], E, K, &sel[r * K]);
    std::vector<float> l(K), w(K);
    for (size_t k = 0; k < K; ++k) l[k] = lg[r * E + sel[r * K + k]];
    softmax(l.data(), K, w.data());
    for (size_t k = 0; k < K; ++k) {
      wts[r * K + k] = bf16_round(w[k]);
      routes.push_back({sel[r * K + k], (uint32_t)r, (uint32_t)k, wts[r * K + k]});
    }
  }
  // stable_group_routes (cpu_runner.rs:3780-3782).
  std::stable_sort(routes.begin(), routes.end(), [](const Route& a, const Route& b) { return a.expert < b.expert; });
  std::vector<float> y(m * K * H);  // per (row, rank)
  std::vector<float> xf(H), gu, act, dn;
  for (size_t s = 0; s < routes.size();) {
    size_t e_end = s;
    while (e_end < routes.size() && routes[e_end].expert == routes[s].expert) ++e_end;
    const size_t e = routes[s].expert, mb = e_end - s;
    // gate_up over the bucket's gathered rows (cpu_runner.rs:2878-2901).
    gu.assign(mb * N1, 0.0f);
    const uint8_t* wgu = L->gate_up + e * N1 * B1 * kRecord;
    std::vector<ResidualQ8Block> qa(mb * B1);
    std::vector<Q8Block> qa1(mb * B1);
    for (size_t i = 0; i < mb && projection != 2; ++i) {
      for (size_t h = 0; h < H; ++h) xf[h] = bf16_to_f32(x[routes[s + i].row * H + h]);
      int st = projection == 1 ? quantize_q8(xf.data(), H, &qa1[i * B1])
                               : quantize_residual_q8(xf.data(), H, &qa[i * B1]);
      if (st) return st;
    }
    MatmulArgs a1{wgu, N1, B1, 1, 2, qa.data(), mb, B1, L->gate_up_bias + e * N1, gu.data(), N1};
    if (projection == 1) {
      a1.kind = 1;
      a1.act = qa1.data();
    }
    std::vector<uint8_t> x8;
    if (projection == 2) {
      for (size_t i = 0; i < mb; ++i)
        exact_bf16_project(wgu, N1, B1, x + routes[s + i].row * H, L->gate_up_bias + e * N1, &gu[i * N1]);
    } else if (auto_lane == 1 && projection == 0) {
      x8.resize(N1 * B1 * kRecord);
      oracle_pack_x8(wgu, N1, B1, x8.data());
      a1.weights = x8.data();
      a1.layout = 2;
      auto_matmul(a1, threads);
    } else if (auto_lane == 4 || auto_lane == 8) {
      x8.resize(N1 * B1 * kRecord);
      pack_x8_threaded(wgu, N1, B1, x8.data(), threads);
      a1.weights = x8.data();
      a1.layout = 2;
      panel_matmul(a1, auto_lane, threads);
    } else {
      scalar_matmul_rows(a1, 0, mb, 0, N1);
    }
    // bf16 round trip, SwiGLU, bf16 (cpu_runner.rs:2903-2919).
    act.assign(mb * I, 0.0f);
    for (size_t i = 0; i < mb; ++i) {
      for (size_t n = 0; n < N1; ++n) gu[i * N1 + n] = bf16_round(gu[i * N1 + n]);
      for (size_t n = 0; n < I; ++n)
        act[i * I + n] = bf16_round(swiglu_one(gu[i * N1 + 2 * n], gu[i * N1 + 2 * n + 1], L->alpha, L->limit));
    }
    // Down projection over the activated rows (cpu_runner.rs:2933-2947).
    std::vector<ResidualQ8Block> qd(mb * B2);
    std::vector<Q8Block> qd1(mb * B2);
    for (size_t i = 0; i < mb && projection != 2; ++i) {
      int st = projection == 1 ? quantize_q8(&act[i * I], I, &qd1[i * B2]) : quantize_residual_q8(&act[i * I], I, &qd[i * B2]);
      if (st) return st;
    }
    dn.assign(mb * N2, 0.0f);
    const uint8_t* wdn = L->down + e * N2 * B2 * kRecord;
    MatmulArgs a2{wdn, N2, B2, 1, 2, qd.data(), mb, B2, L->down_bias + e * N2, dn.data(), N2};
    if (projection == 1) {
      a2.kind = 1;
      a2.act = qd1.data();
    }
    if (projection == 2) {
      std::vector<uint16_t> act16(I);
      for (size_t i = 0; i < mb; ++i) {
        for (size_t n = 0; n < I; ++n) act16[n] = bf16_bits(act[i * I + n]);  // activated_bf16 (:2917)
        exact_bf16_project(wdn, N2, B2, act16.data(), L->down_bias + e * N2, &dn[i * N2]);
      }
    } else if (auto_lane == 1 && projection == 0) {
      x8.resize(N2 * B2 * kRecord);
      oracle_pack_x8(wdn, N2, B2, x8.data());
      a2.weights = x8.data();
      a2.layout = 2;
      auto_matmul(a2, threads);
    } else if (auto_lane == 4 || auto_lane == 8) {
      x8.resize(N2 * B2 * kRecord);
      pack_x8_threaded(wdn, N2, B2, x8.data(), threads);
      a2.weights = x8.data();
      a2.layout = 2;
      panel_matmul(a2, auto_lane, threads);
    } else {
      scalar_matmul_rows(a2, 0, mb, 0, N2);
    }
    for (size_t i = 0; i < mb; ++i) {
      const Route& rt = routes[s + i];
      const size_t slot = rt.row * K + rt.rank;
      for (size_t h = 0; h < H; ++h) y[slot * H + h] = bf16_round(dn[i * N2 + h]);
      if (trace_gate_up) std::memcpy(trace_gate_up + slot * N1, &gu[i * N1], N1 * 4);
      if (trace_swiglu) std::memcpy(trace_swiglu + slot * I, &act[i * I], I * 4);
      if (trace_down) std::memcpy(trace_down + slot * H, &y[slot * H], H * 4);
    }
    s = e_end;
  }
  combine_rows(y.data(), wts.data(), m, K, H, output, output_unrounded);
  if (logits) std::memcpy(logits, lg.data(), m * E * 4);
  if (selected) std::memcpy(selected, sel.data(), m * K * 4);
  if (weights) std::memcpy(weights, wts.data(), m * K * 4);
  if (route_order)
    for (size_t i = 0; i < routes.size(); ++i) route_order[i] = routes[i].row * (uint32_t)K + routes[i].rank;
  return OK;
}

// Deterministic synthetic data. Byte tensors (MXFP4 codes and E8M0 scales)
// use a counter hash so the GPU library can generate the same bytes on the
// device; Gaussian tensors are generated here only and uploaded.
uint64_t oracle_stream_hash(uint64_t seed, uint64_t stream, uint64_t index) { return stream_hash(seed, stream, index); }

// Canonical v1 MXFP4 tensor [experts][rows][blocks][17]: codes uniform over
// the 16 E2M1 codes, E8M0 byte 127 + U{-8..-4}. Record index
// i = (expert * rows + row) * blocks + block draws two 64-bit hashes.
void oracle_gen_mxfp4(uint64_t seed, uint64_t stream, size_t experts, size_t rows, size_t blocks, uint8_t* out) {
  const size_t n = experts * rows * blocks;
  for (size_t i = 0; i < n; ++i) {
    const uint64_t h0 = stream_hash(seed, stream, 2 * i), h1 = stream_hash(seed, stream, 2 * i + 1);
    uint8_t* rec = out + i * kRecord;
    rec[0] = (uint8_t)(119 + (h1 >> 61) % 5);
    for (int j = 0; j < 8; ++j) rec[1 + j] = (uint8_t)(h0 >> (8 * j));
    for (int j = 0; j < 8; ++j) rec[9 + j] = (uint8_t)(h1 >> (8 * j));
  }
}

// Gaussian N(mean, std) via Box-Muller on the counter hash, rounded to bf16.
void oracle_gen_bf16_normal(uint64_t seed, uint64_t stream, size_t n, float mean, float stddev, uint16_t* out) {
  for (size_t i = 0; i < n; ++i) {
    const uint64_t a = stream_hash(seed, stream, 2 * i), b = stream_hash(seed, stream, 2 * i + 1);
    const double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53;  // (0, 1]
    const double u2 = (double)(b >> 11) * 0x1.0p-53;          // [0, 1)
    const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    out[i] = bf16_bits((float)(mean + stddev * z));
  }
}

// Hidden rows: bf16(N(0,1)), RMS-normalised with unit weight (lib.rs:699-730,
// eps 1e-5), rounded to bf16 (norm_boundary, cpu_runner.rs:2680-2687).
void oracle_gen_hidden(uint64_t seed, uint64_t stream, size_t m, size_t h, int normalise, uint16_t* out) {
  oracle_gen_bf16_normal(seed, stream, m * h, 0.0f, 1.0f, out);
  if (!normalise) return;
  std::vector<float> in(h), w(h, 1.0f), o(h);
  for (size_t r = 0; r < m; ++r) {
    for (size_t i = 0; i < h; ++i) in[i] = bf16_to_f32(out[r * h + i]);
    rms_norm(in.data(), w.data(), h, 1e-5f, o.data());
    for (size_t i = 0; i < h; ++i) out[r * h + i] = bf16_bits(o[i]);
  }
}

}  // extern "C"

namespace {
// ---------------------------------------------------------------------------
// The dense path around the block (crates/gpt-oss-model-runner/src/cpu_runner.rs),
// restated with the reference's own data structures: CpuKvCache's shifting
// vectors, staged rows per step, rows attended one after another.

// YarnRope::new (cpu_runner.rs:3933-3990) and apply (:3992-4012).
struct OracleRope {
  size_t head_dim;
  double theta;
  int32_t yarn;
  double factor;
  size_t original_max;
  double beta_fast, beta_slow;
  int32_t truncate;
};

void yarn_inv_freq(const OracleRope& c, std::vector<float>& inv_freq, float& attention_scale) {
  const size_t dim = c.head_dim;
  inv_freq.clear();
  attention_scale = 1.0f;
  if (!c.yarn) {
    for (size_t index = 0; index < dim; index += 2)
      inv_freq.push_back(1.0f / std::pow((float)c.theta, (float)index / (float)dim));
    return;
  }
  const double pi = 3.141592653589793;
  auto correction = [&](double rotations) {
    return ((double)dim * std::log((double)c.original_max / (rotations * 2.0 * pi))) / (2.0 * std::log(c.theta));
  };
  double low = correction(c.beta_fast), high = correction(c.beta_slow);
  if (c.truncate) {
    low = std::floor(low);
    high = std::ceil(high);
  }
  low = std::fmax(low, 0.0);
  high = std::fmin(high, (double)(dim - 1));
  const double range = std::fmax(std::fabs(high - low), 0.001);
  for (size_t index = 0; index < dim / 2; ++index) {
    const float frequency = std::pow((float)c.theta, (float)(index * 2) / (float)dim);
    const float extrapolation = 1.0f / frequency;
    const float interpolation = 1.0f / ((float)c.factor * frequency);
    const float ramp = std::clamp(((float)index - (float)low) / (float)range, 0.0f, 1.0f);
    inv_freq.push_back(interpolation * ramp + extrapolation * (1.0f - ramp));
  }
  attention_scale = (float)(0.1 * std::log(c.factor) + 1.0);
}

void yarn_apply(const std::vector<float>& inv_freq, float attention_scale, size_t head_dim, float* values,
                size_t heads, size_t position) {
  const size_t half = head_dim / 2;
  for (size_t head = 0; head < heads; ++head) {
    const size_t start = head * head_dim;
    for (size_t index = 0; index < half; ++index) {
      const float angle = (float)position * inv_freq[index];
      const float cosine = bf16_round(std::cos(angle) * attention_scale);
      const float sine = bf16_round(std::sin(angle) * attention_scale);
      const float left = bf16_round(values[start + index]);
      const float right = bf16_round(values[start + half + index]);
      const float left_cosine = bf16_round(left * cosine);
      const float right_sine = bf16_round(right * sine);
      const float right_cosine = bf16_round(right * cosine);
      const float left_sine = bf16_round(left * sine);
      values[start + index] = bf16_round(left_cosine - right_sine);
      values[start + half + index] = bf16_round(right_cosine + left_sine);
    }
  }
}

// CpuKvCache (cpu_runner.rs:653-740): append_validated drops the oldest row
// when full by shifting the vectors.
struct OracleKvCache {
  std::vector<uint16_t> keys, values;
  size_t len = 0, token_width = 0, capacity = 0, start_position = 0;
  void append(size_t position, const uint16_t* key, const uint16_t* value) {
    if (len == capacity) {
      keys.erase(keys.begin(), keys.begin() + token_width);
      values.erase(values.begin(), values.begin() + token_width);
      --len;
      ++start_position;
    }
    if (len == 0) start_position = position;
    keys.insert(keys.end(), key, key + token_width);
    values.insert(values.end(), value, value + token_width);
    ++len;
  }
};

struct StagedRow {
  std::vector<uint16_t> key, value;
};

// attention_one_staged, cpu_runner.rs:3840-3924.
void attention_one_staged(const float* query, const OracleKvCache& cache, const std::vector<StagedRow>& staged,
                          const float* sinks, size_t num_heads, size_t num_kv_heads, size_t head_dim, float* output) {
  const size_t groups = num_heads / num_kv_heads;
  const float scale = 1.0f / std::sqrt((float)head_dim);
  const size_t combined_len = cache.len + staged.size();
  const size_t visible_len = std::min(combined_len, cache.capacity);
  const size_t skipped = combined_len - visible_len;
  std::fill(output, output + num_heads * head_dim, 0.0f);
  for (size_t head = 0; head < num_heads; ++head) {
    const float* q = query + head * head_dim;
    const size_t kv_head = head / groups;
    auto row = [&](size_t combined, bool key) -> const uint16_t* {
      if (combined < cache.len)
        return (key ? cache.keys.data() : cache.values.data()) + combined * cache.token_width + kv_head * head_dim;
      const StagedRow& s = staged[combined - cache.len];
      return (key ? s.key.data() : s.value.data()) + kv_head * head_dim;
    };
    std::vector<float> scores;
    for (size_t token = 0; token < visible_len; ++token) {
      const uint16_t* key = row(skipped + token, true);
      float dot = -0.0f;
      for (size_t d = 0; d < head_dim; ++d) dot += q[d] * bf16_to_f32(key[d]);
      dot = bf16_round(dot);
      scores.push_back(bf16_round(dot * scale));
    }
    float maximum = sinks[head];
    for (float s : scores) maximum = std::fmax(maximum, s);
    float sum = -0.0f;
    for (float s : scores) sum += std::exp(s - maximum);
    const float denominator = std::exp(sinks[head] - maximum) + sum;
    float* destination = output + head * head_dim;
    for (size_t token = 0; token < scores.size(); ++token) {
      const float probability = bf16_round(std::exp(scores[token] - maximum) / denominator);
      const uint16_t* value = row(skipped + token, false);
      for (size_t d = 0; d < head_dim; ++d) destination[d] += probability * bf16_to_f32(value[d]);
    }
    for (size_t d = 0; d < head_dim; ++d) destination[d] = bf16_round(destination[d]);
  }
}

// project_bf16_batch (cpu_runner.rs:2734-2792): out[r][o] = bf16_dot(w[o], x[r]) + bias[o],
// output rows split over `threads` (each output element is one dot).
void project_rows(const uint16_t* w, size_t rows, size_t cols, const uint16_t* x, size_t m, const float* bias,
                  float* out, int threads) {
  auto part = [&](size_t lo, size_t hi) {
    for (size_t o = lo; o < hi; ++o)
      for (size_t r = 0; r < m; ++r) {
        float v = bf16_dot(w + o * cols, x + r * cols, cols);
        if (bias) v += bias[o];
        out[r * rows + o] = v;
      }
  };
  const size_t t = (size_t)std::max(1, threads);
  if (t == 1 || rows < 64) {
    part(0, rows);
    return;
  }
  std::vector<std::thread> pool;
  for (size_t i = 0; i < t; ++i) pool.emplace_back(part, rows * i / t, rows * (i + 1) / t);
  for (auto& th : pool) th.join();
}

}  // namespace

extern "C" {

// Weights of one decoder layer as load_layer produces them (cpu_runner.rs:3526-3671).
struct OracleDenseLayer {
  const float* input_norm;
  const uint16_t* q_weight;
  const float* q_bias;
  const uint16_t* k_weight;
  const float* k_bias;
  const uint16_t* v_weight;
  const float* v_bias;
  const uint16_t* o_weight;
  const float* o_bias;
  const float* sinks;
  const float* post_attention_norm;
  int32_t sliding;
  OracleLayer moe;
};

struct OracleModel {
  size_t vocab, hidden, layers, heads, kv_heads, head_dim, sliding_window, context_cap;
  float rms_norm_eps;
  OracleRope rope;
  const uint16_t* embedding;  // [vocab][hidden]
  const float* final_norm;    // [hidden]
  const uint16_t* lm_head;    // [vocab][hidden]
  const OracleDenseLayer* layer;
};

int oracle_yarn_rope(const OracleRope* c, float* values, size_t heads, size_t position) {
  std::vector<float> inv_freq;
  float attention_scale;
  yarn_inv_freq(*c, inv_freq, attention_scale);
  yarn_apply(inv_freq, attention_scale, c->head_dim, values, heads, position);
  return OK;
}

// attention_one over a cache of capacity `window` after appending `tokens`
// rows (CpuKvCache::append then attention_one, cpu_runner.rs:3829-3838).
int oracle_attention(const float* query, const uint16_t* keys, const uint16_t* values, size_t tokens, size_t window,
                     const float* sinks, size_t heads, size_t kv_heads, size_t head_dim, float* out,
                     size_t* cache_len, size_t* cache_start) {
  OracleKvCache cache;
  cache.token_width = kv_heads * head_dim;
  cache.capacity = window;
  for (size_t t = 0; t < tokens; ++t)
    cache.append(t, keys + t * cache.token_width, values + t * cache.token_width);
  attention_one_staged(query, cache, {}, sinks, heads, kv_heads, head_dim, out);
  if (cache_len) *cache_len = cache.len;
  if (cache_start) *cache_start = cache.start_position;
  return OK;
}

// greedy_token, crates/gpt-oss-bench/src/bin/cpu_parity.rs:750-762.
int oracle_greedy_token(const float* logits, size_t n, uint32_t* token) {
  bool found = false;
  size_t best = 0;
  for (size_t i = 0; i < n; ++i) {
    if (!std::isfinite(logits[i])) continue;
    if (!found || logits[i] > logits[best]) best = i;  // ties keep the lower index
    found = true;
  }
  if (!found) return NON_FINITE_LOGITS;
  *token = (uint32_t)best;
  return OK;
}

// prefill_layer_major (cpu_runner.rs:1827-1855) of `n` prompt tokens, then
// `decode_steps` decode calls (:1877-1885), each fed the previous greedy token.
// prefill_chunk > 0 splits the prompt into steps of that many rows (prepare_step
// and commit per chunk); 0 keeps it one step. tokens_out [decode_steps + 1]
// receives the greedy token after the prompt and after every decode step;
// logits_out (nullable) [decode_steps + 1][vocab]. Each step runs
// prepare_step_inner (:2103-2333) over its rows: forward_layer_batch
// (:2335-2586) per layer, then the final norm and lm_head of the last row.
int oracle_model_generate(const OracleModel* M, const uint32_t* prompt, size_t n, size_t prefill_chunk,
                          size_t decode_steps, int threads, uint32_t* tokens_out, float* logits_out) {
  const size_t H = M->hidden, V = M->vocab, QW = M->heads * M->head_dim, KW = M->kv_heads * M->head_dim;
  if (!n || n + decode_steps > M->context_cap) return INVALID_DIMENSIONS;
  std::vector<float> inv_freq;
  float attention_scale;
  yarn_inv_freq(M->rope, inv_freq, attention_scale);
  std::vector<OracleKvCache> caches(M->layers);
  for (size_t li = 0; li < M->layers; ++li) {
    caches[li].token_width = KW;
    caches[li].capacity = M->layer[li].sliding ? M->sliding_window : M->context_cap;
  }
  size_t position = 0;
  std::vector<float> logits(V);
  const size_t chunk = prefill_chunk ? prefill_chunk : n;
  size_t consumed = std::min(chunk, n), step = 0;
  std::vector<uint32_t> rows(prompt, prompt + consumed);
  for (;;) {
    const size_t m = rows.size();
    std::vector<uint16_t> hidden(m * H), normalized(m * H), attention(m * QW), after(m * H), post(m * H);
    std::vector<float> q(m * QW), k(m * KW), v(m * KW), ctx(QW), projected(m * H), moe_out(m * H);
    std::vector<std::vector<StagedRow>> staged(M->layers);
    for (size_t r = 0; r < m; ++r) {
      if (rows[r] >= V) return INVALID_DIMENSIONS;
      std::memcpy(&hidden[r * H], M->embedding + (size_t)rows[r] * H, H * 2);
    }
    for (size_t li = 0; li < M->layers; ++li) {
      const OracleDenseLayer& L = M->layer[li];
      for (size_t r = 0; r < m; ++r) oracle_norm_boundary(&hidden[r * H], L.input_norm, H, M->rms_norm_eps, &normalized[r * H]);
      project_rows(L.q_weight, QW, H, normalized.data(), m, L.q_bias, q.data(), threads);
      project_rows(L.k_weight, KW, H, normalized.data(), m, L.k_bias, k.data(), threads);
      project_rows(L.v_weight, KW, H, normalized.data(), m, L.v_bias, v.data(), threads);
      for (size_t r = 0; r < m; ++r) {
        float* qr = &q[r * QW];
        float* kr = &k[r * KW];
        for (size_t i = 0; i < QW; ++i) qr[i] = bf16_round(qr[i]);
        for (size_t i = 0; i < KW; ++i) kr[i] = bf16_round(kr[i]);
        yarn_apply(inv_freq, attention_scale, M->head_dim, qr, M->heads, position + r);
        yarn_apply(inv_freq, attention_scale, M->head_dim, kr, M->kv_heads, position + r);
        for (size_t i = 0; i < QW; ++i) qr[i] = bf16_round(qr[i]);
        for (size_t i = 0; i < KW; ++i) kr[i] = bf16_round(kr[i]);
        StagedRow row;
        for (size_t i = 0; i < KW; ++i) {
          row.key.push_back(bf16_bits(kr[i]));
          row.value.push_back(bf16_bits(v[r * KW + i]));
        }
        staged[li].push_back(std::move(row));
        attention_one_staged(qr, caches[li], staged[li], L.sinks, M->heads, M->kv_heads, M->head_dim, ctx.data());
        for (size_t i = 0; i < QW; ++i) attention[r * QW + i] = bf16_bits(ctx[i]);
      }
      project_rows(L.o_weight, H, QW, attention.data(), m, L.o_bias, projected.data(), threads);
      for (size_t r = 0; r < m; ++r) {
        for (size_t i = 0; i < H; ++i) projected[r * H + i] = bf16_round(projected[r * H + i]);
        oracle_add_residual(&hidden[r * H], &projected[r * H], H, &after[r * H]);
        oracle_norm_boundary(&after[r * H], L.post_attention_norm, H, M->rms_norm_eps, &post[r * H]);
      }
      const int st = oracle_moe_batch(&L.moe, post.data(), m, nullptr, nullptr, nullptr, nullptr, moe_out.data(),
                                      nullptr, nullptr, nullptr, nullptr, 1, threads);
      if (st) return st;
      for (size_t r = 0; r < m; ++r) oracle_add_residual(&after[r * H], &moe_out[r * H], H, &hidden[r * H]);
    }
    std::vector<uint16_t> fin(H);
    oracle_norm_boundary(&hidden[(m - 1) * H], M->final_norm, H, M->rms_norm_eps, fin.data());
    project_rows(M->lm_head, V, H, fin.data(), 1, nullptr, logits.data(), threads);
    for (float& x : logits) {
      x = bf16_round(x);
      if (!std::isfinite(x)) return NON_FINITE_LOGITS;
    }
    // PreparedCpuStep::commit: the staged rows enter the caches in order.
    for (size_t li = 0; li < M->layers; ++li)
      for (size_t r = 0; r < m; ++r) caches[li].append(position + r, staged[li][r].key.data(), staged[li][r].value.data());
    position += m;
    if (consumed < n) {  // the next prompt chunk
      const size_t next = std::min(n, consumed + chunk);
      rows.assign(prompt + consumed, prompt + next);
      consumed = next;
      continue;
    }
    if (logits_out) std::memcpy(logits_out + step * V, logits.data(), V * 4);
    if (int st = oracle_greedy_token(logits.data(), V, &tokens_out[step])) return st;
    if (step == decode_steps) break;
    rows.assign(1, tokens_out[step]);
    ++step;
  }
  return OK;
}

// Counter-hash Gaussian bf16 tensor split over threads (each element depends
// only on its index, so the result is oracle_gen_bf16_normal's).
void oracle_gen_bf16_normal_mt(uint64_t seed, uint64_t stream, size_t n, float mean, float stddev, uint16_t* out,
                               int threads) {
  const size_t t = (size_t)std::max(1, threads);
  std::vector<std::thread> pool;
  for (size_t i = 0; i < t; ++i) {
    const size_t lo = n * i / t, hi = n * (i + 1) / t;
    pool.emplace_back([=] {
      for (size_t j = lo; j < hi; ++j) {
        const uint64_t a = stream_hash(seed, stream, 2 * j), b = stream_hash(seed, stream, 2 * j + 1);
        const double u1 = ((double)(a >> 11) + 1.0) * 0x1.0p-53;
        const double u2 = (double)(b >> 11) * 0x1.0p-53;
        const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
        out[j] = bf16_bits((float)(mean + stddev * z));
      }
    });
  }
  for (auto& th : pool) th.join();
}

}  // extern "C"
