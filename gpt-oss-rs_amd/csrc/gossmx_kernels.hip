// gfx950 kernels of the GPT-OSS MXFP4 mixture-of-experts block.
//
// Exactness contract (crates/gpt-oss-cpu-kernels and cpu_runner.rs of
// gpt-oss-rs v0.1.0): every integer FP4 x Q8 block dot is exact, and every
// float chain keeps the reference's operation order, so the outputs are
// bit-identical to the scalar CPU path. Build with -ffp-contract=off: no
// multiply-add below may be fused unless written as fma() on purpose.
//
// Expert GEMM: v_mfma_f32_16x16x32_f16 with K = 32 = one MXFP4 block. The B
// operand is the weight tile converted from FP4 by v_cvt_scalef32_pk_f16_fp4
// (E2M1 values are exact in f16); the A operand holds the Q8 codes as f16
// (exact). Each product is exact in f32 and every partial sum is a multiple of
// 0.5 below 2^15, so the MFMA returns p / 2 exactly, where p is the reference's
// doubled-LUT integer dot (lib.rs:1067-1098). The reference term
// (p * (0.5 * e8m0)) * act_scale equals ((p / 2) * e8m0) * act_scale bit for
// bit: the first product is the same real number rounded once.
#include "gossmx_internal.h"

#include <hip/hip_ext.h>

#include <algorithm>
#include <cmath>

namespace gossmx {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint64_t u64x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Scalar helpers.

// bf16::from_f32 of half 2.7.1 (round to nearest even, NaN quieted), used by
// fp32_to_bf16_roundtrip, cpu_runner.rs:3740-3744.
// f32 -> bf16 as half 2.7.1's from_f32: round to nearest even, NaN kept with
// its sign and upper payload and the quiet bit set ((x >> 16) | 0x40). gfx950's
// conversion instruction (v_cvt_pk_bf16_f32, which the __bf16 cast compiles
// to) gives exactly these bits: compared on every one of the 2^32 f32
// patterns, and checked again by the context self-test on edge cases.
__device__ __forceinline__ uint16_t bf16_bits(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ float bf16r(float f) { return bf16_to_f32(bf16_bits(f)); }

// e8m0_scale, lib.rs:957-963: 0x00 -> 2^-127, 0xff -> NaN, else 2^(s-127).
__device__ __forceinline__ float e8m0(uint32_t s) {
  return s == 0 ? __uint_as_float(0x00400000u) : (s == 0xffu ? __uint_as_float(0x7fc00000u) : __uint_as_float(s << 23));
}

// expf with the exact results of the host's glibc 2.35 expf, which is what
// Rust's f32::exp calls on x86_64 Linux (softmax cpu_runner.rs:3784-3795,
// gpt_oss_swiglu :3797-3826). Algorithm of glibc sysdeps/ieee754/flt-32/e_expf.c
// (Szabolcs Nagy, ARM optimized-routines): x * 32/ln2 split by the 0x1.8p52
// shift into k and r, a 32-entry table of 2^(i/32), and a cubic in r, all in
// double with fused multiply-adds as the FMA build of glibc evaluates it.
// Table entries: bits of 2^(i/32) rounded to double, minus i << 47.
__constant__ uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// `tab` is kExp2Tab or a copy of it (e.g. in LDS).
__device__ float expf_glibc(float x, const uint64_t* tab = kExp2Tab) {
  const uint32_t ux = __float_as_uint(x);
  const uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {  // |x| >= 88 (top 12 bits of 88.0f), inf or NaN
    if (ux == 0xff800000u) return 0.0f;
    if (abstop >= 0x7f8u) return x + x;
    if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double inv_ln2_n = 0x1.71547652b82fep+0 * 32;
  const double shift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
  const double xd = (double)x;
  double kd = fma(inv_ln2_n, xd, shift);
  const uint64_t ki = (uint64_t)__double_as_longlong(kd);
  kd -= shift;
  const double r = fma(inv_ln2_n, xd, -kd);
  const uint64_t t = tab[ki % 32] + (ki << 47);
  const double s = __longlong_as_double((long long)t);
  const double z = fma(c0, r, c1);
  const double r2 = r * r;
  double y = fma(c2, r, 1.0);
  y = fma(z, r2, y);
  y = y * s;
  return (float)y;
}

// The SwiGLU sigmoid bf16(1 / (1 + expf(-s))) of gpt_oss_swiglu
// (cpu_runner.rs:3819-3820) for every bf16 value s = bits << 16.
__device__ __forceinline__ uint16_t sigmoid_bf16(uint32_t bits, const uint64_t* tab = kExp2Tab) {
  const float scaled = bf16_to_f32((uint16_t)bits);
  return bf16_bits(1.0f / (1.0f + expf_glibc(-scaled, tab)));
}

// kExp2Tab copied into LDS by every kernel that runs the gate_up epilogue
// (its first 32 threads, before the K loop's barriers), so that the epilogue
// computes each sigmoid with LDS lookups instead of a dependent global gather.
// In two halves: the load with the kernel's first requests, the LDS store once
// they are in flight (the store waits for its data).
__shared__ uint64_t s_exp2_tab[32];
__device__ __forceinline__ uint64_t load_exp2_entry() { return threadIdx.x < 32 ? kExp2Tab[threadIdx.x] : 0ull; }
__device__ __forceinline__ void store_exp2_entry(uint64_t v) {
  if (threadIdx.x < 32) s_exp2_tab[threadIdx.x] = v;
}

// gpt_oss_swiglu for one (gate, up) pair, cpu_runner.rs:3797-3826: gate =
// min(g, limit) (NaN-ignoring like f32::min), up = clamp(u, -limit, limit)
// (NaN kept), then bf16 after every tensor operation. The sigmoid's input is
// a bf16 value, so it is read from `sig_tab`, the 65,536 values of
// sigmoid_bf16 computed by the same code (build_sigmoid_table).
// The table index of a pair's sigmoid: the bf16 bits of min(g, limit) * alpha.
__device__ __forceinline__ uint32_t swiglu_sigmoid_index(float g, float alpha, float limit) {
  return bf16_bits(fminf(g, limit) * alpha);
}

// The rest of gpt_oss_swiglu once the pair's bf16 sigmoid value is known.
__device__ __forceinline__ float swiglu_finish(float g, float u, float limit, float sig) {
  const float gate = fminf(g, limit);
  float up = u;
  if (up < -limit) up = -limit;
  if (up > limit) up = limit;
  const float glu = bf16r(gate * sig);
  const float lin = bf16r(up + 1.0f);
  return bf16r(glu * lin);
}

__device__ __forceinline__ float swiglu_one(float g, float u, float alpha, float limit, const uint16_t* sig_tab) {
  return swiglu_finish(g, u, limit, bf16_to_f32(sig_tab[swiglu_sigmoid_index(g, alpha, limit)]));
}

__global__ void build_sigmoid_table_kernel(uint16_t* tab) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < 65536u) tab[i] = sigmoid_bf16(i);
}

// The partner lane of a butterfly round over groups of 2 O lanes, taken in
// increasing O: O = 1 and 2 swap lanes i ^ O (DPP quad permutes, no LDS
// round trip); O = 4 and 8 take lane i's mirror within its 8- or 16-lane row
// (DPP row_half_mirror, row_mirror), a lane of the other half whose value the
// earlier rounds made equal to its whole half's; O = 16 swaps i ^ 16
// (ds_swizzle), O = 32 i ^ 32 (ds_bpermute). After the rounds up to O every
// lane of a 2 O-lane group holds the same result of an order-free operation
// (max, top-k of distinct keys). Every lane of the group must execute it.
template <int O>
__device__ __forceinline__ uint32_t lane_partner(uint32_t v) {
  if constexpr (O == 1) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
  else if constexpr (O == 2) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
  else if constexpr (O == 4) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false);
  else if constexpr (O == 8) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false);
  else if constexpr (O == 16) return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x401F);
  else return __shfl_xor(v, 32);
}
__device__ __forceinline__ float half_wave_max(float m) {
  m = fmaxf(m, __uint_as_float(lane_partner<1>(__float_as_uint(m))));
  m = fmaxf(m, __uint_as_float(lane_partner<2>(__float_as_uint(m))));
  m = fmaxf(m, __uint_as_float(lane_partner<4>(__float_as_uint(m))));
  m = fmaxf(m, __uint_as_float(lane_partner<8>(__float_as_uint(m))));
  return fmaxf(m, __uint_as_float(lane_partner<16>(__float_as_uint(m))));
}

// quantize_q8_block (lib.rs:1051-1065) for the 32 values held by a 32-lane
// half wave (lane l32 holds value l32): scale = max|v| / 127, inverse =
// 1 / scale (0 when scale is 0), q = clamp(round_half_away(v * inverse)).
// max is order-free, so the butterfly gives the reference's fold.
__device__ __forceinline__ void q8_half_wave(float v, float& q, float& scale) {
  const float mx = half_wave_max(fabsf(v));
  scale = mx / 127.0f;
  const float inv = scale == 0.0f ? 0.0f : 1.0f / scale;
  q = fminf(fmaxf(roundf(v * inv), -127.0f), 127.0f);
}

// quantize_residual_q8 (lib.rs:382-409) of one block held by a half wave;
// writes the f16 codes and the two scales of (row, blk) into `act`. With
// qmode kProjQ8, quantize_q8 (lib.rs:347-378): the primary block only, the
// residual codes and scale stored as zeros. With kProjExactBf16 the value's
// bf16 bits go to act.v viewed as [row][blocks * 32] bf16.
__device__ __forceinline__ void residual_q8_store(float v, int l32, size_t row, int blocks, int blk, ActBuffers act,
                                                  int qmode = kProjResidualQ8) {
  if (qmode == kProjExactBf16) {
    reinterpret_cast<uint16_t*>(act.v)[(row * blocks + blk) * kBlock + l32] = bf16_bits(v);
    return;
  }
  float q, s;
  q8_half_wave(v, q, s);
  const float r = qmode == kProjQ8 ? 0.0f : v - q * s;
  float rq, rs;
  q8_half_wave(r, rq, rs);
  _Float16* dst = act.v + ((row * blocks + blk) * 2) * kBlock;
  dst[l32] = (_Float16)q;
  dst[kBlock + l32] = (_Float16)rq;
  if (l32 == 0) {
    float2 sc;
    sc.x = s;
    sc.y = rs;
    reinterpret_cast<float2*>(act.s)[row * blocks + blk] = sc;
  }
}

// Scale = max / 127 and inverse = 1 / scale (0 for a zero scale) of the N
// blocks a half wave quantizes: the max is uniform over the half wave, so
// lane j < N computes block j's pair once (the same correctly rounded
// divisions) and every lane reads its blocks' pairs back by lane permute,
// instead of every lane dividing for every block.
template <int N>
__device__ __forceinline__ void q8_scales_n(const float (&mx)[N], int l32, float (&sc)[N], float (&inv)[N]) {
  float m = mx[0];
#pragma unroll
  for (int i = 1; i < N; ++i) m = (l32 % N) == i ? mx[i] : m;
  const float sl = m / 127.0f;
  const float il = sl == 0.0f ? 0.0f : 1.0f / sl;
  const int base = threadIdx.x & 32;  // this half wave's first lane in the wave
#pragma unroll
  for (int i = 0; i < N; ++i) {
    sc[i] = __shfl(sl, base + i);
    inv[i] = __shfl(il, base + i);
  }
}

// residual_q8_store for N blocks per half wave at once (block i is item
// hw + i * stride: activation row first_row + item / per_row, block
// first_blk + item % per_row); blocks with live[i] false are computed on
// zeros and not stored. The same operations as residual_q8_store per block.
template <int N, bool RESIDUAL>
__device__ __forceinline__ void residual_q8_store_n(const float (&v)[N], const bool (&live)[N], int l32, int hw,
                                                    int stride, int per_row, size_t first_row, int blocks,
                                                    int first_blk, ActBuffers act) {
  float mx[N], q[N], s[N], r[N], rq[N], rs[N], inv[N];
#pragma unroll
  for (int i = 0; i < N; ++i) mx[i] = half_wave_max(fabsf(v[i]));
  if constexpr (N >= 4) {
    q8_scales_n<N>(mx, l32, s, inv);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      s[i] = mx[i] / 127.0f;
      inv[i] = s[i] == 0.0f ? 0.0f : 1.0f / s[i];
    }
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    q[i] = fminf(fmaxf(roundf(v[i] * inv[i]), -127.0f), 127.0f);
    r[i] = RESIDUAL ? v[i] - q[i] * s[i] : 0.0f;  // quantize_q8: no residual block
    mx[i] = fabsf(r[i]);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) mx[i] = half_wave_max(mx[i]);
  if constexpr (N >= 4) {
    q8_scales_n<N>(mx, l32, rs, inv);
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      rs[i] = mx[i] / 127.0f;
      inv[i] = rs[i] == 0.0f ? 0.0f : 1.0f / rs[i];
    }
  }
#pragma unroll
  for (int i = 0; i < N; ++i) rq[i] = fminf(fmaxf(roundf(r[i] * inv[i]), -127.0f), 127.0f);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if (!live[i]) continue;  // uniform per half wave
    const int item = hw + i * stride;
    const size_t row = first_row + item / per_row;
    const int blk = first_blk + item % per_row;
    _Float16* dst = act.v + ((row * blocks + blk) * 2) * kBlock;
    dst[l32] = (_Float16)q[i];
    dst[kBlock + l32] = (_Float16)rq[i];
    if (l32 == 0) {
      float2 sc;
      sc.x = s[i];
      sc.y = rs[i];
      reinterpret_cast<float2*>(act.s)[row * blocks + blk] = sc;
    }
  }
}

// ---------------------------------------------------------------------------
// Router projection and bias with the bf16-rounded logits (the first
// router_groups work-groups of a row, one per 16 experts; the selection
// kernels read the logits), and the gate_up input quantization (the rest: 8
// blocks of 32 values per work-group, one per half wave), for row blockIdx.x
// (moe_batch routing loop, cpu_runner.rs:2808-2854; quantize_residual_q8 of
// the row, cpu_runner.rs:3224-3231).

__device__ __forceinline__ bool route_better(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);  // stable_top_k order, cpu_runner.rs:3768-3778
}

constexpr int kRouteQuantBlocks = 8;  // quantized blocks per work-group (256 threads)

// Router projection staging: a pass covers kRouterGroup experts (16 chains
// each = 256 threads) over kRouterChunk hidden elements held in LDS (x as
// f32, the weight rows as bf16, both loaded with coalesced 16-byte reads), so
// every chain step reads LDS instead of waiting on a global load.
constexpr int kRouterGroup = 16;
constexpr int kRouterChunk = 1440;  // multiple of 16 (chain lanes) and 8 (16-byte pieces)
constexpr int kRouterLoads = (kRouterGroup * kRouterChunk / 8 + 255) / 256;  // 16-byte reads per thread per chunk

__host__ __device__ __forceinline__ int router_groups(const RouteArgs& a) {
  return (a.experts + kRouterGroup - 1) / kRouterGroup;
}

// Grid (m, router_groups + quantization groups): work-group (r, g) computes
// experts [16 g, 16 g + 16) of row r.
// The inverse RMS of row xr (hidden H <= kNormMaxHidden, a multiple of 8,
// 16-byte aligned) for the post-attention RMSNorm (norm_boundary,
// cpu_runner.rs:2680-2687, over Kernels::rms_norm and scalar_sum_squares,
// lib.rs:699-730, 1031-1043), by a whole work-group of 256 or more threads
// (every thread calls it and gets the value): the row is staged in LDS with
// 16-byte loads, then lane l < 16 sums x_i * x_i (multiply, then add) over
// i = l, l + 16, ... in order; the lanes are added 0..15; the inverse is
// 1 / sqrt(sum / H + eps) with correctly rounded division and square root.
__device__ __forceinline__ float row_inverse_rms(const uint16_t* xr, int H, float eps) {
  __shared__ __align__(16) uint16_t s_row[kNormMaxHidden];
  __shared__ float s_lane[16];
  __shared__ float s_inv;
  const int tid = threadIdx.x;
#pragma unroll 4
  for (int v = tid; v < H / 8; v += 256)
    reinterpret_cast<u32x4*>(s_row)[v] = reinterpret_cast<const u32x4*>(xr)[v];
  __syncthreads();
  if (tid < 16) {
    float acc = 0.0f;
#pragma unroll 16
    for (int i = tid; i < H; i += 16) {
      const float v = bf16_to_f32(s_row[i]);
      acc = acc + v * v;
    }
    s_lane[tid] = acc;
  }
  __syncthreads();
  if (tid == 0) {
    float ss = -0.0f;
    for (int l = 0; l < 16; ++l) ss = ss + s_lane[l];
    s_inv = 1.0f / sqrtf(ss / (float)H + eps);
  }
  __syncthreads();
  return s_inv;
}

// x_i of the router's input: the row as given, or with a.norm_w the
// post-attention RMSNorm of it rounded to bf16 (norm_boundary).
__device__ __forceinline__ float route_input(const RouteArgs& a, float xf, int i, float inv) {
  return a.norm_w ? bf16r(xf * inv * a.norm_w[i]) : xf;
}

__global__ __launch_bounds__(256) void route_kernel(RouteArgs a) {
  const int r = blockIdx.x, tid = threadIdx.x;
  const int E = a.experts, H = a.hidden;
  const uint16_t* x = a.x + (size_t)r * H;
  const int n_router = router_groups(a);
  // With the fused post-attention RMSNorm every work-group of the row first
  // computes the row's inverse RMS (uniform branch).
  const float inv = a.norm_w ? row_inverse_rms(x, H, a.norm_eps) : 1.0f;
  if ((int)blockIdx.y >= n_router) {
    const int hw = tid >> 5, l32 = tid & 31;
    const int blocks = H / kBlock;
    const int b = ((int)blockIdx.y - n_router) * kRouteQuantBlocks + hw;
    if (b < blocks) {  // uniform per half wave
      const int i = b * kBlock + l32;
      const float v = route_input(a, bf16_to_f32(x[i]), i, inv);
      // The exact-BF16 projection takes its input unchecked (prepare_expert_input, cpu_runner.rs:3108).
      if (a.qmode != kProjExactBf16 && !isfinite(v)) atomicOr(a.err, kErrNonFiniteInput);
      residual_q8_store(v, l32, (size_t)r, blocks, b, a.act, a.qmode);
    }
    return;
  }
  __shared__ float s_chain[kMaxExperts * 16];
  __shared__ float s_logit[kMaxExperts];
  const int e_begin = (int)blockIdx.y * kRouterGroup;
  const int e_end = min(E, e_begin + kRouterGroup);

  {
    // scalar_bf16_dot (lib.rs:1007-1029): 16 reduction lanes, lane j sums
    // w[i] * x[i] for i = j mod 16 in increasing i, multiply then add.
    __shared__ float s_x[kRouterChunk];
    __shared__ __align__(16) uint16_t s_w[kRouterGroup * kRouterChunk];
    const int l = tid & 15, ge = tid >> 4;
    for (int g0 = e_begin; g0 < e_end; g0 += kRouterGroup) {  // uniform
      const int ng = min(kRouterGroup, e_end - g0);
      float acc = 0.0f;
      for (int c0 = 0; c0 < H; c0 += kRouterChunk) {  // uniform
        const int len = min(kRouterChunk, H - c0);
        const int pieces = len / 8;
        // Every global read of the chunk is issued before the first LDS
        // write, so the chunk costs one memory round trip.
        // Indices past the chunk are clamped to its last piece: such a lane
        // reads and writes exactly what the piece's own lane does.
        u32x4 wv[kRouterLoads];
        uint32_t xv[kRouterChunk / 256 + 1];
        const int n_pieces = ng * pieces;
#pragma unroll
        for (int k = 0; k < kRouterLoads; ++k) {
          const int p = min(tid + k * 256, n_pieces - 1);
          const int re = p / pieces, q = p - re * pieces;
          wv[k] = *reinterpret_cast<const u32x4*>(a.router_w + (size_t)(g0 + re) * H + c0 + q * 8);
        }
        float nv[kRouterChunk / 256 + 1];  // norm weights of the same elements (fused RMSNorm)
#pragma unroll
        for (int k = 0; k < kRouterChunk / 256 + 1; ++k) {
          xv[k] = x[c0 + min(tid + k * 256, len - 1)];
          nv[k] = a.norm_w ? a.norm_w[c0 + min(tid + k * 256, len - 1)] : 1.0f;
        }
        __syncthreads();  // the previous chunk's readers are done
#pragma unroll
        for (int k = 0; k < kRouterLoads; ++k) {
          const int p = min(tid + k * 256, n_pieces - 1);
          const int re = p / pieces, q = p - re * pieces;
          *reinterpret_cast<u32x4*>(&s_w[re * kRouterChunk + q * 8]) = wv[k];
        }
#pragma unroll
        for (int k = 0; k < kRouterChunk / 256 + 1; ++k) {
          const int idx = min(tid + k * 256, len - 1);
          const float xf = __uint_as_float(xv[k] << 16);
          s_x[idx] = a.norm_w ? bf16r(xf * inv * nv[k]) : xf;
        }
        __syncthreads();
        if (ge < ng) {
          const uint16_t* w = s_w + ge * kRouterChunk;
#pragma unroll 5
          for (int i = l; i < len; i += 16) acc = acc + bf16_to_f32(w[i]) * s_x[i];
        }
      }
      if (ge < ng) s_chain[(g0 + ge) * 16 + l] = acc;
    }
    __syncthreads();
    for (int e = e_begin + tid; e < e_end; e += blockDim.x) {
      float s = s_chain[e * 16];
      for (int j = 1; j < 16; ++j) s = s + s_chain[e * 16 + j];
      s_logit[e] = bf16r(s + a.router_b[e]);  // += bias (cpu_runner.rs:2781-2783), bf16 (:2829)
    }
  }
  __syncthreads();
  // The selection kernels check these logits for non-finite values.
  for (int e = e_begin + tid; e < e_end; e += blockDim.x) a.logits[(size_t)r * E + e] = s_logit[e];
}

// ---------------------------------------------------------------------------
// Stable grouping of routes by expert (stable_group_routes,
// cpu_runner.rs:3780-3782): route i = row * top_k + rank goes to
// bucket_off[e] + #{j < i : expert(j) == e}. Work-groups of 1024 threads; in
// a wave, ranks come from one ballot per expert present in the wave.
//
// Work items: every bucket is cut into a.chunk-row chunks. Full chunks come
// first (expert order), then the partial last chunks by descending size
// (ties by expert), so the heaviest work items start first.

// From the per-expert totals s_tot (LDS): the bucket offsets s_off (LDS,
// exclusive scan over experts) and, with `meta`, the global bucket_off, work
// list and n_work. Waves 0 and 1 hold one expert per lane (kMaxExperts = 128).
__device__ __forceinline__ void dispatch_offsets(const DispatchArgs& a, const int* s_tot, int* s_off, bool meta) {
  const int E = a.experts;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ int s_scan[4];
  __shared__ int s_parts[2];
  // Per wave w and partial-chunk size v: experts of the wave with a larger
  // partial chunk (s_gt) and with this size (s_eq), for the other wave's
  // ranking.
  __shared__ int s_gt[2][kChunkMax], s_eq[2][kChunkMax];
  int c = 0, full = 0, sc = 0, sf = 0, part = 0, rank_in_wave = 0;
  if (wave < 2) {
    c = tid < E ? s_tot[tid] : 0;
    full = c / a.chunk;
    part = c % a.chunk;
    sc = c;
    sf = full;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(sc, o), v = __shfl_up(sf, o);
      if (lane >= o) { sc += u; sf += v; }
    }
    if (lane == 63) { s_scan[2 * wave] = sc; s_scan[2 * wave + 1] = sf; }
    if (meta) {
      // Partial chunks are ranked by descending size, ties by expert: within
      // the wave, by one ballot per size (lanes past E hold size 0 and never
      // count).
      const unsigned long long lt = (1ull << lane) - 1ull;
      int gt_lane = 0, eq_lane = 0;  // for lane l < chunk: the wave's experts with a partial chunk > l, == l
      for (int v = 1; v < a.chunk; ++v) {  // uniform
        const unsigned long long m = __ballot(part == v);
        const int n = __popcll(m);
        rank_in_wave += (v > part ? n : 0) + (v == part ? __popcll(m & lt) : 0);
        gt_lane += v > lane ? n : 0;
        eq_lane = v == lane ? n : eq_lane;
      }
      const int n_parts = __popcll(__ballot(part > 0));
      if (lane < a.chunk) {
        s_gt[wave][lane] = gt_lane;
        s_eq[wave][lane] = eq_lane;
      }
      if (lane == 0) s_parts[wave] = n_parts;
    }
  }
  __syncthreads();
  int off = 0, full_before = 0, total_full = 0, parts = 0, before = 0;
  if (wave < 2) {
    if (wave == 1) { sc += s_scan[0]; sf += s_scan[1]; }
    total_full = s_scan[1] + s_scan[3];
    off = sc - c;
    full_before = sf - full;
    if (tid < E) {
      s_off[tid] = off;
      if (meta) {
        parts = s_parts[0] + s_parts[1];
        // Wave 0's experts all come before wave 1's.
        before = rank_in_wave + (wave == 0 ? s_gt[1][part] : s_gt[0][part] + s_eq[0][part]);
      }
    }
  }
  __syncthreads();
  // The offsets, work list and item count after the last barrier, so that
  // their stores are off the path to it.
  if (meta && wave < 2 && tid < E) {
    a.bucket_off[tid] = off;
    int4* const rec = reinterpret_cast<int4*>(a.work);
    for (int i = 0; i < full; ++i) rec[full_before + i] = make_int4(tid, off + i * a.chunk, a.chunk, 0);
    if (part > 0) rec[total_full + before] = make_int4(tid, off + full * a.chunk, part, 0);
    if (tid == 0) {
      *a.n_work = total_full + parts;
      a.bucket_off[E] = s_scan[0] + s_scan[2];
    }
  }
}

// Places routes [begin, end) of `sel` (global memory or LDS) in route order:
// route i of expert e goes to s_base[e] + (its rank among the range's routes
// of expert e). s_base (LDS) advances by each pass's counts.
__device__ __forceinline__ void dispatch_place(const DispatchArgs& a, const int* sel, int begin, int end,
                                               int* s_base) {
  const int E = a.experts;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ int s_wcnt[16][kMaxExperts];
  const unsigned long long lt = (1ull << lane) - 1ull;
  for (int base = begin; base < end; base += 1024) {  // uniform
    const int i = base + tid;
    const int e = i < end ? sel[i] : -1;
    for (int ee = lane; ee < E; ee += 64) s_wcnt[wave][ee] = 0;
    int rank = 0;
    unsigned long long pending = __ballot(e >= 0);
    while (pending) {
      // The leader lane is wave-uniform: a scalar read, not a shuffle.
      const int leader = __ffsll((long long)pending) - 1;
      const int ee = __builtin_amdgcn_readlane(e, leader);
      const unsigned long long m = __ballot(e == ee);
      if (e == ee) rank = __popcll(m & lt);
      if (lane == 0) s_wcnt[wave][ee] = __popcll(m);
      pending &= ~m;
    }
    __syncthreads();
    // Per expert: the wave counts become the start of each wave's routes
    // (s_base plus the counts of earlier waves); s_base advances past the pass.
    for (int ee = tid; ee < E; ee += 1024) {
      int run = s_base[ee];
#pragma unroll
      for (int w = 0; w < 16; ++w) {
        const int c = s_wcnt[w][ee];
        s_wcnt[w][ee] = run;
        run += c;
      }
      s_base[ee] = run;
    }
    __syncthreads();
    if (e >= 0) {
      const int pos = s_wcnt[wave][e] + rank;
      a.route_tok[pos] = i / a.top_k;
      a.route_slot[pos] = i;
    }
    __syncthreads();
  }
}

// The whole grouping in one work-group for at most kMaskRoutes routes (one
// per thread): route i sets bit i of its expert's route mask in LDS; an
// expert's count is its mask's popcount, and route i's place among its
// expert's routes is the popcount of the mask's bits below i
// (stable_group_routes's order), with no per-wave ballot loop.
constexpr int kMaskRoutes = 1024;

__device__ __forceinline__ void dispatch_body_masked(const DispatchArgs& a, const int* sel) {
  const int tid = threadIdx.x, E = a.experts, R = a.routes;
  const int nw = (R + 31) / 32;  // mask words in use
  __shared__ uint32_t s_mask[kMaxExperts][kMaskRoutes / 32];
  __shared__ int s_tot[kMaxExperts];
  __shared__ int s_off[kMaxExperts];
  for (int v = tid; v < E * nw; v += 1024) s_mask[v / nw][v % nw] = 0u;
  __syncthreads();
  const int e = tid < R ? sel[tid] : -1;
  if (e >= 0) atomicOr(&s_mask[e][tid >> 5], 1u << (tid & 31));
  __syncthreads();
  if (tid < E) {
    int c = 0;
    for (int w = 0; w < nw; ++w) c += __popc(s_mask[tid][w]);
    s_tot[tid] = c;
  }
  __syncthreads();
  dispatch_offsets(a, s_tot, s_off, true);
  if (e >= 0) {
    int rank = __popc(s_mask[e][tid >> 5] & ((1u << (tid & 31)) - 1u));
    for (int w = 0; w < (tid >> 5); ++w) rank += __popc(s_mask[e][w]);
    const int pos = s_off[e] + rank;
    a.route_tok[pos] = tid / a.top_k;
    a.route_slot[pos] = tid;
  }
}

// The whole grouping in one work-group; `sel` is the selected experts of
// every route in route order (global memory or LDS).
__device__ __forceinline__ void dispatch_body(const DispatchArgs& a, const int* sel) {
  const int tid = threadIdx.x;
  __shared__ int s_tot[kMaxExperts];
  __shared__ int s_off[kMaxExperts];
  for (int e = tid; e < kMaxExperts; e += 1024) s_tot[e] = 0;
  __syncthreads();
  for (int i = tid; i < a.routes; i += 1024) atomicAdd(&s_tot[sel[i]], 1);
  __syncthreads();
  dispatch_offsets(a, s_tot, s_off, true);
  dispatch_place(a, sel, 0, a.routes, s_off);
}


// stable_top_k order (route_better) as one unsigned 64-bit key per (logit,
// expert) for the fused kernel: NaN ranks as -inf and -0.0 as +0.0 (they
// compare equal as floats), the float bits are mapped to an order-preserving
// unsigned word, and the low word is ~e so that equal logits favour the lower
// index. A larger key is a better route; key 0 is below every real key.
__device__ __forceinline__ uint64_t route_key(float v, int e) {
  v = isnan(v) ? -INFINITY : v;
  v = v + 0.0f;  // -0.0 -> +0.0
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)u << 32) | (uint64_t)(~(uint32_t)e);
}
__device__ __forceinline__ int route_key_expert(uint64_t key) { return key == 0 ? 0 : (int)(~(uint32_t)key); }

// One step of a running top-K list of keys, sorted best first (slots k >= K
// stay 0). A key enters at the first slot it beats; the slots it beats form a
// suffix of the sorted list, so after all experts the list equals K rounds of
// argmax (the order is strict: keys are distinct). Branch-free.
template <int KMAX>
__device__ __forceinline__ void topk_insert(uint64_t (&keys)[KMAX], const uint64_t key, const int K) {
  bool beats[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) beats[k] = (k < K) & (key > keys[k]);
#pragma unroll
  for (int k = KMAX - 1; k >= 1; --k) keys[k] = beats[k - 1] ? keys[k - 1] : (beats[k] ? key : keys[k]);
  keys[0] = beats[0] ? key : keys[0];
}

// stable_top_k and the routing softmax of one row by T lanes (T a power of two
// dividing 64 and >= K, consecutive lanes): lane j scans experts j, j + T,
// ..., then a butterfly over the T lanes merges the lists (the top K of a
// strictly ordered set is unique, so the merged list is the sequential one).
// Lanes j < K finish rank j of the softmax. `lg`: the row's logits in LDS;
// `tab`: kExp2Tab. Every lane of the wave must call this (the shuffles);
// has_row = false lanes carry empty lists and write nothing.
template <int KMAX>
__device__ __forceinline__ void select_row_lanes(const float* lg, bool has_row, int j, int T, int E, int K, int* sel,
                                                 float* w, int* sel_copy, const uint64_t* tab) {
  uint64_t keys[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) keys[k] = 0;
  // Loops stay rolled: this code runs once per launch from a cold
  // instruction cache, so its size costs more than its instruction count.
  if (has_row) {
#pragma unroll 1
    for (int e = j; e < E; e += T) topk_insert<KMAX>(keys, route_key(lg[e], e), K);
  }
#pragma unroll 1
  for (int o = 1; o < T; o <<= 1) {
    uint64_t pk[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      const uint32_t lo = __shfl_xor((uint32_t)keys[k], o);
      const uint32_t hi = __shfl_xor((uint32_t)(keys[k] >> 32), o);
      pk[k] = ((uint64_t)hi << 32) | lo;
    }
#pragma unroll
    for (int k = 0; k < KMAX; ++k) topk_insert<KMAX>(keys, pk[k], K);
  }
  // Softmax over the selected logits in rank order (select_row's float
  // operations): lane j < K of the row holds rank j. Every lane computes the
  // same max (fmaxf folded in rank order); lane j computes its exponential;
  // the sum is folded in rank order from 0.0f by shuffles and broadcast.
  const int rank = j < K ? j : 0;
  uint64_t mine = keys[0];
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    if (k < K) {
      int ek = route_key_expert(keys[k]);
      if (ek < 0 || ek >= E) ek = 0;
      mx = fmaxf(mx, lg[ek]);
    }
    mine = k == rank ? keys[k] : mine;
  }
  int my_e = route_key_expert(mine);
  if (my_e < 0 || my_e >= E) my_e = 0;
  const float ex = expf_glibc(lg[my_e] - mx, tab);
  const int row_lane0 = (threadIdx.x & 63) - j;
  float sum = 0.0f;
#pragma unroll 1
  for (int k = 0; k < K; ++k) sum = sum + __shfl(ex, row_lane0 + k);
  if (has_row && j < K) {
    sel[j] = my_e;
    w[j] = bf16r(ex / sum);
    sel_copy[j] = my_e;
  }
}

// Fused selection and dispatch for batches whose logits fit one work-group
// (m * (experts + 1) <= kSelectLds floats): work-group 0 reads every row's
// logits into LDS (injected ones are bf16-rounded here, as route_kernel does;
// rows padded to experts + 1 floats so that lanes on consecutive rows hit
// different banks), selects per row with one lane per row, and runs the
// dispatch on the LDS copy of the selections. Work-groups 1.. quantize the
// gate_up input when no route_kernel ran: kSelectQuantBlocks blocks of 32
// values each, one per half wave.
constexpr int kSelectQuantBlocks = 32;

// Quantization work-group `qwg` of the select kernels: kSelectQuantBlocks
// blocks of 32 values, one per half wave. With r.norm_w the values are the
// post-attention RMSNorm of their row rounded to bf16 (norm_boundary,
// cpu_runner.rs:2680-2687); the inverse RMS of every row the work-group
// touches is computed first, by the whole work-group (uniform loop).
__device__ __forceinline__ void select_quantize(const RouteArgs& r, int qwg) {
  const int tid = threadIdx.x;
  const int blocks = r.hidden / kBlock;
  const int g0 = qwg * kSelectQuantBlocks, g = g0 + (tid >> 5), row = g / blocks;
  float inv = 1.0f;
  if (r.norm_w) {
    const int last = min(g0 + kSelectQuantBlocks, r.m * blocks) - 1;
    for (int rr = g0 / blocks; rr <= last / blocks; ++rr) {
      const float v = row_inverse_rms(r.x + (size_t)rr * r.hidden, r.hidden, r.norm_eps);
      if (rr == row) inv = v;
    }
  }
  if (g < r.m * blocks) {  // uniform per half wave
    const int b = g % blocks, i = b * kBlock + (tid & 31);
    float v = bf16_to_f32(r.x[(size_t)row * r.hidden + i]);
    if (r.norm_w) v = bf16r(v * inv * r.norm_w[i]);
    if (r.qmode != kProjExactBf16 && !isfinite(v)) atomicOr(r.err, kErrNonFiniteInput);
    residual_q8_store(v, tid & 31, (size_t)row, blocks, b, r.act, r.qmode);
  }
}

// stable_top_k and the routing softmax of one row by one wave (experts <=
// kMaxExperts): lane e holds the keys of experts e and e + 64, and a key's
// rank is the number of larger keys among all experts (keys are distinct, so
// ranks are too); ranks below K are the selection in stable_top_k order. The
// softmax then follows select_row_lanes's operations: max folded in rank
// order, each rank's exponential, the sum folded in rank order from 0.0f.
// `ws`: this wave's LDS scratch (keys, picks, exponentials).
struct RankScratch {
  uint64_t key[kMaxExperts];
  int pick[kMaxTopK];
  float ex[kMaxTopK];
};

__device__ __forceinline__ void select_row_ranked(const RouteArgs& r, const float* lg, int row, int* s_sel,
                                                  const uint64_t* tab, RankScratch& ws) {
  const int lane = threadIdx.x & 63;
  const int E = r.experts, K = r.top_k;
  const uint64_t k0 = lane < E ? route_key(lg[lane], lane) : 0;
  const uint64_t k1 = lane + 64 < E ? route_key(lg[lane + 64], lane + 64) : 0;
  ws.key[lane] = k0;
  ws.key[lane + 64] = k1;
  __builtin_amdgcn_wave_barrier();  // LDS of one wave is in order: the keys are in place
  int r0 = 0, r1 = 0;
#pragma unroll 8
  for (int f = 0; f < E; ++f) {
    const uint64_t kf = ws.key[f];
    r0 += kf > k0;
    r1 += kf > k1;
  }
  if (lane < E && r0 < K) ws.pick[r0] = lane;
  if (lane + 64 < E && r1 < K) ws.pick[r1] = lane + 64;
  __builtin_amdgcn_wave_barrier();
  float mx = -INFINITY;
  for (int k = 0; k < K; ++k) mx = fmaxf(mx, lg[ws.pick[k]]);
  const int my_e = ws.pick[lane < K ? lane : 0];
  const float ex = expf_glibc(lg[my_e] - mx, tab);
  if (lane < K) ws.ex[lane] = ex;
  __builtin_amdgcn_wave_barrier();
  float sum = 0.0f;
  for (int k = 0; k < K; ++k) sum = sum + ws.ex[k];
  if (lane < K) {
    r.selected[(size_t)row * K + lane] = my_e;
    r.weights[(size_t)row * K + lane] = bf16r(ex / sum);
    s_sel[row * K + lane] = my_e;
  }
  __builtin_amdgcn_wave_barrier();  // the next row's key writes follow this row's reads
}

// Selection and dispatch of m <= kFusedRouteRows rows by one wave, with no
// work-group barrier (route_select_kernel's last router work-group). The
// logits are read with device-scope atomic loads. Routes R = m * top_k and
// every bucket holds at most m <= chunk routes, so each touched expert is one
// partial work item, and dispatch_offsets's order reduces to descending size,
// ties by expert. Route i of expert e goes to bucket_off[e] + #{j < i routed
// to e} (stable_group_routes).
__device__ __forceinline__ void select_dispatch_tiny(const RouteArgs& r, const DispatchArgs& d) {
  const int lane = threadIdx.x & 63;
  const int E = r.experts, K = r.top_k, M = r.m, R = M * K;
  __shared__ float s_lg[kFusedRouteRows][kMaxExperts];
  __shared__ int s_sel[kFusedRouteRows * kMaxTopK];
  __shared__ int s_cnt[kMaxExperts], s_off[kMaxExperts], s_nz[kFusedRouteRows * kMaxTopK];
  __shared__ uint64_t s_tab[32];
  __shared__ RankScratch s_rank;
  if (lane < 32) s_tab[lane] = kExp2Tab[lane];
  for (int i = lane; i < M * E; i += 64) {
    const float v = __hip_atomic_load(r.logits + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (!isfinite(v)) atomicOr(r.err, kErrNonFiniteLogits);
    s_lg[i / E][i % E] = v;
  }
  __builtin_amdgcn_wave_barrier();
  for (int row = 0; row < M; ++row) select_row_ranked(r, s_lg[row], row, s_sel, s_tab, s_rank);
  // Per-expert counts and their exclusive scan (experts lane and lane + 64).
  int c0 = 0, c1 = 0;
  for (int j = 0; j < R; ++j) {
    const int e = s_sel[j];
    c0 += e == lane;
    c1 += e == lane + 64;
  }
  int i0 = c0, i1 = c1;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u0 = __shfl_up(i0, o), u1 = __shfl_up(i1, o);
    if (lane >= o) {
      i0 += u0;
      i1 += u1;
    }
  }
  const int total0 = __shfl(i0, 63);
  const int off0 = i0 - c0, off1 = total0 + i1 - c1;
  if (lane < E) {
    s_cnt[lane] = c0;
    s_off[lane] = off0;
    d.bucket_off[lane] = off0;
  }
  if (lane + 64 < E) {
    s_cnt[lane + 64] = c1;
    s_off[lane + 64] = off1;
    d.bucket_off[lane + 64] = off1;
  }
  if (lane == 0) d.bucket_off[E] = R;
  // Touched experts in expert order (ballots over the two halves).
  const unsigned long long m0 = __ballot(lane < E && c0 > 0), m1 = __ballot(lane + 64 < E && c1 > 0);
  const unsigned long long below = (1ull << lane) - 1ull;
  const int nz0 = __popcll(m0);
  if (lane < E && c0 > 0) s_nz[__popcll(m0 & below)] = lane;
  if (lane + 64 < E && c1 > 0) s_nz[nz0 + __popcll(m1 & below)] = lane + 64;
  const int n_items = nz0 + __popcll(m1);
  __builtin_amdgcn_wave_barrier();
  // Route lane i: its rank among earlier routes of its expert, then its place.
  if (lane < R) {
    const int e = s_sel[lane];
    int rank = 0;
    for (int j = 0; j < lane; ++j) rank += s_sel[j] == e;
    const int pos = s_off[e] + rank;
    d.route_tok[pos] = lane / K;
    d.route_slot[pos] = lane;
  }
  // Work item of touched expert lane (< n_items): records by descending
  // size, ties by expert.
  if (lane < n_items) {
    const int e = s_nz[lane], c = s_cnt[e];
    int before = 0;
    for (int j = 0; j < n_items; ++j) {
      const int f = s_nz[j], cf = s_cnt[f];
      before += cf > c || (cf == c && f < e);
    }
    reinterpret_cast<int4*>(d.work)[before] = make_int4(e, s_off[e], c, 0);
  }
  if (lane == 0) *d.n_work = n_items;
}

// Top-k, softmax and dispatch of every row by one work-group of 1024 threads.
// The outputs are stored after the last work-group barrier, from LDS, so that
// no store's address and data computation sits between the phases.
__device__ __forceinline__ void select_dispatch_body(const RouteArgs& r, const DispatchArgs& d) {
  const int tid = threadIdx.x;
  const int E = r.experts, K = r.top_k, M = r.m, stride = E + 1;
  __shared__ float s_lg[kSelectLds];
  __shared__ int s_sel[kSelectMaxRoutes];
  __shared__ float s_w[kSelectMaxRoutes];
  __shared__ uint64_t s_tab[32];
  if (tid < 32) s_tab[tid] = kExp2Tab[tid];
  // Element i is (i / E, i % E), the quotient by a multiply-high (exact for
  // i < 2^32 / E). Loops stay short and rolled: this code runs once per
  // launch from a cold instruction cache.
  const uint32_t inv_e = 0xffffffffu / (uint32_t)E + 1u;
  bool bad = false;
#pragma unroll 2
  for (int i = tid; i < M * E; i += 1024) {
    float v = r.injected != nullptr ? r.injected[i] : r.logits[i];
    if (r.injected != nullptr) v = bf16r(v);
    bad = bad || !isfinite(v);
    const int row = (int)__umulhi((uint32_t)i, inv_e);
    s_lg[row * stride + (i - row * E)] = v;
  }
  if (bad) atomicOr(r.err, kErrNonFiniteLogits);
  __syncthreads();
  // T lanes per row: the largest power of two <= 64 with T * M <= 1024 and T
  // <= E / 4 (a few experts per lane), but at least top_k (<= 4).
  int T = 64;
  while (T > 1 && (T * M > 1024 || 4 * T > E)) T >>= 1;
  while (T < K) T <<= 1;
  const int rows_per_pass = 1024 / T;
  for (int base = 0; base < M; base += rows_per_pass) {  // uniform
    // A row's T lanes share a wave: waves whose first row is past the batch
    // have nothing to select and skip (wave-uniform).
    if (base + (tid & ~63) / T >= M) continue;
    const int row = base + tid / T, j = tid % T;
    const bool has_row = row < M;
    const int rr = has_row ? row : 0;
    select_row_lanes<kSelectTopK>(s_lg + rr * stride, has_row, j, T, E, K, s_sel + rr * K, s_w + rr * K,
                                  s_sel + rr * K, s_tab);
  }
  __syncthreads();
  if (d.routes <= kMaskRoutes) dispatch_body_masked(d, s_sel);
  else dispatch_body(d, s_sel);
  // No barrier follows: the selection, weights and (injected) logits.
  for (int i = tid; i < M * K; i += 1024) {
    r.selected[i] = s_sel[i];
    r.weights[i] = s_w[i];
  }
  if (r.injected != nullptr && r.logits != nullptr) {
    for (int i = tid; i < M * E; i += 1024) {
      const int row = (int)__umulhi((uint32_t)i, inv_e);
      r.logits[i] = s_lg[row * stride + (i - row * E)];
    }
  }
}

__global__ __launch_bounds__(1024) void select_dispatch_kernel(RouteArgs r, DispatchArgs d) {
  if (blockIdx.x > 0) {
    select_quantize(r, (int)blockIdx.x - 1);
    return;
  }
  select_dispatch_body(r, d);
}

// Router, selection and dispatch of a small batch (m <= kFusedRouteRows,
// hidden <= kFusedRouteHidden) in one launch. Work-group e < experts
// computes expert e's logit for every row: the rows (normalized as
// route_kernel does) and the router row are staged in LDS, lane l of a row
// sums w[i] * x[i] over i = l mod 16 in increasing i (scalar_bf16_dot,
// lib.rs:1007-1029), the lanes are added 0..15, then bias and bf16
// (cpu_runner.rs:2781-2783, 2829). Each work-group releases its logits
// (device-scope release fence) and counts itself on `counter`; the last one
// to arrive (it has seen every other count) reads them all with device-scope
// atomic loads, resets the counter for the next launch and selects and
// dispatches with one wave (select_dispatch_tiny). Work-groups past the
// experts quantize the gate_up input (select_quantize). With a null counter
// the launch writes the logits only.
__global__ __launch_bounds__(1024) void route_select_kernel(RouteArgs r, DispatchArgs d, int* counter) {
  const int tid = threadIdx.x;
  const int E = r.experts, H = r.hidden, M = r.m;
  if ((int)blockIdx.x >= E) {
    select_quantize(r, (int)blockIdx.x - E);
    return;
  }
  const int e = blockIdx.x;
  // Products w[i] * x[i] (f32, rounded as the reference's multiply) by chain
  // lane: element i of a row sits at [i % 16][i / 16] (lanes padded by 16
  // bytes against bank conflicts), so lane l adds its products 4 at a time in
  // increasing i; the pad up to a multiple of 4 is +0.0, which leaves the
  // chain unchanged (it is never -0.0).
  constexpr int kLane = kFusedRouteHidden / 16 + 4;
  __shared__ __align__(16) float s_pt[kFusedRouteRows][16][kLane];
  __shared__ float s_chain[kFusedRouteRows][16];
  __shared__ float s_inv[kFusedRouteRows];
  __shared__ int s_last;
  if (r.norm_w) {
    for (int rr = 0; rr < M; ++rr) {  // uniform
      const float v = row_inverse_rms(r.x + (size_t)rr * H, H, r.norm_eps);
      if (tid == 0) s_inv[rr] = v;
    }
    __syncthreads();
  }
  const int per_lane = H / 16, padded = (per_lane + 3) & ~3;
  for (int v = tid; v < M * 16 * (padded - per_lane); v += 1024) {  // the pad
    const int rr = v / (16 * (padded - per_lane)), rest = v % (16 * (padded - per_lane));
    s_pt[rr][rest / (padded - per_lane)][per_lane + rest % (padded - per_lane)] = 0.0f;
  }
  const int pieces = H / 8;  // 16-byte pieces: elements 8c..8c+7 are lanes (8c) % 16 + 0..7 at k = c / 2
  for (int v = tid; v < M * pieces; v += 1024) {
    const int rr = v / pieces, c = v - rr * pieces;
    const int l0 = (c & 1) * 8, k = c >> 1;
    const u32x4 wv = reinterpret_cast<const u32x4*>(r.router_w + (size_t)e * H)[c];
    const u32x4 xv = reinterpret_cast<const u32x4*>(r.x + (size_t)rr * H)[c];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      float lo = bf16_to_f32((uint16_t)(xv[q] & 0xffffu)), hi = bf16_to_f32((uint16_t)(xv[q] >> 16));
      if (r.norm_w) {  // post-attention RMSNorm, bf16 (norm_boundary; route_input)
        const int i = c * 8 + 2 * q;
        lo = bf16r(lo * s_inv[rr] * r.norm_w[i]);
        hi = bf16r(hi * s_inv[rr] * r.norm_w[i + 1]);
      }
      s_pt[rr][l0 + 2 * q][k] = __uint_as_float(wv[q] << 16) * lo;
      s_pt[rr][l0 + 2 * q + 1][k] = __uint_as_float(wv[q] & 0xffff0000u) * hi;
    }
  }
  __syncthreads();
  if (tid < M * 16) {
    const int rr = tid >> 4, l = tid & 15;
    const float4* pl = reinterpret_cast<const float4*>(s_pt[rr][l]);
    float acc = 0.0f;
#pragma unroll 4
    for (int c = 0; c < padded / 4; ++c) {
      const float4 v = pl[c];
      acc = acc + v.x;
      acc = acc + v.y;
      acc = acc + v.z;
      acc = acc + v.w;
    }
    s_chain[rr][l] = acc;
  }
  __syncthreads();
  if (tid < M) {
    float sum = s_chain[tid][0];
    for (int j = 1; j < 16; ++j) sum = sum + s_chain[tid][j];
    r.logits[(size_t)tid * E + e] = bf16r(sum + r.router_b[e]);
    if (counter != nullptr) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");  // the logit reaches device scope before the count
  }
  if (counter == nullptr) return;  // logits only (route_gemv_kernel selects in the next launch)
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(counter, 1) == E - 1;
  __syncthreads();
  if (!s_last) return;
  if (tid == 0) atomicExch(counter, 0);
  if (tid < 64) select_dispatch_tiny(r, d);
}

// Selection and grouping of batches past the fused kernel's limits, in two
// launches. select_count_kernel: work-group w selects rows [w RW, w RW + RW)
// with T = 1024 / RW lanes per row (RW a power of two with RW * (E + 1) <=
// kSelectLds and RW * top_k <= 1024, so T >= top_k) and writes the per-expert
// route counts of its rows to cnt[w][E]; work-groups past the selection ones
// quantize the gate_up input when no route_kernel ran. place_kernel: work-group
// w places the routes of the same rows at bucket_off[e] + (routes of expert e
// in earlier work-groups) + (rank within its own routes); work-group 0 also
// writes bucket_off and the work list.
template <int KMAX>
__global__ __launch_bounds__(1024) void select_count_kernel(RouteArgs r, int rows_per_wg, int n_sel, int* cnt) {
  const int tid = threadIdx.x;
  if ((int)blockIdx.x >= n_sel) {
    select_quantize(r, (int)blockIdx.x - n_sel);
    return;
  }
  const int E = r.experts, K = r.top_k, stride = E + 1;
  const int r0 = (int)blockIdx.x * rows_per_wg, nrows = min(rows_per_wg, r.m - r0);
  __shared__ float s_lg[kSelectLds];
  __shared__ int s_sel[1024];
  __shared__ int s_cnt[kMaxExperts];
  __shared__ uint64_t s_tab[32];
  if (tid < 32) s_tab[tid] = kExp2Tab[tid];
  if (tid < kMaxExperts) s_cnt[tid] = 0;
  // Unrolled so that a thread's loads go out together.
#pragma unroll 4
  for (int i = tid; i < nrows * E; i += 1024) {
    const size_t gi = (size_t)r0 * E + i;
    float v;
    if (r.injected != nullptr) {
      v = bf16r(r.injected[gi]);
      if (r.logits) r.logits[gi] = v;
    } else {
      v = r.logits[gi];
    }
    if (!isfinite(v)) atomicOr(r.err, kErrNonFiniteLogits);
    s_lg[(i / E) * stride + i % E] = v;
  }
  __syncthreads();
  const int T = 1024 / rows_per_wg;
  const int lr = tid / T, j = tid % T;
  const bool has_row = lr < nrows;
  const int rr = has_row ? lr : 0;
  if ((tid & ~63) / T < nrows)  // waves with no row of the batch skip (wave-uniform)
    select_row_lanes<KMAX>(s_lg + rr * stride, has_row, j, T, E, K, r.selected + (size_t)(r0 + rr) * K,
                           r.weights + (size_t)(r0 + rr) * K, s_sel + rr * K, s_tab);
  __syncthreads();
  for (int i = tid; i < nrows * K; i += 1024) atomicAdd(&s_cnt[s_sel[i]], 1);
  __syncthreads();
  if (tid < E) cnt[(size_t)blockIdx.x * E + tid] = s_cnt[tid];
}

__global__ __launch_bounds__(1024) void place_kernel(DispatchArgs a, int routes_per_wg, int n_sel, const int* cnt) {
  const int tid = threadIdx.x, E = a.experts, w = blockIdx.x;
  __shared__ int s_tot[kMaxExperts];
  __shared__ int s_pre[kMaxExperts];
  __shared__ int s_off[kMaxExperts];
  if (tid < kMaxExperts) {
    int tot = 0, pre = 0;
    if (tid < E) {
      // Eight selection work-groups' counts requested at a time.
      for (int v0 = 0; v0 < n_sel; v0 += 8) {  // uniform
        int cv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) cv[i] = v0 + i < n_sel ? cnt[(size_t)(v0 + i) * E + tid] : 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          tot += cv[i];
          if (v0 + i < w) pre += cv[i];
        }
      }
    }
    s_tot[tid] = tot;
    s_pre[tid] = pre;
  }
  __syncthreads();
  dispatch_offsets(a, s_tot, s_off, w == 0);
  if (tid < E) s_off[tid] += s_pre[tid];
  __syncthreads();
  const int begin = w * routes_per_wg;
  dispatch_place(a, a.selected, begin, min(a.routes, begin + routes_per_wg), s_off);
}

// ---------------------------------------------------------------------------
// Expert GEMM on the resident v3 layout. One work-group = C::kWaves waves,
// C::kWaveTiles 16-row weight tiles per wave (C::kGemmRows rows), times one
// work item of at most C::kChunk activation rows. Each lane owns one weight
// row (lane % 16) per tile and two activation rows per group of 8, and runs
// the reference's per-row float chain in order:
//   total = bias; for each block: total += (p * ws) * ps; total += (r * ws) * rs
// (mxfp4_residual_q8_gemv_rows lib.rs:673-696, scalar_matmul_range
// matmul.rs:529-578).
//
// Pipeline: K advances in steps of C::kStep blocks (C::kGroups 4-block groups
// of the v3 layout). Each wave keeps its tiles' nibbles (one 16-byte load per
// lane, tile and group) and scale dwords three steps deep in a register ring.
// The step's activations (f16 codes and scales) move from global memory into
// a ring of three LDS slots by DMA (buffer_load ... lds) two steps ahead,
// published by one barrier per step. Every wave issues the same vector-memory
// instructions in the same order, so one s_waitcnt immediate covers every
// step, and all per-step addressing is scalar.

__device__ __forceinline__ half8 fp4x8_to_half8(uint32_t w) {
  const half2v h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 0);
  const half2v h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 1);
  const half2v h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 2);
  const half2v h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, 1.0f, 3);
  half8 b;
  b[0] = h0[0]; b[1] = h0[1]; b[2] = h1[0]; b[3] = h1[1];
  b[4] = h2[0]; b[5] = h2[1]; b[6] = h3[0]; b[7] = h3[1];
  return b;
}

// E8M0 bytes whose scaled E2M1 values are exact f16 normals: 0.5 * 2^(s-127)
// >= 2^-14 and 6 * 2^(s-127) <= 65504.
constexpr uint32_t kFastScaleLo = 114, kFastScaleHi = 139;

__device__ __forceinline__ half8 fp4x8_to_half8_scaled(uint32_t w, float scale) {
  const half2v h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 0);
  const half2v h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 1);
  const half2v h2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 2);
  const half2v h3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, scale, 3);
  half8 b;
  b[0] = h0[0]; b[1] = h0[1]; b[2] = h1[0]; b[3] = h1[1];
  b[4] = h2[0]; b[5] = h2[1]; b[6] = h3[0]; b[7] = h3[1];
  return b;
}

// The scale operand of fp4x8_to_half8_scaled for E8M0 byte j of the dword s
// (j a compile-time constant): one shift that moves the byte into the f32
// exponent field. v_cvt_scalef32_pk_f16_fp4 reads only that field of its
// scale operand (a probe over every FP4 byte, exponents 100..154 and set sign
// and mantissa bits found no difference from the clean 2^(e - 127) scale), so
// the neighbouring bytes that land in the sign and mantissa do not matter.
__device__ __forceinline__ float e8m0_scale_operand(uint32_t s, int j) {
  return __uint_as_float(j == 3 ? s >> 1 : s << (23 - 8 * j));
}

// e8m0_scale without branches (lib.rs:957-963).
__device__ __forceinline__ float e8m0_select(uint32_t s) {
  const float normal = __uint_as_float(s << 23);
  const float v = s == 0u ? __uint_as_float(0x00400000u) : normal;
  return s == 0xffu ? __uint_as_float(0x7fc00000u) : v;
}

typedef __attribute__((address_space(3))) void* lds_ptr;

// Geometry of one GEMM instantiation. TILES 16-row weight tiles per wave,
// work items of NTOK activation rows (NTOK / 8 MFMA token groups), K steps of
// GROUPS 4-block groups, WAVES waves per work-group, and MIN_WAVES waves per
// SIMD that the register budget must allow.
//  GemmBig (2 tiles, 16 rows, 4 blocks, 4 waves) serves batches of 9..511
//    rows: 96 VGPRs and 27.7 KB of LDS give 5 work-groups per CU, 5 waves per
//    SIMD to hide the LDS and MFMA latency of the ordered chain.
//  GemmSmall (1 tile, 8 rows, 8 blocks, 4 waves) serves batches of at most 8
//    rows, whose work items are one expert each and whose time is the weight
//    stream's latency: 64-row work-groups (four times the big geometry's
//    count per expert), 73 VGPRs, 5 work-groups per CU.
//  GemmHuge (2 tiles, 32 rows, 4 blocks, 8 waves) serves prefill-sized
//    batches, where the FP4->f16 conversion of a weight block is shared by
//    four token groups. Its gate_up grid pins weight tiles to XCDs (PIN_XCD).
//
// PIN_XCD: work-groups reach the eight XCDs round-robin in launch order, so
// with a grid row of n_x work-groups the chunks of one expert (consecutive
// rows) would read the same tile through different L2s whenever n_x is not a
// multiple of 8. A pinned gate_up grid pads its rows to a multiple of 8
// (padding work-groups return at once) and rotates each row by the item's
// expert, so tile column x of expert e always runs on XCD (x + e) mod 8: the
// later chunks of a popular expert hit the L2 the first one filled, and the
// XCDs that get one column fewer differ from expert to expert. It pays when
// experts have many chunks (prefill); with one or two chunks per expert the
// padding's imbalance costs more than the L2 hits save.
template <int TILES, int NTOK, int GROUPS, int WAVES = 8, int MIN_WAVES = 4, int WLEAD = 2, bool PIN_XCD = false>
struct GemmCfg {
  static constexpr int kWaves = WAVES;                    // waves per work-group
  static constexpr int kThreads = 64 * WAVES;
  static constexpr int kMinWaves = MIN_WAVES;             // waves per SIMD the register budget must allow
  static constexpr int kSclSlot = 64 * WAVES;             // floats written by one step's scale DMA (a dword per lane)
  static constexpr int kWaveTiles = TILES;
  static constexpr int kWgTiles = WAVES * TILES;
  static constexpr int kGemmRows = kTileRows * kWgTiles;  // weight rows per work-group
  static constexpr int kChunk = NTOK;                     // activation rows per work item
  static constexpr int kNtg = NTOK / 8;                   // MFMA token groups per work item
  static constexpr int kGroups = GROUPS;                  // 4-block groups per step
  static constexpr int kStep = 4 * GROUPS;                // K blocks per pipeline step
  static constexpr int kSlotBytes = kStep * NTOK * 2 * kBlock * 2;  // f16 codes of one step in LDS
  static constexpr int kCodeDma = kSlotBytes / (16 * kThreads);  // 16-byte DMA per lane per step
  // Vector-memory instructions per wave and step: weights GROUPS x (nibbles,
  // scale dword) per tile; activations kCodeDma code pieces + 1 scale dword.
  static constexpr int kLoadsW = 2 * GROUPS * TILES;
  static constexpr int kLoadsD = kCodeDma + 1;
  // Steps by which the weight requests lead their use (1 or 2; the DMA leads
  // by 2).
  static constexpr int kWLead = WLEAD;
  static constexpr bool kPinXcd = PIN_XCD;  // gate_up grid rows pinned to XCDs (above)
  // s_waitcnt immediate for "the DMA and the weights of step q have landed":
  // issued after them are D(q+1) and, with a two-step lead, W(q+1) (see
  // k_loop). expcnt and lgkmcnt are not waited on.
  static constexpr int kWaitVm = (WLEAD == 2 ? kLoadsW : 0) + kLoadsD;
  static constexpr int kWaitDma = (kWaitVm & 15) | ((kWaitVm >> 4) << 14) | (7 << 4) | (15 << 8);
  static_assert(kSlotBytes == kCodeDma * 16 * kThreads, "code DMA covers a slot exactly");
  static_assert(kStep * NTOK * 2 <= kSclSlot, "one dword DMA per lane covers a step's scales");
  static_assert(NTOK % 8 == 0 && NTOK <= kChunkMax, "token groups of 8");
  static_assert(kGemmRows % 64 == 0, "a work-group's gate_up rows make whole 32-value down-input blocks");
  static_assert(kWaitVm < 64, "vmcnt field");
  static_assert(WLEAD == 1 || WLEAD == 2, "weight lead");
  static_assert((kStep - 1) * 2 * kBlock * 2 <= (int)kActSlack, "a last partial step reads inside the slack");
};
using GemmBig = GemmCfg<2, 16, 1, 4, 5>;
using GemmSmall = GemmCfg<1, 8, 2, 4, 5>;
using GemmHuge = GemmCfg<2, 32, 1, 8, 4, 1, true>;
static_assert(GemmBig::kChunk == kChunk && GemmSmall::kChunk == kSmallChunk && GemmHuge::kChunk == kHugeChunk,
              "work item sizes");
constexpr int kBufferFlags = 0x00020000;    // raw 32-bit buffer resource, gfx9 family

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, kBufferFlags);
}

// One step of a wave's weights: per group of the step and tile, the nibble
// group and its scale dword.
template <class C>
struct WStep {
  u32x4 v[C::kGroups][C::kWaveTiles];
  uint32_t s[C::kGroups][C::kWaveTiles];
};

// Accumulators of one wave: [tile][token group][token of the lane's pair].
template <class C>
using Acc = float[C::kWaveTiles][C::kNtg][2];

// LDS slot layout of one step (written by DMA, read as MFMA A operands): for
// block j and token group tg, 1 KiB = [k-slice g (4)][vector i (16)][16 B]
// with vector i = 2 * (row within the group) + part (0 primary, 1 residual),
// so lane (g, i) of a wave reads the 16 bytes at lane * 16 (conflict-free).
// Scales: float2 (primary, residual) at [j][row].
template <class C>
__device__ __forceinline__ int slot_chunk(int j, int tg) { return j * C::kNtg + tg; }

// One block j of the current step against NTG token groups and the wave's
// tiles: one A operand and one scale read per token group feed an MFMA per
// tile, then the ordered chain updates. SCALED: the weight operand already
// carries the E8M0 scale (exact), so the MFMA returns (p / 2) * e8m0 and a
// term is d * act_scale; otherwise a term is (d * e8m0) * act_scale. Both are
// the reference's (p * (0.5 * e8m0)) * act_scale rounded once.
template <class C, bool RESIDUAL, bool SCALED, int NTG>
__device__ __forceinline__ void block_update(Acc<C>& tot, const char* codes, const float2* scl,
                                             const half8 (&bop)[C::kWaveTiles], const float (&e8)[C::kWaveTiles],
                                             const int j, const int lane, const int G) {
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int tg = 0; tg < NTG; ++tg) {
    const half8 aop = *reinterpret_cast<const half8*>(codes + slot_chunk<C>(j, tg) * 1024 + lane * 16);
    const float4 sc = *reinterpret_cast<const float4*>(&scl[j * C::kChunk + tg * 8 + 2 * G]);
    f32x4 d[C::kWaveTiles];
#pragma unroll
    for (int t = 0; t < C::kWaveTiles; ++t) d[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop[t], zero, 0, 0, 0);
#pragma unroll
    for (int t = 0; t < C::kWaveTiles; ++t) {
      if (SCALED) {
        tot[t][tg][0] = tot[t][tg][0] + d[t][0] * sc.x;
        if (RESIDUAL) tot[t][tg][0] = tot[t][tg][0] + d[t][1] * sc.y;
        tot[t][tg][1] = tot[t][tg][1] + d[t][2] * sc.z;
        if (RESIDUAL) tot[t][tg][1] = tot[t][tg][1] + d[t][3] * sc.w;
      } else {
        tot[t][tg][0] = tot[t][tg][0] + (d[t][0] * e8[t]) * sc.x;
        if (RESIDUAL) tot[t][tg][0] = tot[t][tg][0] + (d[t][1] * e8[t]) * sc.y;
        tot[t][tg][1] = tot[t][tg][1] + (d[t][2] * e8[t]) * sc.z;
        if (RESIDUAL) tot[t][tg][1] = tot[t][tg][1] + (d[t][3] * e8[t]) * sc.w;
      }
    }
  }
}

// The first nb blocks of one 4-block group (per tile: nibble dwords v, scale
// bytes s) at step-relative block jb. FAST: every scale of the wave's tiles is
// in [kFastScaleLo, kFastScaleHi] (checked when the weights were stored), so
// the conversion applies the scale exactly; otherwise the scale multiplies
// the MFMA result, with the reference's 0x00 and 0xff encodings.
template <class C, bool RESIDUAL, int NTG, bool FAST>
__device__ __forceinline__ void group_update(Acc<C>& tot, const char* codes, const float2* scl,
                                             const u32x4 (&v)[C::kWaveTiles], const uint32_t (&s)[C::kWaveTiles],
                                             const int jb, const int nb, const int lane, const int G) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (j < nb) {
      half8 bop[C::kWaveTiles];
      float e8[C::kWaveTiles];
#pragma unroll
      for (int t = 0; t < C::kWaveTiles; ++t) {
        const uint32_t sb = (s[t] >> (8 * j)) & 0xffu;
        if (FAST) {
          bop[t] = fp4x8_to_half8_scaled(v[t][j], e8m0_scale_operand(s[t], j));
          e8[t] = 0.0f;
        } else {
          bop[t] = fp4x8_to_half8(v[t][j]);
          e8[t] = e8m0_select(sb);
        }
      }
      block_update<C, RESIDUAL, FAST, NTG>(tot, codes, scl, bop, e8, jb + j, lane, G);
    }
  }
}

// group_update for one token group, all 4 blocks present and the fast path,
// software-pipelined by hand: the LDS reads of block j + 2 and the
// conversion of block j + 1 are issued before the chain of block j, and the
// MFMAs of block j + 1 right after it, so the LDS and MFMA latencies are
// covered by a block's work instead of stalling each block. Every
// accumulator sees the same operations in the same order as group_update.
template <class C, bool RESIDUAL>
__device__ __forceinline__ void group_update_pipelined(Acc<C>& tot, const char* codes, const float2* scl,
                                                       const u32x4 (&v)[C::kWaveTiles],
                                                       const uint32_t (&s)[C::kWaveTiles], const int jb,
                                                       const int lane, const int G) {
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  half8 aop[2];
  float4 sc[3];
  half8 bop[C::kWaveTiles];
  f32x4 d[C::kWaveTiles];
#define GOSSMX_LDS(J)                                                                               \
  aop[(J) & 1] = *reinterpret_cast<const half8*>(codes + slot_chunk<C>(jb + (J), 0) * 1024 + lane * 16); \
  sc[(J) % 3] = *reinterpret_cast<const float4*>(&scl[(jb + (J)) * C::kChunk + 2 * G]);
#define GOSSMX_CVT(J)                                                                               \
  _Pragma("unroll") for (int t = 0; t < C::kWaveTiles; ++t)                                        \
      bop[t] = fp4x8_to_half8_scaled(v[t][(J)], e8m0_scale_operand(s[t], (J)));
#define GOSSMX_MFMA(J)                                                                              \
  _Pragma("unroll") for (int t = 0; t < C::kWaveTiles; ++t)                                        \
      d[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop[(J) & 1], bop[t], zero, 0, 0, 0);
#define GOSSMX_CHAIN(J)                                                                             \
  _Pragma("unroll") for (int t = 0; t < C::kWaveTiles; ++t) {                                      \
    const float4 c = sc[(J) % 3];                                                                   \
    tot[t][0][0] = tot[t][0][0] + d[t][0] * c.x;                                                    \
    if (RESIDUAL) tot[t][0][0] = tot[t][0][0] + d[t][1] * c.y;                                      \
    tot[t][0][1] = tot[t][0][1] + d[t][2] * c.z;                                                    \
    if (RESIDUAL) tot[t][0][1] = tot[t][0][1] + d[t][3] * c.w;                                      \
  }
  GOSSMX_LDS(0)
  GOSSMX_LDS(1)
  GOSSMX_CVT(0)
  GOSSMX_MFMA(0)
  GOSSMX_LDS(2)
  GOSSMX_CVT(1)
  GOSSMX_CHAIN(0)
  GOSSMX_MFMA(1)
  GOSSMX_LDS(3)
  GOSSMX_CVT(2)
  GOSSMX_CHAIN(1)
  GOSSMX_MFMA(2)
  GOSSMX_CVT(3)
  GOSSMX_CHAIN(2)
  GOSSMX_MFMA(3)
  GOSSMX_CHAIN(3)
#undef GOSSMX_LDS
#undef GOSSMX_CVT
#undef GOSSMX_MFMA
#undef GOSSMX_CHAIN
}

// A full fast step with NTG >= 2 token groups, software-pipelined by one
// token group. Stage s = (block j, token group tg) issues the MFMAs of
// (j, tg), then requests the LDS operands of stage s + 1, then runs the chain
// of stage s - 1, whose MFMAs went out one stage earlier (two MFMAs and 16
// chain instructions before their results are read), and in a block's last
// stage converts the next block's weights. Every accumulator sees the same
// operations in the same order as group_update.
template <class C, bool RESIDUAL, int NTG>
__device__ __forceinline__ void step_pipelined(Acc<C>& tot, const char* codes, const float2* scl, const WStep<C>& w,
                                               const int lane, const int G) {
  constexpr int T = C::kWaveTiles, NS = C::kStep * NTG;
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  half8 aop[2];
  float4 sc[3];
  half8 bop[2][T];
  f32x4 d[2][T];
#define GOSSMX_A(S) \
  (*reinterpret_cast<const half8*>(codes + slot_chunk<C>((S) / NTG, (S) % NTG) * 1024 + lane * 16))
#define GOSSMX_S(S) (*reinterpret_cast<const float4*>(&scl[((S) / NTG) * C::kChunk + ((S) % NTG) * 8 + 2 * G]))
#define GOSSMX_CVT(J, DST)                                                                              \
  _Pragma("unroll") for (int t = 0; t < T; ++t)                                                       \
      DST[t] = fp4x8_to_half8_scaled(w.v[(J) / 4][t][(J) % 4], e8m0_scale_operand(w.s[(J) / 4][t], (J) % 4));
#define GOSSMX_CHAIN(S)                                                                                 \
  _Pragma("unroll") for (int t = 0; t < T; ++t) {                                                     \
    const float4 c = sc[(S) % 3];                                                                       \
    const f32x4 r = d[(S) & 1][t];                                                                      \
    float& p0 = tot[t][(S) % NTG][0];                                                                   \
    float& p1 = tot[t][(S) % NTG][1];                                                                   \
    p0 = p0 + r[0] * c.x;                                                                               \
    if (RESIDUAL) p0 = p0 + r[1] * c.y;                                                                 \
    p1 = p1 + r[2] * c.z;                                                                               \
    if (RESIDUAL) p1 = p1 + r[3] * c.w;                                                                 \
  }
  aop[0] = GOSSMX_A(0);
  sc[0] = GOSSMX_S(0);
  GOSSMX_CVT(0, bop[0])
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < T; ++t)
      d[s & 1][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop[s & 1], bop[(s / NTG) & 1][t], zero, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (s + 1 < NS) {
      aop[(s + 1) & 1] = GOSSMX_A(s + 1);
      sc[(s + 1) % 3] = GOSSMX_S(s + 1);
    }
    if (s > 0) GOSSMX_CHAIN(s - 1)
    if (s % NTG == NTG - 1 && s / NTG + 1 < C::kStep) GOSSMX_CVT(s / NTG + 1, bop[(s / NTG + 1) & 1])
  }
  __builtin_amdgcn_sched_barrier(0);
  GOSSMX_CHAIN(NS - 1)
#undef GOSSMX_A
#undef GOSSMX_S
#undef GOSSMX_CVT
#undef GOSSMX_CHAIN
}

// Shared GEMM epilogue: plain f32 stores, the down projection's bf16 rows,
// or gate_up's SwiGLU and down-input quantization. `s_act` is LDS scratch of
// at least count * (kGemmRows / 2 + 1) floats, free for reuse. Rows of tiles
// past the end (row >= rows) are never stored. `s_slot` (kDown, nullable):
// the item's route slots already in LDS (else they are read from route_slot).
// TABLE: the SwiGLU sigmoids are gathered from a.sig_tab (one global round
// trip, few instructions: the tiled GEMM, whose waves are VALU-bound);
// otherwise each is computed from the LDS copy of kExp2Tab (no round trip:
// the latency-bound small-batch GEMVs). Both give sigmoid_bf16's bits.
template <class C, int MODE, bool RESIDUAL, bool TABLE = false>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& a, const Acc<C>& tot, const int n_tg, const int count,
                                              const int start, const int tile0, float* s_act,
                                              const int* s_slot = nullptr, int wg_x = -1) {
  if (wg_x < 0) wg_x = (int)blockIdx.x;  // the work-group's tile column
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int nl = lane & 15, G = lane >> 4;
  const int rows = (int)a.w.rows;

  if (MODE == kPlain || MODE == kDown) {
#pragma unroll
    for (int t = 0; t < C::kWaveTiles; ++t) {
      const int row = (tile0 + t) * kTileRows + nl;
      if (row < rows) {
#pragma unroll
        for (int tg = 0; tg < C::kNtg; ++tg)
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int c = tg * 8 + 2 * G + u;
            if (c < count) {
              if (MODE == kPlain) {
                a.out[(size_t)(start + c) * a.out_stride + row] = tot[t][tg][u];
              } else {
                const int slot = s_slot != nullptr ? s_slot[c] : a.route_slot[start + c];
                a.y[(size_t)slot * rows + row] = bf16_bits(tot[t][tg][u]);  // bf16 (cpu_runner.rs:2945-2947)
              }
            }
          }
      }
    }
  } else {
    // gate_up epilogue: bf16 (cpu_runner.rs:2905), SwiGLU over (even, odd)
    // rows (:2907-2919), then the down input's residual-Q8 blocks: the
    // kGemmRows rows of this work-group make kGemmRows / 64 blocks of 32
    // values (cpu_runner.rs:3224-3231). The SwiGLU values reuse an LDS slot
    // as [kChunk rows][kGemmRows / 2 values]; tile t of wave w holds values
    // (w * kWaveTiles + t) * 8 .. + 7.
    // (A padding float per row where it fits, against LDS bank conflicts.)
    constexpr int kActStride =
        C::kGemmRows / 2 + (C::kChunk * (C::kGemmRows / 2 + 1) * 4 <= C::kSlotBytes ? 1 : 0);
    static_assert(C::kChunk * kActStride * 4 <= C::kSlotBytes, "SwiGLU values fit one code slot");
    // Lane pairs (even = gate row, odd = up row) hold both values for tokens
    // t0 = 2G and t1 = 2G + 1; the even lane finishes t0 and the odd lane t1.
    // Two passes: every pair's sigmoid is gathered from the table first (one
    // round trip for all of them), then the pairs are finished.
    const bool odd = (nl & 1) != 0;
    float gate_v[C::kWaveTiles][C::kNtg], up_v[C::kWaveTiles][C::kNtg];
    uint16_t sig_v[C::kWaveTiles][C::kNtg];
#pragma unroll
    for (int t = 0; t < C::kWaveTiles; ++t)
#pragma unroll
      for (int tg = 0; tg < C::kNtg; ++tg) {
        if (tg < n_tg) {
          const float own0 = bf16r(tot[t][tg][0]), own1 = bf16r(tot[t][tg][1]);
          const float recv = __uint_as_float(lane_partner<1>(__float_as_uint(odd ? own0 : own1)));
          gate_v[t][tg] = odd ? recv : own0;
          up_v[t][tg] = odd ? own1 : recv;
          sig_v[t][tg] = TABLE ? a.sig_tab[swiglu_sigmoid_index(gate_v[t][tg], a.alpha, a.limit)]
                               : sigmoid_bf16(swiglu_sigmoid_index(gate_v[t][tg], a.alpha, a.limit), s_exp2_tab);
          const int row = (tile0 + t) * kTileRows + nl;
          if (a.trace_gu != nullptr && row < rows) {  // CpuExpertTrace::gate_up_projection (bf16 values)
            for (int u = 0; u < 2; ++u) {
              const int cu = tg * 8 + 2 * G + u;
              if (cu < count) a.trace_gu[(size_t)a.route_slot[start + cu] * rows + row] = u ? own1 : own0;
            }
          }
        }
      }
#pragma unroll
    for (int t = 0; t < C::kWaveTiles; ++t)
#pragma unroll
      for (int tg = 0; tg < C::kNtg; ++tg) {
        const int c = tg * 8 + 2 * G + (odd ? 1 : 0);
        if (tg < n_tg && c < count) {
          const float act = swiglu_finish(gate_v[t][tg], up_v[t][tg], a.limit, bf16_to_f32(sig_v[t][tg]));
          s_act[c * kActStride + (wave * C::kWaveTiles + t) * 8 + (nl >> 1)] = act;
          const int row = (tile0 + t) * kTileRows + nl;
          if (a.trace_sw != nullptr && row < rows)  // CpuExpertTrace::swiglu
            a.trace_sw[(size_t)a.route_slot[start + c] * (rows / 2) + (row >> 1)] = act;
        }
      }
    __syncthreads();
    const int hw = tid >> 5, l32 = tid & 31;
    const int blocks_next = rows / kWgRows;
    constexpr int kBlocksPerWg = C::kGemmRows / 64;
    // Half wave hw quantizes blocks hw, hw + kHalfWaves, ... of the
    // count x kBlocksPerWg; all of them at once, so that their shuffle and
    // division chains overlap instead of running one block after another.
    constexpr int kHalfWaves = C::kThreads / 32;
    constexpr int kPer = (C::kChunk * kBlocksPerWg + kHalfWaves - 1) / kHalfWaves;
    ActBuffers nx;
    nx.v = a.actv_next;
    nx.s = a.acts_next;
    float v[kPer];
    bool live[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int item = hw + i * kHalfWaves;
      const int c = item / kBlocksPerWg, h = item % kBlocksPerWg;
      live[i] = item < count * kBlocksPerWg && wg_x * kBlocksPerWg + h < blocks_next;  // uniform per half wave
      v[i] = live[i] ? s_act[c * kActStride + h * kBlock + l32] : 0.0f;
      if (live[i] && !isfinite(v[i])) atomicOr(a.err, kErrNonFiniteInput);
    }
    residual_q8_store_n<kPer, RESIDUAL>(v, live, l32, hw, kHalfWaves, kBlocksPerWg, (size_t)start, blocks_next,
                                        wg_x * kBlocksPerWg, nx);
  }
}

// Loop-invariant state of the K loop. All members but the DMA and weight
// lane offsets are wave-uniform (scalar registers).
template <class C>
struct KLoop {
  __amdgpu_buffer_rsrc_t nib[C::kWaveTiles], scl[C::kWaveTiles];  // this wave's tiles of the nibble and scale planes
  __amdgpu_buffer_rsrc_t codes, scales;  // the activation operand buffers
  int B, nsteps, nfull4, last_group, wave, lane, G;
  bool wave_ok;                      // the wave's first tile exists
  int vl, vl_tail, vs;               // weight lane offsets: nibbles lane * 16 (full group) or lane * (B % 4) * 4
                                     // (the compact last group), scales (lane % 16) * 4
  int voff[C::kCodeDma];             // DMA source of this lane's code pieces in step 0
  int soff;                          // DMA source of this lane's scale dword in step 0
};

// Weights of step q (4-block groups kGroups q .. kGroups q + kGroups - 1,
// clamped to the last group: loads past the end are issued anyway so that
// every step has the same instruction count, and their data is never used).
// The compact last group (B % 4 blocks) is read with its own lane offset; the
// 16 bytes a lane loads there end at most 772 bytes into the group, inside
// the tile or the plane slack, and the dwords past the group's blocks are
// never used.
template <class C>
__device__ __forceinline__ WStep<C> load_wstep(const KLoop<C>& k, int q) {
  WStep<C> w;
#pragma unroll
  for (int g = 0; g < C::kGroups; ++g) {
    const int gi = min(C::kGroups * q + g, k.last_group);
    const int o = gi < k.nfull4 ? k.vl : k.vl_tail;
#pragma unroll
    for (int t = 0; t < C::kWaveTiles; ++t) {
      w.v[g][t] = __builtin_amdgcn_raw_buffer_load_b128(k.nib[t], o, gi * 1024, 0);
      w.s[g][t] = __builtin_amdgcn_raw_buffer_load_b32(k.scl[t], k.vs, gi * 64, 0);
    }
  }
  return w;
}

// Buffer loads straight into LDS (16 bytes or one dword per lane; the LDS
// address is wave-uniform, lane L lands at dst + L * size).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t src, char* dst, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(src, (lds_ptr)dst, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t src, char* dst, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(src, (lds_ptr)dst, 4, voff, soff, 0, 0);
}

// The DMA of step q (clamped to the last step) into one ring slot.
template <class C>
__device__ __forceinline__ void issue_dma(const KLoop<C>& k, int q_raw, char* codes, float* scl) {
  const int q = min(q_raw, k.nsteps - 1);
#pragma unroll
  for (int i = 0; i < C::kCodeDma; ++i)
    dma16(k.codes, codes + (i * C::kWaves + k.wave) * 1024, k.voff[i], q * (C::kStep * 2 * kBlock * 2));
  dma4(k.scales, reinterpret_cast<char*>(scl) + k.wave * 256, k.soff, q * (C::kStep * 8));
}

// Compute of step q (q < nsteps): its groups, each full, partial or absent.
template <class C, bool RESIDUAL, int NTG, bool FAST>
__device__ __forceinline__ void step_update(const KLoop<C>& k, Acc<C>& tot, const char* codes, const float* scl,
                                            const WStep<C>& w, const int q) {
  const float2* s2 = reinterpret_cast<const float2*>(scl);
  if constexpr (NTG >= 2 && FAST) {
    if (C::kStep * q + C::kStep <= k.B) {
      step_pipelined<C, RESIDUAL, NTG>(tot, codes, s2, w, k.lane, k.G);
      return;
    }
  }
  if (C::kStep * q + C::kStep <= k.B) {
#pragma unroll
    for (int g = 0; g < C::kGroups; ++g) {
      if (NTG == 1 && FAST)
        group_update_pipelined<C, RESIDUAL>(tot, codes, s2, w.v[g], w.s[g], 4 * g, k.lane, k.G);
      else
        group_update<C, RESIDUAL, NTG, FAST>(tot, codes, s2, w.v[g], w.s[g], 4 * g, 4, k.lane, k.G);
    }
  } else {
#pragma unroll
    for (int g = 0; g < C::kGroups; ++g) {
      const int nb = min(4, k.B - C::kStep * q - 4 * g);
      if (nb > 0) group_update<C, RESIDUAL, NTG, FAST>(tot, codes, s2, w.v[g], w.s[g], 4 * g, nb, k.lane, k.G);
    }
  }
}

// The K loop. Vector-memory issue order per wave, fixed so that one
// immediate wait covers every step. With a two-step weight lead:
//   prologue W(0) D(0) W(1) D(1); step q: wait(D(q), W(q)) barrier
//   D(q+2) compute(q) W(q+2);
// at step q's wait the requests after D(q) and W(q) are D(q+1) and W(q+1)
// = kWaitVm instructions. With a one-step lead:
//   prologue W(0) D(0) D(1); step q: wait(D(q), W(q)) barrier
//   W(q+1) D(q+2) compute(q);
// at step q's wait only D(q+1) follows W(q). A three-step weight lead queued
// more requests ahead of each step's own and ran 1% slower on decode batches;
// prefill, with four token groups of compute per step, runs 1-2% faster with
// a one-step lead, decode 0.5% slower.
template <class C, bool RESIDUAL, int NTG, bool FAST>
__device__ __forceinline__ void k_loop(const KLoop<C>& k, Acc<C>& tot, char* c0, char* c1, char* c2, float* s0,
                                       float* s1, float* s2) {
  WStep<C> w0, w1, w2;
  __builtin_amdgcn_sched_barrier(0);
  w0 = load_wstep(k, 0);
  __builtin_amdgcn_sched_barrier(0);
  issue_dma<C>(k, 0, c0, s0);
  __builtin_amdgcn_sched_barrier(0);
  if (C::kWLead == 2) w1 = load_wstep(k, 1);
  __builtin_amdgcn_sched_barrier(0);
  issue_dma<C>(k, 1, c1, s1);
  __builtin_amdgcn_sched_barrier(0);
#define GOSSMX_STEP(QV, SLOT, CODES, SCL, NCODES, NSCL, NEXT1, NEXT2)                               \
  {                                                                                                  \
    const int q = (QV);                                                                              \
    __builtin_amdgcn_sched_barrier(0);                                                               \
    __builtin_amdgcn_s_waitcnt(C::kWaitDma); /* this wave's DMA and weights for step q have landed */\
    __builtin_amdgcn_s_barrier();         /* ... and every other wave's; the slot of q-1 is free */  \
    __builtin_amdgcn_sched_barrier(0);                                                               \
    if (C::kWLead == 1) NEXT1 = load_wstep(k, q + 1);                                                \
    __builtin_amdgcn_sched_barrier(0);                                                               \
    issue_dma<C>(k, q + 2, NCODES, NSCL);                                                            \
    __builtin_amdgcn_sched_barrier(0);                                                               \
    if (k.wave_ok && q < k.nsteps) step_update<C, RESIDUAL, NTG, FAST>(k, tot, CODES, SCL, SLOT, q); \
    __builtin_amdgcn_sched_barrier(0);                                                               \
    if (C::kWLead == 2) NEXT2 = load_wstep(k, q + 2);                                                \
    __builtin_amdgcn_sched_barrier(0);                                                               \
  }
  const int n_pad = (k.nsteps + 2) / 3 * 3;
  for (int q0 = 0; q0 < n_pad; q0 += 3) {
    GOSSMX_STEP(q0, w0, c0, s0, c2, s2, w1, w2)
    GOSSMX_STEP(q0 + 1, w1, c1, s1, c0, s0, w2, w0)
    GOSSMX_STEP(q0 + 2, w2, c2, s2, c1, s1, w0, w1)
  }
#undef GOSSMX_STEP
}

template <class C, int MODE, bool RESIDUAL>
__global__ __launch_bounds__(C::kThreads, C::kMinWaves) void gemm_kernel(GemmArgs a) {
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int nl = lane & 15, G = lane >> 4;
  int expert, start, count;
  if (MODE == kPlain) {
    expert = a.plain_expert;
    start = blockIdx.y * C::kChunk;
    count = min(C::kChunk, a.plain_m - start);
  } else {
    const int wi = blockIdx.y;
    // The item count and the item's record in one round trip (records past
    // the count are in bounds and ignored). A real item has an expert and a
    // start >= 0 and at least one row; testing all three keeps the whole
    // record's load ahead of the branch.
    const int nw = *a.n_work;
    const int4 rec = reinterpret_cast<const int4*>(a.work)[wi];
    if ((wi >= nw) | (min(min(rec.x, rec.y), rec.z - 1) < 0)) return;  // uniform over the work-group
    expert = rec.x;
    start = rec.y;  // grouped index of the item's first route
    count = rec.z;
  }
  const int rows = (int)a.w.rows, B = (int)a.w.blocks;
  int wg_x = (int)blockIdx.x;  // tile column
  if (C::kPinXcd && MODE == kGateUp) {
    const int n_x = ((int)a.w.tiles + C::kWgTiles - 1) / C::kWgTiles;
    const int p_x = (int)gridDim.x;  // n_x padded to a multiple of 8
    wg_x = ((int)blockIdx.x + p_x - (expert & 7)) % p_x;
    if (wg_x >= n_x) return;  // padding; uniform over the work-group
  }
  const int tile0 = (wg_x * C::kWaves + wave) * C::kWaveTiles;
  const int n_tg = (count + 7) >> 3;
  const int nq4 = (B + 3) >> 2;

  // Everything that needs only the item goes out in one round trip: the
  // activation row indices, the tiles' fast-path flags and biases
  // (branch-free, from valid addresses; read after the barrier).
  __shared__ int s_row[C::kChunk];
  __shared__ int s_slot[C::kChunk];  // kDown: the item's route slots, for the epilogue's stores
  int row_idx = -1, slot_idx = -1;
  if (tid < C::kChunk && tid < count) {
    if (MODE == kPlain) row_idx = start + tid;
    else if (MODE == kGateUp) row_idx = a.route_tok[start + tid];
    else row_idx = start + tid;
    if (MODE == kDown) slot_idx = a.route_slot[start + tid];
  }
  KLoop<C> k;
  k.B = B;
  k.nsteps = (B + C::kStep - 1) / C::kStep;
  k.nfull4 = B >> 2;
  k.last_group = nq4 - 1;
  k.wave = wave;
  k.lane = lane;
  k.G = G;
  k.wave_ok = tile0 < (int)a.w.tiles;
  k.vl = lane * 16;
  k.vl_tail = lane * (B & 3) * 4;
  k.vs = nl * 4;
  uint8_t fast_raw[C::kWaveTiles];
  float bias_raw[C::kWaveTiles];
#pragma unroll
  for (int t = 0; t < C::kWaveTiles; ++t) {
    const int tile = tile0 + t;
    const bool ok = tile < (int)a.w.tiles;
    // Tiles past the end stream tile 0 and discard it.
    const int safe_tile = ok ? tile : 0;
    const uint8_t* nib = a.w.nib + (size_t)expert * a.w.nib_stride + (size_t)safe_tile * 256 * B;
    const uint8_t* scl = a.w.scl + (size_t)expert * a.w.scl_stride + (size_t)safe_tile * 64 * nq4;
    k.nib[t] = buffer_rsrc(nib);
    k.scl[t] = buffer_rsrc(scl);
  }
#pragma unroll
  for (int t = 0; t < C::kWaveTiles; ++t) {
    const int tile = tile0 + t;
    const int safe_tile = tile < (int)a.w.tiles ? tile : 0;
    fast_raw[t] = a.w.fast[(size_t)expert * a.w.tiles + safe_tile];
    // Without a bias the load reads the first word of the scales instead
    // (discarded).
    const int row = min(tile * kTileRows + nl, rows - 1);
    const float* bp = a.bias != nullptr ? a.bias + (size_t)expert * a.bias_expert_stride + row
                                        : reinterpret_cast<const float*>(a.w.scl);
    bias_raw[t] = *bp;
  }

  // LDS ring of three steps, filled by DMA two steps ahead.
  __shared__ __align__(16) char s_codes0[C::kSlotBytes], s_codes1[C::kSlotBytes], s_codes2[C::kSlotBytes];
  __shared__ __align__(16) float s_scl0[C::kSclSlot], s_scl1[C::kSclSlot], s_scl2[C::kSclSlot];
  if (tid < C::kChunk) s_row[tid] = row_idx;
  if (MODE == kDown && tid < C::kChunk) s_slot[tid] = slot_idx;
  __syncthreads();

  bool fast = a.fast_ok != 0;
  Acc<C> tot;
#pragma unroll
  for (int t = 0; t < C::kWaveTiles; ++t) {
    const int tile = tile0 + t;
    const bool ok = tile < (int)a.w.tiles;
    fast = fast && (!ok || fast_raw[t] != 0);
    const int row = tile * kTileRows + nl;
    // A -0.0 bias becomes +0.0, as the reference's first add does.
    const float b0 = (a.bias != nullptr && ok && row < rows ? bias_raw[t] : 0.0f) + 0.0f;
#pragma unroll
    for (int tg = 0; tg < C::kNtg; ++tg) { tot[t][tg][0] = b0; tot[t][tg][1] = b0; }
  }

  // DMA lane map, the same for every step. Code piece i of this wave fills
  // slot bytes c * 16 with c = (i * C::kWaves + wave) * 64 + lane, i.e. block j,
  // token group tg, k-slice g, vector v (row tg*8 + v/2, part v%2) in the
  // slot layout above; its source is piece (part, g) of the row's 128-byte
  // block record. Scale dword d = wave * 64 + lane holds half d % 2 of
  // (block d / (2 kChunk), row (d / 2) % kChunk). Lanes with nothing to move
  // read the start of the buffer (valid memory) into slot bytes no row uses.
  // A last partial step reads up to kStep - 1 blocks past a row, inside the
  // buffers' slack.
  k.codes = buffer_rsrc(a.actv);
  k.scales = buffer_rsrc(a.acts);
#pragma unroll
  for (int i = 0; i < C::kCodeDma; ++i) {
    const int c = (i * C::kWaves + wave) * 64 + lane;
    const int ch = c >> 6, p = c & 63;
    const int j = ch / C::kNtg, tg = ch % C::kNtg, g = p >> 4, v = p & 15;
    const int t = tg * 8 + (v >> 1), part = v & 1;
    k.voff[i] = t < count ? ((s_row[t] * B + j) * 8 + part * 4 + g) * 16 : 0;
  }
  {
    const int d = wave * 64 + lane;
    const int j = d / (C::kChunk * 2), t = (d >> 1) % C::kChunk;
    k.soff = (d < C::kStep * C::kChunk * 2 && t < count) ? ((s_row[t] * B + j) * 2 + (d & 1)) * 4 : 0;
  }

  if (n_tg == 1) {
    if (fast) k_loop<C, RESIDUAL, 1, true>(k, tot, s_codes0, s_codes1, s_codes2, s_scl0, s_scl1, s_scl2);
    else k_loop<C, RESIDUAL, 1, false>(k, tot, s_codes0, s_codes1, s_codes2, s_scl0, s_scl1, s_scl2);
  } else {
    if (fast) k_loop<C, RESIDUAL, C::kNtg, true>(k, tot, s_codes0, s_codes1, s_codes2, s_scl0, s_scl1, s_scl2);
    else k_loop<C, RESIDUAL, C::kNtg, false>(k, tot, s_codes0, s_codes1, s_codes2, s_scl0, s_scl1, s_scl2);
  }
  // Drain the trailing DMA into the ring before the LDS is reused or the
  // work-group ends.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  gemm_epilogue<C, MODE, RESIDUAL, true>(a, tot, n_tg, count, start, tile0, reinterpret_cast<float*>(s_codes0),
                                   MODE == kDown ? s_slot : nullptr, wg_x);
}

// ---------------------------------------------------------------------------
// Small-batch GEMV: batches of at most kTinyMaxRows rows (every work item is
// at most kTinyMaxRows tokens of one expert) with at most kTinyMaxBlocks
// blocks per row. A work-group is 4 waves, one 16-row weight tile each (64
// rows: whole 32-value blocks of the down input for the gate_up epilogue),
// each over the whole K range.
//
// Block packing. With the launch's tokens per item padded to mp in {1, 2, 4},
// a block has V = 2 mp activation vectors (token, part), so the 16 rows of an MFMA A
// operand hold P = 16 / V consecutive blocks of one "set": row i = p V + v is
// vector v (token v / 2, part v % 2) of block s P + p. MFMA p of set s takes
// the weights of block s P + p and an A operand whose rows of the other
// positions are zero (those lanes read a zero piece of LDS), and the P MFMAs
// of a set accumulate into one result, so each row of the result holds
// exactly one block's integer dot (the other MFMAs add +0 to it; the sign of
// a zero term never changes the chain, whose running total is never -0.0).
// Every lane of the wave then holds useful dots, where one block per MFMA
// leaves 7 of every 8 vectors empty at one token.
// Lane (G, n) holds result rows 4G..4G+3 of weight row n; its term for row i
// is (D_i * e8) * act_scale(block, token, part): the reference's
// (p * ws) * ps rounded once (on the fast path the conversion applied the
// E8M0 scale exactly and e8 is 1.0; otherwise e8 is e8m0_scale of the
// block). The terms go through per-wave LDS buffers laid out
// [p][token][row][part], from which lane 16 t + n runs the ordered chain of
// (row n, token t): total += term_p; total += term_r, block after block,
// the same sequence of operations per output as gemm_kernel's.
//
// LDS (dynamic, sized for mp): the activation image, set s at
// s * kTinySetBytes as 64 pieces of 16 bytes [position][vector][k-slice]
// (piece 4 i + g: k-slice g of row i) followed by a zero piece; the
// activation scales [block][token][part] f32 (the 16 scales of set s at
// 16 s); kTinyTermBufs term buffers of 1 KiB per wave.

// Weight groups in flight per wave (measured at one token: 8 and 16 groups
// run alike, the whole K range at once is slower); fewer at four tokens,
// whose sets hold more operands in registers.
__host__ __device__ constexpr int tiny_ring(int P) { return P == 2 ? 12 : 16; }
constexpr int kTinySetBytes = 1024 + 16;                        // a set's 64 pieces and its zero piece
constexpr int kTinyTermBytes = 1024;                            // [8 (position, token)][16 rows][2] f32
constexpr int kTinyTermBufs = 4;                                // term buffers per wave (the chain lags 2 sets)
static_assert(kTinyMaxBlocks % 8 == 0, "whole sets at one token (8 blocks per set)");

__host__ __device__ constexpr int tiny_sets(int mp) { return kTinyMaxBlocks * mp / 8; }
__host__ __device__ constexpr int tiny_image_bytes(int mp) { return tiny_sets(mp) * kTinySetBytes; }

// The geometry fields gemm_epilogue reads.
struct GemmTinyCfg {
  static constexpr int kWaves = 4;
  static constexpr int kThreads = 256;
  static constexpr int kWaveTiles = 1;
  static constexpr int kWgTiles = 4;
  static constexpr int kGemmRows = kTileRows * kWgTiles;
  static constexpr int kChunk = kSmallChunk;                   // token slots of a work item
  static constexpr int kNtg = 1;
  static constexpr int kSlotBytes = tiny_image_bytes(1);     // LDS the epilogue may reuse
};

struct GemvLoads {
  __amdgpu_buffer_rsrc_t nib, scl;
  int vl, vl_tail, vs, nq4, nfull4;
};

__device__ __forceinline__ void gemv_load(const GemvLoads& L, int q, u32x4& wn, uint32_t& ws) {
  const int gi = min(q, L.nq4 - 1);  // groups past the end re-load the last one (unused)
  wn = __builtin_amdgcn_raw_buffer_load_b128(L.nib, gi < L.nfull4 ? L.vl : L.vl_tail, gi * 1024, 0);
  ws = __builtin_amdgcn_raw_buffer_load_b32(L.scl, L.vs, gi * 64, 0);
}

// The K loop of one wave over sets [S0, S1) of P blocks (mp = 8 / P tokens),
// straight line, with a ring of R weight groups. Blocks past B contribute
// +0.0 terms, which leave the running total unchanged (it is never -0.0).
// Their weights are the last group's bytes (loads past the end are clamped
// to it) or the plane slack: E2M1 codes and zeroed or stored scale bytes, all
// of which convert to finite values, so the zero rows of the A operand keep
// every real row exact (0 x finite = 0). With `fast` the conversion applies
// the tile's scales (all in the exact range) and e8 is 1.0 (d * 1.0 is d);
// otherwise the conversion is unscaled and e8 is e8m0_scale of the block.
// STORE = false: set s's terms go to buffer s % kTinyTermBufs and the chain
// of set s - 2 runs after set s is produced (its LDS round trip and adds
// overlap the MFMAs of the sets in between). STORE = true: set s's terms go
// to buffer s - S0 and no chain runs (another wave continues the chain).
template <int P>
__device__ __forceinline__ void gemv_chain_set(float& tot, const float* tb, const int n, const int t_read) {
  constexpr int mp = 8 / P;
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const float2 v = reinterpret_cast<const float2*>(tb)[(p * mp + t_read) * 16 + n];
    tot = tot + v.x;
    tot = tot + v.y;
  }
}

template <int P, int R, int S0, int S1, bool STORE>
__device__ __forceinline__ float gemv_sets(float tot, const GemvLoads& L, u32x4 (&wn)[R], uint32_t (&ws)[R],
                                           const char* img, const float* scl, float* terms, const int B,
                                           const int lane, const bool fast) {
  constexpr int V = 16 / P, mp = 8 / P;
  constexpr int G1 = S1 * P / 4;  // groups of this range end here
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  const int G = lane >> 4, n = lane & 15;
  // A operand of MFMA p: lane (g = lane / 16, i = lane % 16) reads piece
  // 4 i + g of the set when row i belongs to position p, else the zero piece.
  int off[P];
#pragma unroll
  for (int p = 0; p < P; ++p) off[p] = (n / V == p) ? (4 * n + G) * 16 : 1024;
  // Positions of this lane's result rows 4G, 4G+1 and 4G+2, 4G+3.
  const int pos_a = (4 * G) / V, pos_b = (4 * G + 2) / V;
  // Chain lane 16 t + n reads entry p * mp + t of a term buffer (t past mp
  // folds onto a real token; its total is never stored).
  const int t_read = G & (mp - 1);
#pragma unroll
  for (int s = S0; s < S1; ++s) {
    f32x4 d = zero;
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int b = s * P + p, q = b >> 2, j = b & 3;
      const uint32_t sw = ws[q % R];
      const half8 bop = fp4x8_to_half8_scaled(wn[q % R][j], fast ? e8m0_scale_operand(sw, j) : 1.0f);
      const half8 aop = *reinterpret_cast<const half8*>(img + s * kTinySetBytes + off[p]);
      d = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, d, 0, 0, 0);
    }
    // e8 of the blocks of this lane's rows (branch-free, then 1.0 on the
    // fast path).
    float e8a, e8b;
    if (P == 8) {  // rows 4G, 4G+1: block 8 s + 2G; rows 4G+2, 4G+3: block 8 s + 2G + 1 (group 2 s + G / 2)
      const uint32_t sw = G < 2 ? ws[(2 * s) % R] : ws[(2 * s + 1) % R];
      const int sh = 16 * (G & 1);
      e8a = e8m0_select((sw >> sh) & 0xffu);
      e8b = e8m0_select((sw >> (sh + 8)) & 0xffu);
    } else if (P == 4) {  // block 4 s + G (group s)
      e8a = e8b = e8m0_select((ws[s % R] >> (8 * G)) & 0xffu);
    } else {  // block 2 s + G / 2 (group s / 2, byte 2 (s % 2) + G / 2)
      e8a = e8b = e8m0_select((ws[(s / 2) % R] >> (8 * (2 * (s & 1) + (G >> 1)))) & 0xffu);
    }
    e8a = fast ? 1.0f : e8a;
    e8b = fast ? 1.0f : e8b;
    // Groups whose blocks are all converted take the group R ahead.
#pragma unroll
    for (int q = (s * P) / 4; q < ((s + 1) * P) / 4; ++q)
      if (q + R < G1) gemv_load(L, q + R, wn[q % R], ws[q % R]);
    const float4 sc = *reinterpret_cast<const float4*>(scl + s * 16 + 4 * G);
    // Terms of blocks past B become +0.0 by a bit mask (no branch).
    const uint32_t ma = s * P + pos_a < B ? ~0u : 0u, mb = s * P + pos_b < B ? ~0u : 0u;
    float2 t01, t23;
    t01.x = __uint_as_float(__float_as_uint((d[0] * e8a) * sc.x) & ma);
    t01.y = __uint_as_float(__float_as_uint((d[1] * e8a) * sc.y) & ma);
    t23.x = __uint_as_float(__float_as_uint((d[2] * e8b) * sc.z) & mb);
    t23.y = __uint_as_float(__float_as_uint((d[3] * e8b) * sc.w) & mb);
    // Rows 4G, 4G+1 are entry 2G, rows 4G+2, 4G+3 entry 2G+1 ([p][token]).
    float* tb = terms + (STORE ? s - S0 : s % kTinyTermBufs) * (kTinyTermBytes / 4);
    reinterpret_cast<float2*>(tb)[(2 * G) * 16 + n] = t01;
    reinterpret_cast<float2*>(tb)[(2 * G + 1) * 16 + n] = t23;
    if (!STORE && s >= S0 + 2)
      gemv_chain_set<P>(tot, terms + ((s - 2) % kTinyTermBufs) * (kTinyTermBytes / 4), n, t_read);
  }
  if (!STORE) {
    gemv_chain_set<P>(tot, terms + ((S1 - 2) % kTinyTermBufs) * (kTinyTermBytes / 4), n, t_read);
    gemv_chain_set<P>(tot, terms + ((S1 - 1) % kTinyTermBufs) * (kTinyTermBytes / 4), n, t_read);
  }
  return tot;
}

// Geometry of a gemv_kernel launch: HALVES = 2 splits each tile's K range
// over two waves (one token only): wave (half 0, tile t) produces and chains
// the first half of the sets, wave (half 1, tile t) produces the second
// half's terms into an LDS buffer, and after a barrier wave (0, t) continues
// its chain through them; twice the waves keep the SIMDs busier where one
// wave per SIMD would otherwise issue alone.
template <int P, int HALVES, int RING = (HALVES == 2 ? 6 : tiny_ring(P))>
struct GemvGeom {
  static constexpr int kMp = 8 / P;
  static constexpr int kSets = kTinyMaxBlocks / P;
  static constexpr int kHalfSets = kSets / HALVES;
  static constexpr int kWaves = 4 * HALVES;
  static constexpr int kThreads = 64 * kWaves;
  // Weight groups in flight per wave. A half's first group is a multiple of
  // the ring, so ring slots are compile-time in both halves.
  static constexpr int kRing = RING;
  // Per-wave term region: the chain's ring, or half 1's buffered sets.
  static constexpr int kTermRegion = (HALVES == 2 ? (kHalfSets > kTinyTermBufs ? kHalfSets : kTinyTermBufs)
                                                  : kTinyTermBufs) * kTinyTermBytes;
  static constexpr int kLds = tiny_image_bytes(kMp) + tiny_sets(kMp) * 64 + kWaves * kTermRegion;
  static_assert(kSets % HALVES == 0 && (kHalfSets * P) % 4 == 0, "halves end on whole groups");
  static_assert(HALVES == 1 || ((kHalfSets * P) / 4) % kRing == 0, "a half starts on ring slot 0");
};

template <int MODE, int P, int HALVES>
__global__ __launch_bounds__(64 * 4 * HALVES, HALVES == 2 ? 4 : 2) void gemv_kernel(GemmArgs a) {
  using C = GemmTinyCfg;
  using Geo = GemvGeom<P, HALVES>;
  extern __shared__ __align__(16) char s_dyn[];
  const int tid = threadIdx.x;
  const uint64_t exp2_entry = MODE == kGateUp ? load_exp2_entry() : 0ull;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int half = wave >> 2, wt = wave & 3;  // K half, and the wave's tile within the work-group
  const int nl = lane & 15;
  int expert, start, count;
  if (MODE == kPlain) {
    expert = a.plain_expert;
    start = blockIdx.y * kTinyMaxRows;
    count = min(kTinyMaxRows, a.plain_m - start);
  } else {
    const int wi = blockIdx.y;
    // The item count and the item's record in one round trip (records past
    // the count are in bounds and ignored). A real item has an expert and a
    // start >= 0 and at least one row; testing all three keeps the whole
    // record's load ahead of the branch.
    const int nw = *a.n_work;
    const int4 rec = reinterpret_cast<const int4*>(a.work)[wi];
    if ((wi >= nw) | (min(min(rec.x, rec.y), rec.z - 1) < 0)) return;  // uniform over the work-group
    expert = rec.x;
    start = rec.y;
    count = rec.z;
  }
  constexpr int mp = Geo::kMp, V = 2 * mp;  // every item of the launch holds at most mp tokens
  const int rows = (int)a.w.rows, B = (int)a.w.blocks;
  const int tile0 = blockIdx.x * C::kWaves + wt;
  const bool ok = tile0 < (int)a.w.tiles;
  const int safe_tile = ok ? tile0 : 0;  // tiles past the end stream tile 0 and discard it
  const int nq4 = (B + 3) >> 2;

  // Per-tile state first (fast-path flag, bias), branch-free and read after
  // the barrier (without a bias, the first word of the scales, discarded).
  const uint8_t fast_raw = a.w.fast[(size_t)expert * a.w.tiles + safe_tile];
  const int row = tile0 * kTileRows + nl;
  const float bias_raw = *(a.bias != nullptr ? a.bias + (size_t)expert * a.bias_expert_stride + min(row, rows - 1)
                                             : reinterpret_cast<const float*>(a.w.scl));

  // The first four weight groups of the wave's range, then the activation
  // rows, then the rest of the ring: the weights need only the expert.
  GemvLoads L;
  L.nib = buffer_rsrc(a.w.nib + (size_t)expert * a.w.nib_stride + (size_t)safe_tile * 256 * B);
  L.scl = buffer_rsrc(a.w.scl + (size_t)expert * a.w.scl_stride + (size_t)safe_tile * 64 * nq4);
  L.vl = lane * 16;
  L.vl_tail = lane * (B & 3) * 4;
  L.vs = nl * 4;
  L.nq4 = nq4;
  L.nfull4 = B >> 2;
  constexpr int R = Geo::kRing;
  const int g0 = HALVES == 2 ? half * (Geo::kHalfSets * P / 4) : 0;  // first group of the wave's range (slot 0)
  u32x4 wn[R];
  uint32_t ws[R];
  constexpr int kFirst = R < 4 ? R : 4;
#pragma unroll
  for (int q = 0; q < kFirst; ++q) gemv_load(L, g0 + q, wn[q], ws[q]);

  // Activation rows of the item's tokens (absent tokens read row 0: valid
  // memory whose products are never stored).
  int r[kTinyMaxRows];
#pragma unroll
  for (int t = 0; t < kTinyMaxRows; ++t)
    r[t] = t < count ? (MODE == kGateUp ? a.route_tok[start + t] : start + t) : 0;

  char* img = s_dyn;
  float* s_scl = reinterpret_cast<float*>(s_dyn + tiny_image_bytes(mp));
  float* term_base = reinterpret_cast<float*>(s_dyn + tiny_image_bytes(mp) + tiny_sets(mp) * 64);
  float* terms = term_base + wave * (Geo::kTermRegion / 4);
  const int nsets = (B + P - 1) / P;
  const __amdgpu_buffer_rsrc_t act_codes = buffer_rsrc(a.actv), act_scl = buffer_rsrc(a.acts);
  {
    // Image piece `lane` of set k: row i = lane / 4 (position i / V, vector
    // i % V), k-slice lane % 4.
    const int i = lane >> 2, g = lane & 3, v = i % V, t = v >> 1, part = v & 1;
    const int rt = t == 0 ? r[0] : (t == 1 ? r[1] : (t == 2 ? r[2] : r[3]));
    for (int k = wave; k < nsets; k += Geo::kWaves) {  // uniform per wave
      const int b = k * P + i / V;
      const int voff = (b < B && t < count) ? ((rt * B + b) * 2 + part) * 64 + g * 16 : 0;
      dma16(act_codes, img + k * kTinySetBytes, voff, 0);
    }
    // Scale f of the image: block f / (2 mp), token (f / 2) % mp, part f % 2.
    for (int k = wave; k * 64 < nsets * 16; k += Geo::kWaves) {  // uniform per wave
      const int f = k * 64 + lane;
      const int b = f / (2 * mp), ts = (f >> 1) % mp, ps = f & 1;
      const int rs = ts == 0 ? r[0] : (ts == 1 ? r[1] : (ts == 2 ? r[2] : r[3]));
      const int voff = (b < B && ts < count) ? ((rs * B + b) * 2 + ps) * 4 : 0;
      dma4(act_scl, reinterpret_cast<char*>(s_scl) + k * 256, voff, 0);
    }
  }
  for (int k = tid; k < nsets; k += Geo::kThreads)
    *reinterpret_cast<u32x4*>(img + k * kTinySetBytes + 1024) = u32x4{};
  if (MODE == kGateUp) store_exp2_entry(exp2_entry);
#pragma unroll
  for (int q = kFirst; q < R; ++q) gemv_load(L, g0 + q, wn[q], ws[q]);
  // The DMA and the first groups have landed once at most the later groups'
  // loads are outstanding; then every wave's part is in.
  constexpr int kWait = 2 * (R - kFirst);
  static_assert(kWait < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((kWait & 15) | ((kWait >> 4) << 14) | (7 << 4) | (15 << 8));
  __syncthreads();

  const bool fast = a.fast_ok && fast_raw != 0;
  // A -0.0 bias becomes +0.0, as the reference's first add does.
  float tot = (a.bias != nullptr && ok && row < rows ? bias_raw : 0.0f) + 0.0f;
  if (HALVES == 1) {
    tot = gemv_sets<P, R, 0, Geo::kSets, false>(tot, L, wn, ws, img, s_scl, terms, B, lane, fast);
  } else if (half == 0) {
    tot = gemv_sets<P, R, 0, Geo::kHalfSets, false>(tot, L, wn, ws, img, s_scl, terms, B, lane, fast);
  } else {
    gemv_sets<P, R, Geo::kHalfSets, Geo::kSets, true>(tot, L, wn, ws, img, s_scl, terms, B, lane, fast);
  }
  if (HALVES == 2) {
    __syncthreads();  // the second half's terms are in LDS
    if (half == 0) {
      const float* tb2 = term_base + (wave + 4) * (Geo::kTermRegion / 4);
      const int n = lane & 15, t_read = (lane >> 4) & (mp - 1);
#pragma unroll
      for (int s = 0; s < Geo::kHalfSets; ++s) gemv_chain_set<P>(tot, tb2 + s * (kTinyTermBytes / 4), n, t_read);
    }
  }

  // Lane 16 t + n holds (row n, token t); the epilogue's lane (G, n) holds
  // tokens 2G and 2G + 1.
  const int G = lane >> 4;
  Acc<C> acc;
  acc[0][0][0] = __shfl(tot, ((2 * G) * 16 + nl) & 63);
  acc[0][0][1] = __shfl(tot, ((2 * G + 1) * 16 + nl) & 63);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // every wave is done with the LDS image before the epilogue reuses it
  if (half == 0) {
    gemm_epilogue<C, MODE, true>(a, acc, 1, count, start, tile0, reinterpret_cast<float*>(s_dyn));
  } else if (MODE == kGateUp) {
    __syncthreads();  // gemm_epilogue's one barrier (gate_up), matched by the second half's waves
  }
}

// ---------------------------------------------------------------------------
// Down projection and weighted combine of a one-row batch in one launch
// (cpu_runner.rs:2933-2947 then :2959-2999 at m = 1). The row's top_k routes
// go to top_k distinct experts, so the work list holds top_k items of one
// route each. Work-group x covers 16-row tile x of the down output for every
// item: wave (k, half) streams item k's expert over half of the K range
// exactly as gemv_kernel<kDown, 8, 2> does (sets of 8 blocks, half 1's terms
// buffered in LDS, half 0 continuing the ordered chain through them), from
// item k's own activation image. The bf16 outputs of the items then meet in
// LDS by rank, and 16 lanes run the combine of the tile's rows in rank order
// from 0.0 (and the residual add), so no other launch reads them back.
struct DownCombineGeom {
  // Four weight groups in flight per wave: deeper rings queue more requests
  // ahead of each wave's next group and ran slower (6: +2%, 12: +3%).
  using Geo = GemvGeom<8, 2, 4>;
  static constexpr int kItems = 4;                         // routes of the row (top_k <= 4)
  static constexpr int kWaves = 2 * kItems;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kImage = tiny_image_bytes(1);       // one item's activation sets
  static constexpr int kScl = tiny_sets(1) * 64;           // one item's activation scales
  static constexpr int kLds = kItems * (kImage + kScl) + kWaves * Geo::kTermRegion + kItems * kTileRows * 4;
  static_assert(kLds <= 160 * 1024, "LDS of one work-group");
};

struct CombineArgs {
  const float* weights;    // [top_k] routing weights by rank
  int top_k;
  float* out;              // [rows] f32 (bf16 values), or null
  uint16_t* out16;         // [rows] the same values as bf16 bits, or null
  float* trace;            // [top_k][rows] down outputs by rank, or null
  const uint16_t* resid;   // [rows] bf16 residual stream, or null
  uint16_t* next;          // [rows] bf16(resid + out), or null
  float* unrounded;        // [rows] the weighted sum before its bf16 round trip, or null
};

__global__ __launch_bounds__(DownCombineGeom::kThreads, 2) void gemv_down_combine_kernel(GemmArgs a, CombineArgs c) {
  using DC = DownCombineGeom;
  using Geo = DC::Geo;
  constexpr int P = 8, V = 2, R = Geo::kRing;
  __shared__ __align__(16) char s_img[DC::kItems * DC::kImage];
  __shared__ __align__(16) float s_scl[DC::kItems * DC::kScl / 4];
  __shared__ __align__(16) float s_terms[DC::kWaves * Geo::kTermRegion / 4];
  __shared__ float s_y[DC::kItems * kTileRows];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int item = wave & 3, half = wave >> 2;
  const int nl = lane & 15;
  const int rows = (int)a.w.rows, B = (int)a.w.blocks;
  const int tile = blockIdx.x;
  const int row = tile * kTileRows + nl;
  const int nsets = (B + P - 1) / P;
  char* img = s_img + item * DC::kImage;
  float* scl = s_scl + item * (DC::kScl / 4);
  // LDS stores first (none may follow the DMA into the same arrays).
  if (tid < DC::kItems * kTileRows) s_y[tid] = 0.0f;
  if (half == 0)
    for (int k = lane; k < nsets; k += 64) *reinterpret_cast<u32x4*>(img + k * kTinySetBytes + 1024) = u32x4{};
  // The item count and the wave's record in one round trip: records
  // 0 .. top_k - 1 exist (the work list holds more than top_k), so the read
  // is clamped to them and discarded for an item past the count.
  const int nw = *a.n_work;
  const int4 rec = reinterpret_cast<const int4*>(a.work)[min(item, c.top_k - 1)];
  // With one row every item is one route, and the routes are grouped in item
  // order, so item k's down input is route row k: its image moves into LDS
  // while the record is on its way (the two waves of the item take alternate
  // sets; piece `lane` of a set: row i = lane / 4 (block i / 2, part i % 2),
  // k-slice lane % 4).
  if (item < c.top_k) {
    const __amdgpu_buffer_rsrc_t act_codes = buffer_rsrc(a.actv), act_scl = buffer_rsrc(a.acts);
    const int i = lane >> 2, g = lane & 3, part = i & 1;
    for (int k = half; k < nsets; k += 2) {
      const int b = k * P + i / V;
      dma16(act_codes, img + k * kTinySetBytes, b < B ? ((item * B + b) * 2 + part) * 64 + g * 16 : 0, 0);
    }
    // Scale f of the image: block f / 2, part f % 2.
    for (int k = half; k * 64 < nsets * 16; k += 2) {
      const int f = k * 64 + lane, b = f >> 1;
      dma4(act_scl, reinterpret_cast<char*>(scl) + k * 256, b < B ? ((item * B + b) * 2 + (f & 1)) * 4 : 0, 0);
    }
  }
  const bool live = item < nw;  // uniform per wave
  const int expert = live ? rec.x : 0, start = live ? rec.y : 0;
  if (live && start != item && lane == 0) atomicOr(a.err, kErrWorkOrder);
  // What needs only the record goes out together, branch-free, and is read
  // after the barrier: the tile's fast-path flag and bias (without a bias,
  // the first word of the scales, discarded), the weight ring, and the
  // route's rank (one row: slot = rank; requested last, as its first use
  // would otherwise wait for the image DMA issued before it).
  const uint8_t fast_raw = a.w.fast[(size_t)expert * a.w.tiles + tile];
  const float bias_raw = *(a.bias != nullptr ? a.bias + (size_t)expert * a.bias_expert_stride + min(row, rows - 1)
                                             : reinterpret_cast<const float*>(a.w.scl));
  const int nq4 = (B + 3) >> 2;

  GemvLoads L;
  L.nib = buffer_rsrc(a.w.nib + (size_t)expert * a.w.nib_stride + (size_t)tile * 256 * B);
  L.scl = buffer_rsrc(a.w.scl + (size_t)expert * a.w.scl_stride + (size_t)tile * 64 * nq4);
  L.vl = lane * 16;
  L.vl_tail = lane * (B & 3) * 4;
  L.vs = nl * 4;
  L.nq4 = nq4;
  L.nfull4 = B >> 2;
  const int g0 = half * (Geo::kHalfSets * P / 4);
  u32x4 wn[R];
  uint32_t ws[R];
  float* terms = s_terms + wave * (Geo::kTermRegion / 4);
  if (live) {
#pragma unroll
    for (int q = 0; q < R; ++q) gemv_load(L, g0 + q, wn[q], ws[q]);
  }
  const int slot = a.route_slot[start];
  __builtin_amdgcn_s_waitcnt(0);  // the image and the ring are in
  __syncthreads();

  const bool fast = live && a.fast_ok && fast_raw != 0;
  // A -0.0 bias becomes +0.0, as the reference's first add does.
  float tot = (live && a.bias != nullptr && row < rows ? bias_raw : 0.0f) + 0.0f;
  if (live) {
    if (half == 0)
      tot = gemv_sets<P, R, 0, Geo::kHalfSets, false>(tot, L, wn, ws, img, scl, terms, B, lane, fast);
    else
      gemv_sets<P, R, Geo::kHalfSets, Geo::kSets, true>(tot, L, wn, ws, img, scl, terms, B, lane, fast);
  }
  __syncthreads();  // the second halves' terms are in LDS
  if (live && half == 0) {
    const float* tb2 = s_terms + (wave + 4) * (Geo::kTermRegion / 4);
#pragma unroll
    for (int s = 0; s < Geo::kHalfSets; ++s) gemv_chain_set<P>(tot, tb2 + s * (kTinyTermBytes / 4), nl, 0);
    // Lane n < 16 holds (row n, the item's one token): the down output in bf16
    // (cpu_runner.rs:2945-2947).
    const float yv = bf16r(tot);
    if (lane < kTileRows && slot < DC::kItems) {
      s_y[slot * kTileRows + nl] = yv;
      if (c.trace != nullptr && row < rows) c.trace[(size_t)slot * rows + row] = yv;
    }
  }
  __syncthreads();
  if (tid < kTileRows && row < rows) {
    float acc = 0.0f;
    for (int k = 0; k < c.top_k; ++k) acc = acc + s_y[k * kTileRows + nl] * c.weights[k];
    const float o = bf16r(acc);
    if (c.out != nullptr) c.out[row] = o;
    if (c.out16 != nullptr) c.out16[row] = (uint16_t)(__float_as_uint(o) >> 16);
    if (c.unrounded != nullptr) c.unrounded[row] = acc;
    if (c.next != nullptr) c.next[row] = bf16_bits(bf16_to_f32(c.resid[row]) + o);
  }
}

// ---------------------------------------------------------------------------
// Selection, dispatch and the gate_up GEMV of a one-row batch in one launch
// (the moe_batch routing loop, cpu_runner.rs:2808-2889, and the gate_up
// projection with SwiGLU, :2893-2919, at m = 1), after route_select_kernel
// has written the row's bf16 logits and quantized the row (launched without
// its arrival counter). Every work-group selects for itself, so that no
// cross-work-group signal or serial selection step separates the logits from
// the weight stream: the logits are requested first; wave 0 ranks the keys
// (stable_top_k, :3768-3778; experts e and e + 64 per lane, the keys read
// 16 at a time from LDS); the selected experts in increasing index are the
// work items (every bucket holds one route, so dispatch_offsets's order is
// expert order). Work-group (x, y) then requests the row's activation image
// (DMA into LDS), its tiles' flags and biases and its weight ring together,
// and runs gemv_kernel<kGateUp, 8, 2>'s tile group x for item y. (The DMA
// cannot go out before the selection: the compiler waits for LDS DMA before
// the selection's LDS accesses.) Work-group (0, 0) also writes what the selection
// kernels write for the down launch and the caller: the selection, the
// softmax weights (select_row_ranked's operations), bucket offsets, route
// order and the work list, and the non-finite flag.
struct RouteGemvGeom {
  // Two weight groups (one set) in flight per wave: with 16 waves per CU, a
  // deeper ring queues more requests ahead of each wave's next group (4 and 6
  // groups ran 4% and 8% slower per layer).
  using Geo = GemvGeom<8, 2, 2>;
  static constexpr int kThreads = Geo::kThreads;
  static constexpr int kLds = Geo::kLds;
};

__global__ __launch_bounds__(RouteGemvGeom::kThreads, 4) void route_gemv_kernel(RouteArgs r, DispatchArgs d,
                                                                                 GemmArgs a) {
  using C = GemmTinyCfg;
  using RG = RouteGemvGeom;
  using Geo = RG::Geo;
  constexpr int P = 8, V = 2, R = Geo::kRing;
  __shared__ __align__(16) char s_dyn[RG::kLds];
  __shared__ float s_lg[kMaxExperts];
  __shared__ __align__(16) uint64_t s_key[kMaxExperts];
  __shared__ int s_item[kSelectTopK], s_pick[kSelectTopK];
  __shared__ int s_rank[kMaxExperts], s_slot[kMaxExperts];  // each expert's rank and item (or route) index
  __shared__ float s_ex[kSelectTopK];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int E = r.experts, K = r.top_k;
  const int B = (int)a.w.blocks;
  const int nsets = (B + P - 1) / P;
  const bool first = blockIdx.x == 0 && blockIdx.y == 0;  // writes the routing outputs
  char* img = s_dyn;
  float* s_scl = reinterpret_cast<float*>(s_dyn + tiny_image_bytes(1));
  float* term_base = reinterpret_cast<float*>(s_dyn + tiny_image_bytes(1) + tiny_sets(1) * 64);
  // The logits (0 past the experts: a key below every real one), requested
  // together with the exp2 table's entries.
  const uint64_t exp2_entry = load_exp2_entry();
  const float lg = tid < E ? r.logits[tid] : 0.0f;
  for (int k = tid; k < nsets; k += Geo::kThreads) *reinterpret_cast<u32x4*>(img + k * kTinySetBytes + 1024) = u32x4{};
  if (tid < kMaxExperts) {
    s_lg[tid] = lg;
    s_key[tid] = tid < E ? route_key(lg, tid) : 0;
  }
  store_exp2_entry(exp2_entry);
  __syncthreads();

  // Waves 1-7 request the row's activation image (DMA into LDS; the row does
  // not depend on the selection) and wait for it while wave 0 selects, so
  // the image is complete at the selection's barrier.
  if (wave != 0) {
    const __amdgpu_buffer_rsrc_t act_codes = buffer_rsrc(a.actv), act_scl = buffer_rsrc(a.acts);
    const int i = lane >> 2, g = lane & 3, part = i & 1;
    for (int k = wave - 1; k < nsets; k += Geo::kWaves - 1) {  // uniform per wave
      const int b = k * P + i / V;
      dma16(act_codes, img + k * kTinySetBytes, b < B ? (b * 2 + part) * 64 + g * 16 : 0, 0);
    }
    for (int k = wave - 1; k * 64 < nsets * 16; k += Geo::kWaves - 1) {  // uniform per wave
      const int f = k * 64 + lane, b = f >> 1;
      dma4(act_scl, reinterpret_cast<char*>(s_scl) + k * 256, b < B ? (b * 2 + (f & 1)) * 4 : 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's share of the image is in LDS
  }
  // Wave 0 selects: lane e's key ranks among all keys (16 per LDS round
  // trip), experts e and e + 64 per lane.
  if (wave == 0) {
    int r0 = 0, r1 = 0;
    const uint64_t k0 = s_key[lane], k1 = s_key[lane + 64];
    for (int c = 0; c < E; c += 16) {  // uniform
      u64x2 kk[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) kk[j] = reinterpret_cast<const u64x2*>(s_key + c)[j];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        r0 += (kk[j][0] > k0) + (kk[j][1] > k0);
        r1 += (kk[j][0] > k1) + (kk[j][1] > k1);
      }
    }
    const bool sel0 = lane < E && r0 < K, sel1 = lane + 64 < E && r1 < K;
    const unsigned long long m0 = __ballot(sel0), m1 = __ballot(sel1), below = (1ull << lane) - 1ull;
    const int item0 = __popcll(m0 & below), item1 = __popcll(m0) + __popcll(m1 & below);
    if (sel0) {
      s_item[item0] = lane;
      s_pick[r0] = lane;
    }
    if (sel1) {
      s_item[item1] = lane + 64;
      s_pick[r1] = lane + 64;
    }
    s_rank[lane] = r0;
    s_rank[lane + 64] = r1;
    s_slot[lane] = item0;
    s_slot[lane + 64] = item1;
  }
  __syncthreads();

  // The wave's weight ring (gemv_kernel<kGateUp, 8, 2>: tile group x, item y).
  const int y = blockIdx.y;
  const int expert = s_item[y];
  const int half = wave >> 2, wt = wave & 3;
  const int nl = lane & 15;
  const int start = y, count = 1;
  const int rows = (int)a.w.rows;
  const int tile0 = blockIdx.x * C::kWaves + wt;
  const bool ok = tile0 < (int)a.w.tiles;
  const int safe_tile = ok ? tile0 : 0;
  const int nq4 = (B + 3) >> 2;
  GemvLoads L;
  L.nib = buffer_rsrc(a.w.nib + (size_t)expert * a.w.nib_stride + (size_t)safe_tile * 256 * B);
  L.scl = buffer_rsrc(a.w.scl + (size_t)expert * a.w.scl_stride + (size_t)safe_tile * 64 * nq4);
  L.vl = lane * 16;
  L.vl_tail = lane * (B & 3) * 4;
  L.vs = nl * 4;
  L.nq4 = nq4;
  L.nfull4 = B >> 2;
  const int g0 = half * (Geo::kHalfSets * P / 4);
  // The tile's fast-path flag and bias (branch-free, from valid addresses),
  // then the ring: all in flight together.
  const int row = tile0 * kTileRows + nl;
  const uint8_t fast_raw = a.w.fast[(size_t)expert * a.w.tiles + safe_tile];
  const float* bias_p =
      a.bias != nullptr ? a.bias + (size_t)expert * a.bias_expert_stride + min(row, rows - 1) : r.router_b;
  const float bias_raw = *bias_p;
  u32x4 wn[R];
  uint32_t ws[R];
#pragma unroll
  for (int q = 0; q < R; ++q) gemv_load(L, g0 + q, wn[q], ws[q]);

  const bool fast = a.fast_ok && fast_raw != 0;
  const float bias = (a.bias != nullptr && ok && row < rows) ? bias_raw : 0.0f;

  float* terms = term_base + wave * (Geo::kTermRegion / 4);
  float tot = bias + 0.0f;  // a -0.0 bias becomes +0.0, as the reference's first add does
  if (half == 0)
    tot = gemv_sets<P, R, 0, Geo::kHalfSets, false>(tot, L, wn, ws, img, s_scl, terms, B, lane, fast);
  else
    gemv_sets<P, R, Geo::kHalfSets, Geo::kSets, true>(tot, L, wn, ws, img, s_scl, terms, B, lane, fast);
  __syncthreads();  // the second half's terms are in LDS
  if (half == 0) {
    const float* tb2 = term_base + (wave + 4) * (Geo::kTermRegion / 4);
#pragma unroll
    for (int s = 0; s < Geo::kHalfSets; ++s) gemv_chain_set<P>(tot, tb2 + s * (kTinyTermBytes / 4), nl, 0);
  }
  const int G = lane >> 4;
  Acc<C> acc;
  acc[0][0][0] = __shfl(tot, ((2 * G) * 16 + nl) & 63);
  acc[0][0][1] = __shfl(tot, ((2 * G + 1) * 16 + nl) & 63);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // every wave is done with the LDS image before the epilogue reuses it
  if (half == 0) {
    gemm_epilogue<C, kGateUp, true>(a, acc, 1, count, start, tile0, reinterpret_cast<float*>(s_dyn));
  } else {
    __syncthreads();  // gemm_epilogue's one barrier (gate_up), matched by the second half's waves
    // Work-group (0, 0): the routing outputs, written after the last barrier
    // by a wave that has no epilogue work.
    if (first && wave == 4) {
      const int e0 = lane, e1 = lane + 64;
      const bool sel0 = e0 < E && s_rank[e0] < K, sel1 = e1 < E && s_rank[e1] < K;
      if ((e0 < E && !isfinite(s_lg[e0])) || (e1 < E && !isfinite(s_lg[e1]))) atomicOr(r.err, kErrNonFiniteLogits);
      if (e0 < E) d.bucket_off[e0] = s_slot[e0];  // routes of the experts below
      if (e1 < E) d.bucket_off[e1] = s_slot[e1];
      if (lane == 0) {
        d.bucket_off[E] = K;
        *d.n_work = K;
      }
      if (sel0) {
        d.route_tok[s_slot[e0]] = 0;
        d.route_slot[s_slot[e0]] = s_rank[e0];
        reinterpret_cast<int4*>(d.work)[s_slot[e0]] = make_int4(e0, s_slot[e0], 1, 0);
      }
      if (sel1) {
        d.route_tok[s_slot[e1]] = 0;
        d.route_slot[s_slot[e1]] = s_rank[e1];
        reinterpret_cast<int4*>(d.work)[s_slot[e1]] = make_int4(e1, s_slot[e1], 1, 0);
      }
      float mx = -INFINITY;
      for (int k = 0; k < K; ++k) mx = fmaxf(mx, s_lg[s_pick[k]]);
      const int my_e = s_pick[lane < K ? lane : 0];
      const float ex = expf_glibc(s_lg[my_e] - mx, s_exp2_tab);
      if (lane < K) s_ex[lane] = ex;
      __builtin_amdgcn_wave_barrier();
      float sum = 0.0f;
      for (int k = 0; k < K; ++k) sum = sum + s_ex[k];
      if (lane < K) {
        r.selected[lane] = my_e;
        r.weights[lane] = bf16r(ex / sum);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Exact-BF16 expert projection (CpuExpertProjection::ExactBf16; project_mxfp4,
// cpu_runner.rs:3497-3519): per output, total = bias; total += the 16 lane
// sums folded 0..15 from -0.0. Lane l sums bf16(decode(code) * e8m0) * x over
// the input values k = l mod 16 in increasing k, multiply then add
// (accumulate_mxfp4_bf16_block, lib.rs:932-945: value v of a block feeds lane
// v % 16, so lane l takes k = 32 b + l, then 32 b + l + 16, block after
// block). A conformance path, VALU only: a work-group is one 16-row weight
// tile x 16 lanes (one thread per row and lane) over one work item of the
// dispatch's list (at most kChunkMax routes, one accumulator each).
// gate_up: bf16 round trip, SwiGLU pairs (rows 2i, 2i + 1 of the tile) into
// the down input [grouped route][rows / 2] bf16; down: y [slot][rows] bf16.

__constant__ float kE2M1[16] = {0.0f,  0.5f,  1.0f,  1.5f,  2.0f,  3.0f,  4.0f,  6.0f,
                                -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

template <int MODE>
__global__ __launch_bounds__(256) void exact_kernel(GemmArgs a) {
  const int tid = threadIdx.x, nn = tid >> 4, l = tid & 15;
  const int wi = blockIdx.y;
  const int nw = *a.n_work;
  const int4 rec = reinterpret_cast<const int4*>(a.work)[wi];
  if (wi >= nw) return;  // uniform over the work-group
  const int expert = rec.x, start = rec.y, count = rec.z;
  const int rows = (int)a.w.rows, B = (int)a.w.blocks, K = B * kBlock;
  const int tile = blockIdx.x, n = tile * kTileRows + nn;
  const int nq4 = (B + 3) >> 2;
  const uint8_t* nib = a.w.nib + (size_t)expert * a.w.nib_stride + (size_t)tile * 256 * B;
  const uint8_t* scl = a.w.scl + (size_t)expert * a.w.scl_stride + (size_t)tile * 64 * nq4;
  __shared__ const uint16_t* s_in[kChunkMax];
  if (tid < kChunkMax) {
    const int t = min(tid, count - 1);
    const size_t src = MODE == kGateUp ? (size_t)a.route_tok[start + t] : (size_t)(start + t);
    s_in[tid] = a.xin + src * K;
  }
  __syncthreads();
  float acc[kChunkMax];
#pragma unroll
  for (int t = 0; t < kChunkMax; ++t) acc[t] = 0.0f;
  const int g_lo = l >> 3, shift = 4 * (l & 7);
  for (int b = 0; b < B; ++b) {
    const int q = b >> 2, j = b & 3, nb = min(4, B - 4 * q);
    // Codes l and l + 16 of row nn: k-slices l / 8 and 2 + l / 8 of the group.
    const uint32_t d0 = *reinterpret_cast<const uint32_t*>(nib + q * 1024 + (g_lo * 16 + nn) * nb * 4 + j * 4);
    const uint32_t d1 = *reinterpret_cast<const uint32_t*>(nib + q * 1024 + ((2 + g_lo) * 16 + nn) * nb * 4 + j * 4);
    const float scale = e8m0(scl[q * 64 + nn * 4 + j]);
    const float w0 = bf16r(kE2M1[(d0 >> shift) & 15u] * scale);
    const float w1 = bf16r(kE2M1[(d1 >> shift) & 15u] * scale);
#pragma unroll
    for (int t = 0; t < kChunkMax; ++t) {
      if (t < count) {
        const uint16_t* xr = s_in[t] + b * kBlock;
        acc[t] = acc[t] + w0 * bf16_to_f32(xr[l]);
        acc[t] = acc[t] + w1 * bf16_to_f32(xr[l + 16]);
      }
    }
  }
  __shared__ float s_lane[kTileRows][16][kChunkMax + 1];
  __shared__ float s_gu[kTileRows][kChunkMax];
#pragma unroll
  for (int t = 0; t < kChunkMax; ++t)
    if (t < count) s_lane[nn][l][t] = acc[t];
  __syncthreads();
  for (int t = l; t < count; t += 16) {
    float sum = -0.0f;
    for (int ll = 0; ll < 16; ++ll) sum = sum + s_lane[nn][ll][t];
    const float bias = (a.bias != nullptr && n < rows) ? a.bias[(size_t)expert * a.bias_expert_stride + n] : 0.0f;
    const float total = bias + sum;
    const int slot = a.route_slot[start + t];
    if (MODE == kDown) {
      if (n < rows) a.y[(size_t)slot * rows + n] = bf16_bits(total);  // bf16 (cpu_runner.rs:2945-2947)
    } else {
      const float gu = bf16r(total);  // bf16 (cpu_runner.rs:2905)
      s_gu[nn][t] = gu;
      if (a.trace_gu != nullptr && n < rows) a.trace_gu[(size_t)slot * rows + n] = gu;
    }
  }
  if (MODE == kGateUp) {
    __syncthreads();
    const int half = rows / 2;
    for (int idx = tid; idx < (kTileRows / 2) * count; idx += blockDim.x) {
      const int p = idx % (kTileRows / 2), t = idx / (kTileRows / 2);
      const int i = tile * (kTileRows / 2) + p;
      if (i < half) {
        const float act = swiglu_one(s_gu[2 * p][t], s_gu[2 * p + 1][t], a.alpha, a.limit, a.sig_tab);
        a.act_next16[(size_t)(start + t) * half + i] = bf16_bits(act);  // activated_bf16 (cpu_runner.rs:2917)
        if (a.trace_sw != nullptr) a.trace_sw[(size_t)a.route_slot[start + t] * half + i] = act;
      }
    }
  }
}

// Exactness flag per (expert, tile): 1 when every E8M0 byte of the tile's
// blocks lies in [kFastScaleLo, kFastScaleHi]. One work-group per tile.
__global__ __launch_bounds__(256) void tile_flags_kernel(TiledWeights w) {
  const size_t e = blockIdx.y, t = blockIdx.x;
  const size_t nq = (w.blocks + 3) / 4;
  const uint8_t* scl = w.scl + e * w.scl_stride + t * 64 * nq;
  int bad = 0;
  for (size_t i = threadIdx.x; i < kTileRows * w.blocks; i += blockDim.x) {
    const size_t n = i / w.blocks, b = i % w.blocks;
    const uint32_t s = scl[(b / 4) * 64 + n * 4 + (b % 4)];
    bad |= (s - kFastScaleLo) > (kFastScaleHi - kFastScaleLo);
  }
  bad = __syncthreads_or(bad);
  if (threadIdx.x == 0) w.fast[e * w.tiles + t] = bad ? 0 : 1;
}

// ---------------------------------------------------------------------------
// Weighted combine by source row and rank (cpu_runner.rs:2959-2999):
// out = 0; out += y_rank * w_rank in rank order; then bf16.

// Eight consecutive outputs per thread: 16-byte bf16 loads of each rank's
// row, two float4 stores. For 16-byte-aligned outputs (hidden % 8 == 0).
// Combine (cpu_runner.rs:2959-2999): out = bf16(sum over ranks in order of
// y_rank * w_rank), from 0.0. With `next`, also the residual add of the
// decoder layer (add_residual, cpu_runner.rs:3732-3738): next =
// bf16(resid + out). `out` may be null when only `next` is wanted.
__global__ __launch_bounds__(256) void combine8_kernel(const uint16_t* y, const float* w, int top_k, int hidden,
                                                      float* out, uint16_t* out16, float* trace,
                                                      const uint16_t* resid, uint16_t* next, float* unrounded) {
  const int r = blockIdx.y;
  const int h = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (h >= hidden) return;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  // The first kCombineBatch ranks' rows and weights are requested together
  // (one memory round trip), then added in rank order.
  constexpr int kCombineBatch = 4;
  u32x4 pb[kCombineBatch];
  float wb[kCombineBatch];
#pragma unroll
  for (int k = 0; k < kCombineBatch; ++k) {
    const size_t slot = (size_t)r * top_k + (k < top_k ? k : 0);
    pb[k] = *reinterpret_cast<const u32x4*>(y + slot * hidden + h);
    wb[k] = w[slot];
  }
  for (int k = 0; k < top_k; ++k) {
    const size_t slot = (size_t)r * top_k + k;
    const u32x4 p = k < kCombineBatch ? pb[k < kCombineBatch ? k : 0] : *reinterpret_cast<const u32x4*>(y + slot * hidden + h);
    const float wk = k < kCombineBatch ? wb[k < kCombineBatch ? k : 0] : w[slot];
    float v[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[2 * q] = __uint_as_float(p[q] << 16);
      v[2 * q + 1] = __uint_as_float(p[q] & 0xffff0000u);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = acc[e] + v[e] * wk;
    if (trace) {
      float4* t = reinterpret_cast<float4*>(trace + slot * hidden + h);
      t[0] = make_float4(v[0], v[1], v[2], v[3]);
      t[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
  }
  if (unrounded) {  // the sum before fp32_to_bf16_roundtrip (cpu_runner.rs:2991)
    float4* up = reinterpret_cast<float4*>(unrounded + (size_t)r * hidden + h);
    up[0] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    up[1] = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = bf16r(acc[e]);
  if (out) {
    float4* op = reinterpret_cast<float4*>(out + (size_t)r * hidden + h);
    op[0] = make_float4(o[0], o[1], o[2], o[3]);
    op[1] = make_float4(o[4], o[5], o[6], o[7]);
  }
  if (out16) {  // the same values as bf16 bits (exact: every o is a bf16 value)
    u32x4 ob;
#pragma unroll
    for (int q = 0; q < 4; ++q) ob[q] = (__float_as_uint(o[2 * q]) >> 16) | (__float_as_uint(o[2 * q + 1]) & 0xffff0000u);
    *reinterpret_cast<u32x4*>(out16 + (size_t)r * hidden + h) = ob;
  }
  if (next) {
    const u32x4 rp = *reinterpret_cast<const u32x4*>(resid + (size_t)r * hidden + h);
    u32x4 np;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = bf16_bits(__uint_as_float(rp[q] << 16) + o[2 * q]);
      const uint32_t hi = bf16_bits(__uint_as_float(rp[q] & 0xffff0000u) + o[2 * q + 1]);
      np[q] = lo | (hi << 16);
    }
    *reinterpret_cast<u32x4*>(next + (size_t)r * hidden + h) = np;
  }
}

__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* y, const float* w, int top_k, int hidden,
                                                     float* out, uint16_t* out16, float* trace,
                                                     const uint16_t* resid, uint16_t* next, float* unrounded) {
  const int r = blockIdx.y;
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= hidden) return;
  float acc = 0.0f;
  for (int k = 0; k < top_k; ++k) {
    const size_t slot = (size_t)r * top_k + k;
    const float v = bf16_to_f32(y[slot * hidden + h]);
    acc = acc + v * w[slot];
    if (trace) trace[slot * hidden + h] = v;
  }
  if (unrounded) unrounded[(size_t)r * hidden + h] = acc;
  const float o = bf16r(acc);
  if (out) out[(size_t)r * hidden + h] = o;
  if (out16) out16[(size_t)r * hidden + h] = (uint16_t)(__float_as_uint(o) >> 16);
  if (next) next[(size_t)r * hidden + h] = bf16_bits(bf16_to_f32(resid[(size_t)r * hidden + h]) + o);
}

// ---------------------------------------------------------------------------
// Reference activation records -> GEMM operand. Q8Block {f32 scale; i8[32]}
// is 36 bytes, ResidualQ8Block {primary; residual} 72 bytes (lib.rs:732-742).

__global__ __launch_bounds__(256) void prep_records_kernel(const uint8_t* rec, int kind, int m, int blocks,
                                                          size_t row_stride, ActBuffers act) {
  const int hw = (blockIdx.x * blockDim.x + threadIdx.x) >> 5;
  const int l32 = threadIdx.x & 31;
  if (hw >= m * blocks) return;
  const int r = hw / blocks, b = hw % blocks;
  const size_t rsz = kind == 2 ? 72 : 36;
  const uint8_t* p = rec + ((size_t)r * row_stride + b) * rsz;
  const float ps = *reinterpret_cast<const float*>(p);
  const int8_t pq = (int8_t)p[4 + l32];
  float rs = 0.0f;
  int8_t rq = 0;
  if (kind == 2) {
    rs = *reinterpret_cast<const float*>(p + 36);
    rq = (int8_t)p[40 + l32];
  }
  _Float16* dst = act.v + (((size_t)r * blocks + b) * 2) * kBlock;
  dst[l32] = (_Float16)(float)pq;
  dst[kBlock + l32] = (_Float16)(float)rq;
  if (l32 == 0) {
    float2 sc;
    sc.x = ps;
    sc.y = rs;
    reinterpret_cast<float2*>(act.s)[(size_t)r * blocks + b] = sc;
  }
}

// ---------------------------------------------------------------------------
// Layout conversion into the resident v3 layout.

__device__ __forceinline__ void v3_offsets(const TiledWeights& w, size_t e, size_t row, size_t b, size_t g,
                                           size_t* nib_off, size_t* scl_off) {
  const size_t B = w.blocks, t = row / kTileRows, n = row % kTileRows, q = b / 4, j = b % 4;
  const size_t nb = B - 4 * q < 4 ? B - 4 * q : 4;
  *nib_off = e * w.nib_stride + t * 256 * B + q * 1024 + (g * 16 + n) * nb * 4 + j * 4;
  *scl_off = e * w.scl_stride + t * 64 * ((B + 3) / 4) + q * 64 + n * 4 + j;
}

// Mxfp4MatrixView::block (lib.rs:810-851) for canonical v1 and x8 v2 data of
// one expert: fills the 16 adjacent-packed bytes and the scale byte.
__device__ void view_block(const uint8_t* data, int layout, size_t rows, size_t blocks, size_t row, size_t b,
                           uint8_t packed[16], uint8_t* scale) {
  if (layout == 1) {
    const uint8_t* p = data + (row * blocks + b) * kRecord;
    *scale = p[0];
    for (int i = 0; i < 16; ++i) packed[i] = p[1 + i];
    return;
  }
  const size_t complete = rows / 8 * 8;
  if (row < complete) {
    const size_t group = row / 8, lane = row % 8;
    const uint8_t* x8 = data + (group * blocks + b) * 136;
    uint8_t split[16];
    for (int i = 0; i < 16; ++i) split[i] = x8[8 + (i / 8) * 64 + lane * 8 + i % 8];
    *scale = x8[lane];
    // mxfp4_split_to_adjacent (lib.rs:919-928): split byte i = code(i) | code(i+16) << 4.
    for (int i = 0; i < 16; ++i) {
      const int c0 = 2 * i, c1 = 2 * i + 1;
      const uint8_t lo = c0 < 16 ? (split[c0] & 0x0f) : (split[c0 - 16] >> 4);
      const uint8_t hi = c1 < 16 ? (split[c1] & 0x0f) : (split[c1 - 16] >> 4);
      packed[i] = (uint8_t)(lo | (hi << 4));
    }
    return;
  }
  const uint8_t* p = data + (rows / 8) * blocks * 136 + ((row - complete) * blocks + b) * kRecord;
  *scale = p[0];
  for (int i = 0; i < 16; ++i) packed[i] = p[1 + i];
}

__device__ __forceinline__ void store_v3(const TiledWeights& w, size_t e, size_t row, size_t b, const uint8_t packed[16],
                                         uint8_t scale) {
  for (size_t g = 0; g < 4; ++g) {
    size_t no, so;
    v3_offsets(w, e, row, b, g, &no, &so);
    const uint32_t d = (uint32_t)packed[4 * g] | ((uint32_t)packed[4 * g + 1] << 8) |
                       ((uint32_t)packed[4 * g + 2] << 16) | ((uint32_t)packed[4 * g + 3] << 24);
    *reinterpret_cast<uint32_t*>(w.nib + no) = d;
    if (g == 0) w.scl[so] = scale;
  }
}

__global__ void repack_kernel(const uint8_t* src, int layout, TiledWeights w) {
  const size_t per_expert = w.rows * w.blocks;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= w.experts * per_expert) return;
  const size_t e = i / per_expert, rb = i % per_expert, row = rb / w.blocks, b = rb % w.blocks;
  uint8_t packed[16], scale;
  view_block(src + e * per_expert * kRecord, layout, w.rows, w.blocks, row, b, packed, &scale);
  store_v3(w, e, row, b, packed, scale);
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t stream_hash(uint64_t seed, uint64_t stream, uint64_t index) {
  return splitmix64(splitmix64(seed ^ (stream * 0xD1B54A32D192ED03ull)) + index);
}

__global__ void generate_kernel(uint64_t seed, uint64_t stream, TiledWeights w) {
  const size_t per_expert = w.rows * w.blocks;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= w.experts * per_expert) return;
  const size_t e = i / per_expert, rb = i % per_expert, row = rb / w.blocks, b = rb % w.blocks;
  const uint64_t h0 = stream_hash(seed, stream, 2 * i), h1 = stream_hash(seed, stream, 2 * i + 1);
  uint8_t packed[16];
  for (int j = 0; j < 8; ++j) packed[j] = (uint8_t)(h0 >> (8 * j));
  for (int j = 0; j < 8; ++j) packed[8 + j] = (uint8_t)(h1 >> (8 * j));
  store_v3(w, e, row, b, packed, (uint8_t)(119 + (h1 >> 61) % 5));
}

__global__ void export_kernel(TiledWeights w, uint8_t* dst) {
  const size_t per_expert = w.rows * w.blocks;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= w.experts * per_expert) return;
  const size_t e = i / per_expert, rb = i % per_expert, row = rb / w.blocks, b = rb % w.blocks;
  uint8_t* p = dst + i * kRecord;
  for (size_t g = 0; g < 4; ++g) {
    size_t no, so;
    v3_offsets(w, e, row, b, g, &no, &so);
    const uint32_t d = *reinterpret_cast<const uint32_t*>(w.nib + no);
    for (int k = 0; k < 4; ++k) p[1 + 4 * g + k] = (uint8_t)(d >> (8 * k));
    if (g == 0) p[0] = w.scl[so];
  }
}

// Padding rows of the last tile: zero codes, scale 127.
__global__ void fill_padding_kernel(TiledWeights w) {
  const size_t pad_rows = w.tiles * kTileRows - w.rows;
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= w.experts * pad_rows * w.blocks) return;
  const size_t e = i / (pad_rows * w.blocks), rb = i % (pad_rows * w.blocks);
  const size_t row = w.rows + rb / w.blocks, b = rb % w.blocks;
  const uint8_t zero[16] = {0};
  store_v3(w, e, row, b, zero, 127);
}

__global__ void clear_ints_kernel(int* p, size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// E8M0 exponents, byte positions and neighbour-byte patterns of the dirty
// scale operands the self-test converts with (every other byte of the scale
// dword holds the pattern, so sign and mantissa bits of the operand are set).
__constant__ uint32_t kDirtyExp[5] = {kFastScaleLo, 120, 127, 133, kFastScaleHi};
__constant__ uint32_t kDirtyPattern[6] = {0x00, 0xff, 0x80, 0x7f, 0xa5, 0x01};

// Lane-layout self-test of the two gfx950 builtins the GEMM relies on.
// out[0..7]: v_cvt_scalef32_pk_f16_fp4 of codes 0..7 (bytes 0x10 0x32 0x54 0x76).
// out[8 + 4 * lane + r]: D of a 16x16x32 f16 MFMA with A[i][k] = (k == i) and
// B[k][j] = 10 k + j, expected 10 * (4 * (lane / 16) + r) + lane % 16.
// out[264..271]: codes 0..7 converted with scale 2^-4.
// out[272 + 16 * c + i], case c = (exponent x, byte j, pattern p) in that
// order: code i (0..15) converted through e8m0_scale_operand(s, j) of the
// dword s whose byte j is kDirtyExp[x] and whose other bytes are
// kDirtyPattern[p]; expected decode(i) * 2^(e - 127).
__global__ void selftest_kernel(float* out) {
  const int lane = threadIdx.x;
  const half8 w = fp4x8_to_half8(0x76543210u);
  if (lane == 0)
    for (int i = 0; i < 8; ++i) out[i] = (float)w[i];
  half8 av, bv;
  for (int e = 0; e < 8; ++e) {
    const int k = 8 * (lane >> 4) + e;
    av[e] = (_Float16)((k == (lane & 15)) ? 1.0f : 0.0f);
    bv[e] = (_Float16)(float)(10 * k + (lane & 15));
  }
  const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
  const f32x4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, zero, 0, 0, 0);
  for (int r = 0; r < 4; ++r) out[8 + 4 * lane + r] = d[r];
  // out[264..271]: the scaled conversion with E8M0 byte 123 (2^-4).
  const half8 ws = fp4x8_to_half8_scaled(0x76543210u, __uint_as_float(123u << 23));
  if (lane == 0)
    for (int i = 0; i < 8; ++i) out[264 + i] = (float)ws[i];
  for (int c = lane; c < kSelftestDirty; c += 64) {
    const int x = c / 24, j = (c / 6) % 4, p = c % 6;
    uint32_t s = kDirtyPattern[p] * 0x01010101u;
    s = (s & ~(0xffu << (8 * j))) | (kDirtyExp[x] << (8 * j));
    float sc;
    switch (j) {  // e8m0_scale_operand takes its byte position as a constant
      case 0: sc = e8m0_scale_operand(s, 0); break;
      case 1: sc = e8m0_scale_operand(s, 1); break;
      case 2: sc = e8m0_scale_operand(s, 2); break;
      default: sc = e8m0_scale_operand(s, 3); break;
    }
    const half8 lo = fp4x8_to_half8_scaled(0x76543210u, sc);
    const half8 hi = fp4x8_to_half8_scaled(0xfedcba98u, sc);
    for (int i = 0; i < 8; ++i) {
      out[272 + 16 * c + i] = (float)lo[i];
      out[272 + 16 * c + 8 + i] = (float)hi[i];
    }
  }
  for (int k = lane; k < kSelftestBf16; k += 64)
    out[kSelftestBf16Base + k] = (float)bf16_bits(__uint_as_float(selftest_bf16_input(k)));
}

// ---------------------------------------------------------------------------
// Launchers.

static inline unsigned grid1d(size_t n, unsigned block) { return (unsigned)((n + block - 1) / block); }

hipError_t launch_route(const RouteArgs& a, hipStream_t stream) {
  const int quant_groups = a.quant ? (a.hidden / kBlock + kRouteQuantBlocks - 1) / kRouteQuantBlocks : 0;
  if (a.hidden % 32 != 0 || a.experts > kMaxExperts) return hipErrorInvalidValue;
  hipLaunchKernelGGL(route_kernel, dim3(a.m, router_groups(a) + quant_groups), dim3(256), 0, stream, a);
  return hipGetLastError();
}

// Rows per selection work-group of the two-launch path (a power of two).
int select_rows_per_wg(int experts, int top_k) {
  int rw = 256;
  while (rw > 16 && (rw * (experts + 1) > kSelectLds || rw * top_k > 1024)) rw >>= 1;
  // Then as many work-groups as keep at least four experts per lane (the
  // selection of 256 rows over 128 experts took 29 µs with 64 rows per
  // work-group, 25 µs with 32; two experts per lane was no faster).
  while (rw > 16 && (1024 / (rw / 2)) * 4 <= experts) rw >>= 1;
  return rw;
}

hipError_t launch_select_count(const RouteArgs& r, int quantize, int* cnt, hipStream_t stream) {
  const int rw = select_rows_per_wg(r.experts, r.top_k);
  if (r.top_k > kMaxTopK || r.experts > kMaxExperts || rw * (r.experts + 1) > kSelectLds || rw * r.top_k > 1024 ||
      1024 / rw > 64)
    return hipErrorInvalidValue;
  const int n_sel = (r.m + rw - 1) / rw;
  const size_t qblocks = quantize ? (size_t)r.m * (r.hidden / kBlock) : 0;
  const unsigned grid = (unsigned)n_sel + (unsigned)((qblocks + kSelectQuantBlocks - 1) / kSelectQuantBlocks);
  if (r.top_k <= 4)
    hipLaunchKernelGGL(select_count_kernel<4>, dim3(grid), dim3(1024), 0, stream, r, rw, n_sel, cnt);
  else
    hipLaunchKernelGGL(select_count_kernel<kMaxTopK>, dim3(grid), dim3(1024), 0, stream, r, rw, n_sel, cnt);
  return hipGetLastError();
}

hipError_t launch_place(const DispatchArgs& a, int m, const int* cnt, hipStream_t stream) {
  const int rw = select_rows_per_wg(a.experts, a.top_k);
  const int n_sel = (m + rw - 1) / rw;
  hipLaunchKernelGGL(place_kernel, dim3(n_sel), dim3(1024), 0, stream, a, rw * a.top_k, n_sel, cnt);
  return hipGetLastError();
}

hipError_t launch_select_dispatch(const RouteArgs& r, const DispatchArgs& d, int quantize, hipStream_t stream) {
  if (r.m * (r.experts + 1) > kSelectLds || d.routes > kSelectMaxRoutes || r.top_k > kSelectTopK ||
      r.experts > kMaxExperts)
    return hipErrorInvalidValue;
  const size_t qblocks = quantize ? (size_t)r.m * (r.hidden / kBlock) : 0;
  const unsigned grid = 1u + (unsigned)((qblocks + kSelectQuantBlocks - 1) / kSelectQuantBlocks);
  hipLaunchKernelGGL(select_dispatch_kernel, dim3(grid), dim3(1024), 0, stream, r, d);
  return hipGetLastError();
}

hipError_t launch_route_select(const RouteArgs& r, const DispatchArgs& d, int* counter, hipStream_t stream) {
  // Every bucket must be one work item (at most m routes per expert).
  if (r.m < 1 || r.m > kFusedRouteRows || r.hidden > kFusedRouteHidden || r.hidden % 32 != 0 || r.injected != nullptr ||
      r.top_k > kSelectTopK || r.experts > kMaxExperts || d.chunk < r.m || d.routes != r.m * r.top_k)
    return hipErrorInvalidValue;
  const size_t qblocks = r.quant ? (size_t)r.m * (r.hidden / kBlock) : 0;
  const unsigned grid = (unsigned)r.experts + (unsigned)((qblocks + kSelectQuantBlocks - 1) / kSelectQuantBlocks);
  hipLaunchKernelGGL(route_select_kernel, dim3(grid), dim3(1024), 0, stream, r, d, counter);
  return hipGetLastError();
}

template <class C>
static hipError_t launch_gemm_cfg(GemmMode mode, const GemmArgs& a, int grid_work, hipStream_t stream,
                                  hipEvent_t start, hipEvent_t stop) {
  const unsigned n_x = (unsigned)((a.w.tiles + C::kWgTiles - 1) / C::kWgTiles);
  const bool pin = C::kPinXcd && mode == kGateUp;
  const dim3 grid(pin ? (n_x + 7) & ~7u : n_x, (unsigned)grid_work);
  const dim3 block(C::kThreads);
  auto go = [&](auto kernel) {
    if (start) hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, start, stop, 0, a);
    else hipLaunchKernelGGL(kernel, grid, block, 0, stream, a);
  };
  if (a.residual) {
    switch (mode) {
      case kPlain: go(gemm_kernel<C, kPlain, true>); break;
      case kGateUp: go(gemm_kernel<C, kGateUp, true>); break;
      case kDown: go(gemm_kernel<C, kDown, true>); break;
    }
  } else {
    switch (mode) {
      case kPlain: go(gemm_kernel<C, kPlain, false>); break;
      case kGateUp: go(gemm_kernel<C, kGateUp, false>); break;
      case kDown: go(gemm_kernel<C, kDown, false>); break;
    }
  }
  return hipGetLastError();
}

hipError_t launch_gemm(GemmMode mode, const GemmArgs& a, int chunk, int grid_work, hipStream_t stream,
                       hipEvent_t start, hipEvent_t stop) {
  if (chunk == GemmSmall::kChunk) return launch_gemm_cfg<GemmSmall>(mode, a, grid_work, stream, start, stop);
  if (chunk == GemmBig::kChunk) return launch_gemm_cfg<GemmBig>(mode, a, grid_work, stream, start, stop);
  if (chunk == GemmHuge::kChunk) return launch_gemm_cfg<GemmHuge>(mode, a, grid_work, stream, start, stop);
  return hipErrorInvalidValue;
}

hipError_t launch_gemv(GemmMode mode, const GemmArgs& a, int rows_max, int grid_work, hipStream_t stream,
                       hipEvent_t start, hipEvent_t stop) {
  if (a.w.blocks > (size_t)kTinyMaxBlocks || rows_max < 1 || rows_max > kTinyMaxRows) return hipErrorInvalidValue;
  // Residual-Q8 activations only: the Q8 projection (no residual term) runs
  // the tiled GEMM at every batch size.
  if (!a.residual) return hipErrorInvalidValue;
  const int mp_max = rows_max <= 1 ? 1 : (rows_max <= 2 ? 2 : 4);
  const dim3 grid((unsigned)((a.w.tiles + GemmTinyCfg::kWgTiles - 1) / GemmTinyCfg::kWgTiles), (unsigned)grid_work);
  auto go = [&](auto kernel, int threads, int lds) {
    if (start) hipExtLaunchKernelGGL(kernel, grid, dim3(threads), (unsigned)lds, stream, start, stop, 0, a);
    else hipLaunchKernelGGL(kernel, grid, dim3(threads), (unsigned)lds, stream, a);
  };
  // One token: sets of 8 blocks, each tile's K range over two waves; two
  // tokens: sets of 4; three or four: sets of 2.
  using G8 = GemvGeom<8, 2>;
  using G4 = GemvGeom<4, 1>;
  using G2 = GemvGeom<2, 1>;
  auto pick = [&](auto k8, auto k4, auto k2) {
    if (mp_max == 1) go(k8, G8::kThreads, G8::kLds);
    else if (mp_max == 2) go(k4, G4::kThreads, G4::kLds);
    else go(k2, G2::kThreads, G2::kLds);
  };
  switch (mode) {
    case kPlain: pick(gemv_kernel<kPlain, 8, 2>, gemv_kernel<kPlain, 4, 1>, gemv_kernel<kPlain, 2, 1>); break;
    case kGateUp: pick(gemv_kernel<kGateUp, 8, 2>, gemv_kernel<kGateUp, 4, 1>, gemv_kernel<kGateUp, 2, 1>); break;
    case kDown: pick(gemv_kernel<kDown, 8, 2>, gemv_kernel<kDown, 4, 1>, gemv_kernel<kDown, 2, 1>); break;
  }
  return hipGetLastError();
}

hipError_t launch_route_logits(const RouteArgs& r, hipStream_t stream) {
  if (r.m < 1 || r.m > kFusedRouteRows || r.hidden > kFusedRouteHidden || r.hidden % 32 != 0 || r.injected != nullptr ||
      r.experts > kMaxExperts)
    return hipErrorInvalidValue;
  const size_t qblocks = r.quant ? (size_t)r.m * (r.hidden / kBlock) : 0;
  const unsigned grid = (unsigned)r.experts + (unsigned)((qblocks + kSelectQuantBlocks - 1) / kSelectQuantBlocks);
  hipLaunchKernelGGL(route_select_kernel, dim3(grid), dim3(1024), 0, stream, r, DispatchArgs{}, (int*)nullptr);
  return hipGetLastError();
}

hipError_t launch_route_gemv(const RouteArgs& r, const DispatchArgs& d, const GemmArgs& g, hipStream_t stream,
                             hipEvent_t start, hipEvent_t stop) {
  // One row, its logits in r.logits and its residual-Q8 input in g.actv /
  // g.acts; every selected expert is one work item of one route.
  if (r.m != 1 || r.injected != nullptr || r.experts < 1 || r.experts > kRouteGemvExperts || r.top_k < 1 ||
      r.top_k > kSelectTopK || r.top_k > r.experts || r.hidden % kBlock != 0 ||
      g.w.blocks > (size_t)kTinyMaxBlocks || r.qmode != kProjResidualQ8 || !g.residual ||
      g.w.blocks != (size_t)(r.hidden / kBlock) || g.trace_gu != nullptr || g.trace_sw != nullptr ||
      d.routes != r.top_k)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)((g.w.tiles + GemmTinyCfg::kWgTiles - 1) / GemmTinyCfg::kWgTiles), (unsigned)r.top_k);
  const dim3 block(RouteGemvGeom::kThreads);
  if (start) hipExtLaunchKernelGGL(route_gemv_kernel, grid, block, 0, stream, start, stop, 0, r, d, g);
  else hipLaunchKernelGGL(route_gemv_kernel, grid, block, 0, stream, r, d, g);
  return hipGetLastError();
}

hipError_t launch_down_combine(const GemmArgs& d, const float* weights, int top_k, float* out, uint16_t* out16,
                               float* trace_down, const uint16_t* resid, uint16_t* next, float* unrounded,
                               hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  if (d.w.blocks > (size_t)kTinyMaxBlocks || !d.residual || top_k < 1 || top_k > DownCombineGeom::kItems ||
      (next != nullptr && resid == nullptr))
    return hipErrorInvalidValue;
  CombineArgs c{weights, top_k, out, out16, trace_down, resid, next, unrounded};
  const dim3 grid((unsigned)d.w.tiles), block(DownCombineGeom::kThreads);
  if (start) hipExtLaunchKernelGGL(gemv_down_combine_kernel, grid, block, 0, stream, start, stop, 0, d, c);
  else hipLaunchKernelGGL(gemv_down_combine_kernel, grid, block, 0, stream, d, c);
  return hipGetLastError();
}

hipError_t launch_exact(GemmMode mode, const GemmArgs& a, int grid_work, hipStream_t stream) {
  const dim3 grid((unsigned)a.w.tiles, (unsigned)grid_work);
  if (mode == kGateUp) hipLaunchKernelGGL(exact_kernel<kGateUp>, grid, dim3(256), 0, stream, a);
  else if (mode == kDown) hipLaunchKernelGGL(exact_kernel<kDown>, grid, dim3(256), 0, stream, a);
  else return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_tile_flags(TiledWeights w, hipStream_t stream) {
  if (w.experts == 0 || w.tiles == 0) return hipSuccess;
  hipLaunchKernelGGL(tile_flags_kernel, dim3((unsigned)w.tiles, (unsigned)w.experts), dim3(256), 0, stream, w);
  return hipGetLastError();
}

hipError_t launch_combine(const uint16_t* y, const float* weights, int m, int top_k, int hidden, float* out,
                          uint16_t* out16, float* trace_down, const uint16_t* resid, uint16_t* next,
                          float* unrounded, hipStream_t stream) {
  const auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  const bool aligned = hidden % 8 == 0 && a16(y) && a16(out) && a16(out16) && a16(trace_down) && a16(resid) &&
                       a16(next) && a16(unrounded);
  if (aligned)
    hipLaunchKernelGGL(combine8_kernel, dim3(grid1d(hidden / 8, 256), m), dim3(256), 0, stream, y, weights, top_k,
                       hidden, out, out16, trace_down, resid, next, unrounded);
  else
    hipLaunchKernelGGL(combine_kernel, dim3(grid1d(hidden, 256), m), dim3(256), 0, stream, y, weights, top_k,
                       hidden, out, out16, trace_down, resid, next, unrounded);
  return hipGetLastError();
}

hipError_t launch_prep_records(const uint8_t* records, int kind, size_t m, size_t blocks, size_t row_stride,
                               ActBuffers act, int* /*err*/, hipStream_t stream) {
  hipLaunchKernelGGL(prep_records_kernel, dim3(grid1d(m * blocks * 32, 256)), dim3(256), 0, stream, records, kind,
                     (int)m, (int)blocks, row_stride, act);
  return hipGetLastError();
}

hipError_t launch_repack(const uint8_t* src, int layout, TiledWeights w, hipStream_t stream) {
  hipLaunchKernelGGL(repack_kernel, dim3(grid1d(w.experts * w.rows * w.blocks, 256)), dim3(256), 0, stream, src,
                     layout, w);
  return hipGetLastError();
}

hipError_t launch_generate(uint64_t seed, uint64_t stream_id, TiledWeights w, hipStream_t stream) {
  hipLaunchKernelGGL(generate_kernel, dim3(grid1d(w.experts * w.rows * w.blocks, 256)), dim3(256), 0, stream, seed,
                     stream_id, w);
  return hipGetLastError();
}

hipError_t launch_export(TiledWeights w, uint8_t* dst, hipStream_t stream) {
  hipLaunchKernelGGL(export_kernel, dim3(grid1d(w.experts * w.rows * w.blocks, 256)), dim3(256), 0, stream, w, dst);
  return hipGetLastError();
}

hipError_t launch_fill_tiled_padding(TiledWeights w, hipStream_t stream) {
  const size_t n = w.experts * (w.tiles * kTileRows - w.rows) * w.blocks;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_padding_kernel, dim3(grid1d(n, 256)), dim3(256), 0, stream, w);
  return hipGetLastError();
}

// blockIdx.y = piece; work-groups along x stride through it (16 bytes per
// thread where the piece allows, then the 4-byte tail).
__global__ void pack_kernel(PackArgs a) {
  const int pc = blockIdx.y;
  if (pc == 0 && blockIdx.x == 0 && threadIdx.x == 0) reinterpret_cast<int*>(a.dst)[0] = *a.err;
  if (pc >= a.pieces) return;
  const size_t words = a.words[pc];
  const uint32_t* src = static_cast<const uint32_t*>(a.src[pc]);
  uint32_t* dst = reinterpret_cast<uint32_t*>(a.dst + a.off[pc]);
  const size_t stride = (size_t)gridDim.x * blockDim.x, first = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t quads = (reinterpret_cast<uintptr_t>(src) & 15) ? 0 : words / 4;
  for (size_t i = first; i < quads; i += stride)
    reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
  for (size_t i = 4 * quads + first; i < words; i += stride) dst[i] = src[i];
}

hipError_t launch_pack(const PackArgs& a, hipStream_t stream) {
  uint64_t most = 0;
  for (int i = 0; i < a.pieces; ++i) most = std::max(most, a.words[i]);
  const int gx = (int)std::min<uint64_t>(256, std::max<uint64_t>(1, (most / 4 + 255) / 256));
  hipLaunchKernelGGL(pack_kernel, dim3(gx, std::max(1, a.pieces)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_clear_ints(int* p, size_t n, hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(clear_ints_kernel, dim3(grid1d(n, 256)), dim3(256), 0, stream, p, n);
  return hipGetLastError();
}

hipError_t launch_build_sigmoid_table(uint16_t* tab, hipStream_t stream) {
  hipLaunchKernelGGL(build_sigmoid_table_kernel, dim3(256), dim3(256), 0, stream, tab);
  return hipGetLastError();
}

// half 2.7.1's from_f32 restated with integer operations, the check's
// reference for bf16_bits.
__device__ __forceinline__ uint16_t bf16_bits_reference(float f) {
  const uint32_t x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
  if ((x & 0x8000u) != 0 && (x & 0x17fffu) != 0) return (uint16_t)((x >> 16) + 1u);
  return (uint16_t)(x >> 16);
}

__global__ __launch_bounds__(256) void bf16_exhaustive_kernel(uint32_t hi, unsigned long long* count) {
  const uint32_t x = (hi << 24) | (blockIdx.x * 256u + threadIdx.x);
  const float f = __uint_as_float(x);
  const bool bad = bf16_bits(f) != bf16_bits_reference(f);
  const unsigned long long n = __ballot(bad);
  if (n != 0 && (threadIdx.x & 63) == 0) atomicAdd(count, (unsigned long long)__popcll(n));
}

hipError_t launch_bf16_exhaustive(unsigned long long* count, hipStream_t stream) {
  for (uint32_t hi = 0; hi < 256; ++hi) {
    hipLaunchKernelGGL(bf16_exhaustive_kernel, dim3(65536), dim3(256), 0, stream, hi, count);
    if (hipError_t e = hipGetLastError()) return e;
  }
  return hipSuccess;
}

hipError_t launch_selftest(float* out, hipStream_t stream) {
  hipLaunchKernelGGL(selftest_kernel, dim3(1), dim3(64), 0, stream, out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dense bf16 projections of the model around the block: the attention's
// Q/K/V/O projections and lm_head (Kernels::bf16_matvec, gpt-oss-cpu-kernels
// lib.rs:314-341, through project_bf16[_batch] cpu_runner.rs:2689-2792):
// out[r * rows + o] = dot(w[o], x[r]) (+ bias[o]).
//
// dot keeps the reference's 16 reduction lanes (scalar_bf16_dot lib.rs:
// 1007-1029): lane l sums w[k] * x[k] over k = l, l + 16, ... in increasing k,
// from 0.0, each product and each sum rounded to f32 (no fma); the lanes then
// fold as 0.0 + lane 0 + lane 1 + ... + lane 15. x arrives as f32 (the exact
// values of the bf16 inputs).
//
// A work-group is kDenseRows weight rows x 16 lanes: thread tid runs lane
// tid % 16 of row kDenseRows * blockIdx.x + tid / 16 for the TOK rows of x of
// group blockIdx.y. K moves through LDS in chunks of kDenseKc values (a
// multiple of 16, so a lane's elements stay in order), the next chunk's loads
// in flight while the current chunk is summed. At one token the kernel streams
// the weights (lm_head: 201,088 x 2,880 bf16, 1.16 GB per call).
constexpr int kDenseRows = 16;
constexpr int kDenseKc = 256;
constexpr int kDenseWStride = kDenseKc + 8;  // LDS row stride (u16): consecutive rows start 4 banks apart

template <int TOK>
struct DenseChunk {
  static constexpr int kXPieces = (TOK * kDenseKc / 4 + 255) / 256;  // float4 pieces per thread
  u32x4 w[2];  // pieces tid and tid + 256 of the 16 x kDenseKc weight chunk (8 values each)
  float4 x[kXPieces];
};

template <int TOK>
__device__ __forceinline__ void dense_load(DenseChunk<TOK>& c, const uint16_t* w, const float* x, int rows, int cols,
                                           int m, int o0, int r0, int k0, int tid) {
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int p = tid + 256 * q, o = o0 + (p >> 5), k = k0 + (p & 31) * 8;
    if (o < rows && (cols & 7) == 0 && k + 8 <= cols) {
      c.w[q] = *reinterpret_cast<const u32x4*>(w + (size_t)o * cols + k);
    } else {  // ragged edge: values past the matrix read as zero and are never summed
      uint32_t v[4] = {0u, 0u, 0u, 0u};
      for (int e = 0; e < 8; ++e)
        if (o < rows && k + e < cols) v[e >> 1] |= (uint32_t)w[(size_t)o * cols + k + e] << (16 * (e & 1));
      c.w[q] = u32x4{v[0], v[1], v[2], v[3]};
    }
  }
#pragma unroll
  for (int q = 0; q < DenseChunk<TOK>::kXPieces; ++q) {
    const int p = tid + 256 * q, r = r0 + (p >> 6), k = k0 + (p & 63) * 4;
    if (p < TOK * kDenseKc / 4 && r < m && (cols & 3) == 0 && k + 4 <= cols) {
      c.x[q] = *reinterpret_cast<const float4*>(x + (size_t)r * cols + k);
    } else {
      float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int e = 0; e < 4; ++e)
        if (p < TOK * kDenseKc / 4 && r < m && k + e < cols) v[e] = x[(size_t)r * cols + k + e];
      c.x[q] = make_float4(v[0], v[1], v[2], v[3]);
    }
  }
}

// Work-group columns [wg_begin[p], wg_begin[p + 1]) serve projection p of
// `set` (up to three projections of the same input in one launch).
template <int TOK>
__global__ __launch_bounds__(256) void dense_proj_kernel(DenseSet set, const float* __restrict__ x, int cols, int m) {
  static_assert(kDenseRows * 16 == 256 && kDenseKc % 16 == 0 && TOK <= 16, "thread map");
  __shared__ __align__(16) uint16_t s_w[kDenseRows * kDenseWStride];
  __shared__ __align__(16) float s_x[TOK * kDenseKc];  // also the fold buffer: [row][token][lane]
  const int tid = threadIdx.x, i = tid >> 4, l = tid & 15;
  const int b = (int)blockIdx.x;
  const int pi = b >= set.wg_begin[2] ? 2 : (b >= set.wg_begin[1] ? 1 : 0);
  const uint16_t* w = set.w[pi];
  const float* bias = set.bias[pi];
  float* out = set.out[pi];
  const int rows = set.rows[pi];
  const int o0 = (b - set.wg_begin[pi]) * kDenseRows, r0 = blockIdx.y * TOK;
  float acc[TOK];
#pragma unroll
  for (int t = 0; t < TOK; ++t) acc[t] = 0.0f;
  DenseChunk<TOK> c;
  dense_load<TOK>(c, w, x, rows, cols, m, o0, r0, 0, tid);
  for (int k0 = 0; k0 < cols; k0 += kDenseKc) {
    __syncthreads();  // every lane has summed the previous chunk
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int p = tid + 256 * q;
      *reinterpret_cast<u32x4*>(&s_w[(p >> 5) * kDenseWStride + (p & 31) * 8]) = c.w[q];
    }
#pragma unroll
    for (int q = 0; q < DenseChunk<TOK>::kXPieces; ++q) {
      const int p = tid + 256 * q;
      if (p < TOK * kDenseKc / 4) *reinterpret_cast<float4*>(&s_x[(p >> 6) * kDenseKc + (p & 63) * 4]) = c.x[q];
    }
    __syncthreads();
    if (k0 + kDenseKc < cols) dense_load<TOK>(c, w, x, rows, cols, m, o0, r0, k0 + kDenseKc, tid);
    const int kc = min(kDenseKc, cols - k0);
#pragma unroll 4
    for (int j = 0; j < kDenseKc / 16; ++j) {
      const int k = j * 16 + l;
      if (k < kc) {
        const float wv = __uint_as_float((uint32_t)s_w[i * kDenseWStride + k] << 16);
#pragma unroll
        for (int t = 0; t < TOK; ++t) acc[t] = acc[t] + wv * s_x[t * kDenseKc + k];
      }
    }
  }
  // The 16 lanes of each (row, token) fold in lane order, from 0.0.
  __syncthreads();
#pragma unroll
  for (int t = 0; t < TOK; ++t) s_x[(i * TOK + t) * 16 + l] = acc[t];
  __syncthreads();
  if (tid < kDenseRows * TOK) {
    const int fi = tid % kDenseRows, ft = tid / kDenseRows;  // consecutive threads: consecutive outputs
    const int o = o0 + fi, r = r0 + ft;
    if (o < rows && r < m) {
      const float* v = &s_x[(fi * TOK + ft) * 16];
      float s = 0.0f;
#pragma unroll
      for (int q = 0; q < 16; ++q) s = s + v[q];
      if (bias != nullptr) s = s + bias[o];
      out[(size_t)r * rows + o] = s;
    }
  }
}

// One token, up to three projections of the same input in one launch (Q, K
// and V): the same dot, with the work-group's 16 weight rows for the whole K
// range staged in LDS by loads that are all in flight at once, so the
// work-group waits for one memory round trip instead of one per K chunk.
// Work-groups [wg_begin[i], wg_begin[i + 1]) serve projection i. cols is a
// multiple of 8 and at most kDenseGemvMaxCols.
constexpr int kDenseGemvMaxCols = 4096;
constexpr int kDenseGemvPieces = kDenseRows * kDenseGemvMaxCols / 8 / 256;  // 16-byte weight pieces per thread

__global__ __launch_bounds__(256) void dense_gemv_kernel(DenseSet set, const float* __restrict__ x, int cols) {
  extern __shared__ __align__(16) char s_dyn[];
  __shared__ float s_fold[kDenseRows * 16];
  const int stride = cols + 8;  // u16 per LDS row
  uint16_t* s_w = reinterpret_cast<uint16_t*>(s_dyn);
  float* s_x = reinterpret_cast<float*>(s_dyn + (size_t)kDenseRows * stride * 2);
  const int tid = threadIdx.x, i = tid >> 4, l = tid & 15;
  const int b = (int)blockIdx.x;
  const int pi = b >= set.wg_begin[2] ? 2 : (b >= set.wg_begin[1] ? 1 : 0);
  const uint16_t* w = set.w[pi];
  const int rows = set.rows[pi], o0 = (b - set.wg_begin[pi]) * kDenseRows;
  const int per_row = cols >> 3, n_w = kDenseRows * per_row;
  u32x4 v[kDenseGemvPieces];
#pragma unroll
  for (int q = 0; q < kDenseGemvPieces; ++q) {
    const int p = tid + 256 * q;
    const int r = p / per_row, k = (p - r * per_row) * 8;
    v[q] = u32x4{0u, 0u, 0u, 0u};
    if (p < n_w && o0 + r < rows) v[q] = *reinterpret_cast<const u32x4*>(w + (size_t)(o0 + r) * cols + k);
  }
  float4 xv[kDenseGemvMaxCols / 4 / 256];
#pragma unroll
  for (int q = 0; q < kDenseGemvMaxCols / 4 / 256; ++q) {
    const int p = tid + 256 * q;
    xv[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (p * 4 < cols) xv[q] = *reinterpret_cast<const float4*>(x + p * 4);
  }
#pragma unroll
  for (int q = 0; q < kDenseGemvPieces; ++q) {
    const int p = tid + 256 * q;
    const int r = p / per_row, k = (p - r * per_row) * 8;
    if (p < n_w) *reinterpret_cast<u32x4*>(&s_w[r * stride + k]) = v[q];
  }
#pragma unroll
  for (int q = 0; q < kDenseGemvMaxCols / 4 / 256; ++q) {
    const int p = tid + 256 * q;
    if (p * 4 < cols) *reinterpret_cast<float4*>(&s_x[p * 4]) = xv[q];
  }
  __syncthreads();
  float acc = 0.0f;
  const uint16_t* wr = &s_w[i * stride];
#pragma unroll 8
  for (int k = l; k < cols; k += 16) acc = acc + __uint_as_float((uint32_t)wr[k] << 16) * s_x[k];
  s_fold[i * 16 + l] = acc;
  __syncthreads();
  if (tid < kDenseRows && o0 + tid < rows) {
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 16; ++q) s = s + s_fold[tid * 16 + q];
    if (set.bias[pi] != nullptr) s = s + set.bias[pi][o0 + tid];
    set.out[pi][o0 + tid] = s;
  }
}

size_t dense_gemv_lds(int cols) { return (size_t)kDenseRows * (cols + 8) * 2 + (size_t)cols * 4; }

hipError_t launch_dense_gemv(const DenseSet& set, int count, const float* x, int cols, hipStream_t stream) {
  if (count <= 0 || count > 3 || cols <= 0 || cols % 8 != 0 || cols > kDenseGemvMaxCols) return hipErrorInvalidValue;
  DenseSet s = set;
  int wg = 0;
  for (int i = 0; i < 3; ++i) {
    s.wg_begin[i] = wg;
    if (i < count) wg += (s.rows[i] + kDenseRows - 1) / kDenseRows;
  }
  s.wg_begin[3] = wg;
  if (wg == 0) return hipSuccess;
  hipLaunchKernelGGL(dense_gemv_kernel, dim3((unsigned)wg), dim3(256), (unsigned)dense_gemv_lds(cols), stream, s, x,
                     cols);
  return hipGetLastError();
}

// The attention half's residual add (add_residual, cpu_runner.rs:3732-3738,
// after the O projection's bf16 round trip): after = bf16(hidden + bf16(proj)).
__global__ __launch_bounds__(256) void residual_add_kernel(const uint16_t* __restrict__ hidden,
                                                           const float* __restrict__ proj, uint16_t* __restrict__ after,
                                                           size_t n) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) after[i] = bf16_bits(bf16_to_f32(hidden[i]) + bf16r(proj[i]));
}

hipError_t launch_residual_add(const uint16_t* hidden, const float* proj, uint16_t* after, size_t n,
                               hipStream_t stream) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(residual_add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, hidden, proj, after,
                     n);
  return hipGetLastError();
}

hipError_t launch_dense_proj(const DenseSet& set, int count, const float* x, int cols, int m, hipStream_t stream) {
  if (count <= 0 || count > 3 || cols <= 0 || m <= 0) return hipErrorInvalidValue;
  DenseSet s = set;
  int wg = 0;
  for (int i = 0; i < 3; ++i) {
    s.wg_begin[i] = wg;
    if (i < count) wg += (s.rows[i] + kDenseRows - 1) / kDenseRows;
  }
  s.wg_begin[3] = wg;
  if (wg == 0) return hipSuccess;
  if (m == 1)
    hipLaunchKernelGGL(dense_proj_kernel<1>, dim3((unsigned)wg, 1), dim3(256), 0, stream, s, x, cols, m);
  else if (m <= 4)
    hipLaunchKernelGGL(dense_proj_kernel<4>, dim3((unsigned)wg, 1), dim3(256), 0, stream, s, x, cols, m);
  else
    hipLaunchKernelGGL(dense_proj_kernel<16>, dim3((unsigned)wg, (unsigned)((m + 15) / 16)), dim3(256), 0, stream, s,
                       x, cols, m);
  return hipGetLastError();
}

}  // namespace gossmx
