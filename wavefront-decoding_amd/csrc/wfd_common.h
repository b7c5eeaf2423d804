// Shared device helpers for the wavefront-decode kernels (gfx950 / CDNA4).
//
// Storage types: fp32 tensors are `float`, bf16 tensors are `bf16_t` (raw
// 16-bit pattern). All arithmetic is fp32; bf16 results are rounded once,
// round-to-nearest-even, which is the rounding torch uses for bf16 tensors.
//
// Every kernel in this library is row-invariant: the value written for a row
// depends only on that row's inputs (and the weights), never on how many other
// rows share the launch or where the row sits in it. This is what keeps the
// wavefront decode (W rows per tick) bit-identical to sequential looped decode
// (1 row per tick) -- the losslessness argument of
// src/decoding/parcae_blocks.py:526-597 needs identical per-token arithmetic.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "wfd.h"

namespace wfd {

struct bf16_t {
  uint16_t bits;
};

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

enum DType : int { kF32 = 0, kBF16 = 1 };

enum Status : int {
  kOk = 0,
  kBadArg = -1,
  kUnsupported = -2,
  kLaunch = -3,
  kWorkspace = -4,
};

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// fp32 -> bf16, round to nearest even, NaN kept quiet: one v_cvt_pk_bf16_f32
// per pair on gfx950 (checked on the device against the bit-level RNE
// formula over 2^26 patterns, ties, denormals and specials included: no
// difference).
__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) { return (uint16_t)f32x2_to_bf16x2_bits(f, 0.f); }

template <typename T>
struct Elem;

template <>
struct Elem<float> {
  static constexpr int kVec = 4;  // elements per 16-byte vector
  __device__ __forceinline__ static float load(const float* p) { return *p; }
  __device__ __forceinline__ static void store(float* p, float v) { *p = v; }
  __device__ __forceinline__ static float round(float v) { return v; }
  __device__ __forceinline__ static void unpack(const u32x4& w, float (&o)[4]) {
    o[0] = __uint_as_float(w[0]);
    o[1] = __uint_as_float(w[1]);
    o[2] = __uint_as_float(w[2]);
    o[3] = __uint_as_float(w[3]);
  }
  __device__ __forceinline__ static u32x4 pack(const float (&o)[4]) {
    u32x4 w = {__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]), __float_as_uint(o[3])};
    return w;
  }
  __device__ __forceinline__ static u32x4 pack_ones() { return u32x4{0x3f800000u, 0x3f800000u, 0x3f800000u, 0x3f800000u}; }
};

template <>
struct Elem<bf16_t> {
  static constexpr int kVec = 8;
  __device__ __forceinline__ static float load(const bf16_t* p) { return bf16_bits_to_f32(p->bits); }
  __device__ __forceinline__ static void store(bf16_t* p, float v) { p->bits = f32_to_bf16_bits(v); }
  // the value a store then a load would give back
  __device__ __forceinline__ static float round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }
  __device__ __forceinline__ static void unpack(const u32x4& w, float (&o)[8]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[2 * e] = __uint_as_float(w[e] << 16);
      o[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static u32x4 pack(const float (&o)[8]) {
    u32x4 w;
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = f32x2_to_bf16x2_bits(o[2 * e], o[2 * e + 1]);
    return w;
  }
  __device__ __forceinline__ static u32x4 pack_ones() { return u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u}; }
};

__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }

// Raw buffer view of a small operand (< 2 GiB): a load at an offset at or past
// kBufInvalid reads zeros and sends no request to memory, so lanes that carry
// padding rows cost no bandwidth and need no branch.
constexpr uint32_t kBufInvalid = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}

__device__ __forceinline__ u32x4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0));
}

__device__ __forceinline__ u32x4 zero16() {
  u32x4 z = {0u, 0u, 0u, 0u};
  return z;
}

// Element offset of (cache row, kv head) in a KV slot cache.
//   block_rows <= 1: token-major (rows, Hkv, Dh), one row = all heads of a token;
//   block_rows  > 1: head-major blocks (rows / block_rows, Hkv, block_rows, Dh),
//                    so one head's rows of a block are contiguous.
// 32-bit division whenever the operands fit (every realistic cache).
__device__ __forceinline__ int64_t kv_offset(int64_t row, int head, int Hkv, int Dh, int64_t block_rows) {
  if (block_rows <= 1) return (row * Hkv + head) * Dh;
  int64_t blk;
  if (((uint64_t)row | (uint64_t)block_rows) >> 32 == 0)
    blk = (uint32_t)row / (uint32_t)block_rows;
  else
    blk = row / block_rows;
  return ((blk * Hkv + head) * block_rows + (row - blk * block_rows)) * Dh;
}

// One MFMA "k-step": acc(16x16) += A(16 x KSTEP) * B(KSTEP x 16), where each
// lane supplies one 16-byte fragment of A (row lane%16) and of B (column
// lane%16), both covering k-group lane/16. KSTEP = 4 * kVec: 32 for bf16
// (v_mfma_f32_16x16x32_bf16), 16 for fp32 (four v_mfma_f32_16x16x4_f32, one
// per element of the fragment). A and B use the same k mapping, so the
// product is a true dot product whatever the hardware's internal k order.
// Output layout: lane l holds D[4*(l/16) + r][l%16], r = 0..3.
template <typename T>
__device__ __forceinline__ f32x4 mfma_step(const u32x4& a, const u32x4& b, f32x4 acc);

template <>
__device__ __forceinline__ f32x4 mfma_step<bf16_t>(const u32x4& a, const u32x4& b, f32x4 acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc,
                                                 0, 0, 0);
}

template <>
__device__ __forceinline__ f32x4 mfma_step<float>(const u32x4& a, const u32x4& b, f32x4 acc) {
#pragma unroll
  for (int e = 0; e < 4; ++e)
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[e]), __uint_as_float(b[e]), acc, 0, 0, 0);
  return acc;
}

// K is consumed in chunks of kChunkSteps MFMA k-steps: KC = 128 bf16 / 64
// fp32 elements. Lane group j (= lane / 16) of a wave holds, for step s of a
// chunk, the V elements at chunk*KC + s*KSTEP + j*V.
constexpr int kChunkSteps = 4;

template <typename T>
struct Chunk {
  static constexpr int V = Elem<T>::kVec;
  static constexpr int KSTEP = 4 * V;             // k elements per MFMA step
  static constexpr int KC = KSTEP * kChunkSteps;  // k elements per chunk
};

// Sum of squares of one chunk of a row, held as above by the four lanes
// l, l^16, l^32, l^48: g_j = sequential fma over (s, e) of lane group j, then
// (g0 + g1) + (g2 + g3). A row's sum of squares is ((0 + cp_0) + cp_1) + ...
// over its chunks in order: the RMSNorm kernel reduces in exactly this order,
// the order of the linear layer's K chunks, so a norm fused into a linear
// operand load can reproduce it bit for bit.
template <int V>
__device__ __forceinline__ float chunk_sumsq(const float (&v)[kChunkSteps][V]) {
  float g = 0.f;
#pragma unroll
  for (int s = 0; s < kChunkSteps; ++s)
#pragma unroll
    for (int e = 0; e < V; ++e) g = fmaf(v[s][e], v[s][e], g);
  g += __shfl_xor(g, 16, 64);
  g += __shfl_xor(g, 32, 64);
  return g;
}

__device__ __forceinline__ float rms_inv(float sumsq, int D, float eps) {
  return 1.0f / sqrtf(sumsq / (float)D + eps);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// ---------------------------------------------------------------------------
// Folded RMSNorm pairs (wfd_prep_t in wfd.h). Every product and sum below is
// rounded on its own (contraction off), so the kernels that form these values
// -- a linear's epilogue, the one-wave-per-row norm kernel -- agree bit for
// bit whatever the compiler would fuse elsewhere.

// One element of the residual stream and of the next linear's operand: y the
// linear's fp32 output; with a residual, x = round((r_in * s_in) * w_in)
// (s_in = w_in = 1 for a residual without a norm) and r = round(round(y) + x);
// u = r * wa (wa = 1: norm a absent), A = round(u * wb). Also r^2 and u^2.
struct PrepVal {
  float r, A, sr, su;
};
template <typename T>
__device__ __forceinline__ PrepVal prep_value(float y, bool res, float r_in, float s_in, float w_in, float wa,
                                              float wb) {
#pragma clang fp contract(off)
  PrepVal o;
  const float a = Elem<T>::round(y);
  o.r = a;
  if (res) {
    const float x = Elem<T>::round((r_in * s_in) * w_in);
    o.r = Elem<T>::round(a + x);
  }
  const float u = o.r * wa;
  o.A = Elem<T>::round(u * wb);
  o.sr = o.r * o.r;
  o.su = u * u;
  return o;
}

// The block's last norm of r: round((r * s) * w).
template <typename T>
__device__ __forceinline__ float norm_value(float r, float s, float w) {
#pragma clang fp contract(off)
  return Elem<T>::round((r * s) * w);
}

// ((v0+v1)+(v2+v3)): one half of an 8-column group's tree
__device__ __forceinline__ float tree4(float v0, float v1, float v2, float v3) {
#pragma clang fp contract(off)
  return (v0 + v1) + (v2 + v3);
}

__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// Where a row's group sums sit, and the order they are added in. A row (at
// most one round of 16 chunks: 2048 bf16 / 1024 fp32 values) held by one
// wave in the chunk layout gives lane L = c + 16 j, at step s, the elements
// of chunk c at s KSTEP + j V: bf16, all of group 16 c + 4 s + j; fp32, half
// of group 8 c + 2 s + j / 2 (the other half in lane L ^ 16). The sums of
// that group are stored at slot 4 (c + 16 j) + s of the row's 256 slots (for
// fp32 from the even j), so lane L finds its four groups, in step order, at
// slots 4 L .. 4 L + 3. The row's sums: each lane adds its groups in step
// order from +0 (lanes with no group, past the row or fp32's odd j, add
// nothing), then the lanes' butterfly (xor 32, 16, ..., 1: every lane ends
// with the same bits, each step adding the same two values in either order).
constexpr int kFoldSlots = 256;  // per row

template <typename T>
__host__ __device__ constexpr int fold_max_d() {
  return 16 * Chunk<T>::KC;
}

// slot of 8-column group g
template <typename T>
__device__ __forceinline__ int fold_slot(int g) {
  if constexpr (Chunk<T>::V == 8) return 4 * ((g >> 4) + 16 * (g & 3)) + ((g >> 2) & 3);
  return 4 * ((g >> 3) + 32 * (g & 1)) + ((g >> 1) & 3);
}

// lane `lane` of a wave holds groups of this row (P chunks)?
template <typename T>
__device__ __forceinline__ bool fold_lane_live(int lane, int P) {
  return (lane & 15) < P && (Chunk<T>::V == 8 || ((lane >> 4) & 1) == 0);
}

__device__ __forceinline__ void fold_sums(const float (&gr)[kChunkSteps], const float (&gu)[kChunkSteps], float& sr,
                                          float& su) {
#pragma clang fp contract(off)
  sr = 0.f;
  su = 0.f;
#pragma unroll
  for (int t = 0; t < kChunkSteps; ++t) {
    sr = sr + gr[t];
    su = su + gu[t];
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    sr = sr + __shfl_xor(sr, m, 64);
    su = su + __shfl_xor(su, m, 64);
  }
}

// A consumer's copy of lane `lane`'s four groups of a row (zeros where the
// lane holds none): two 16-byte loads of slots 4 lane .. 4 lane + 3.
template <typename T>
__device__ __forceinline__ void fold_load(float4 (&gpv)[2], const float2* row_slots, int lane, int P) {
  const float4* g4 = reinterpret_cast<const float4*>(row_slots) + 2 * lane;
  const bool live = fold_lane_live<T>(lane, P);
  gpv[0] = live ? g4[0] : float4{0.f, 0.f, 0.f, 0.f};
  gpv[1] = live ? g4[1] : float4{0.f, 0.f, 0.f, 0.f};
}

__device__ __forceinline__ void fold_sums4(const float4 (&gpv)[2], float& sr, float& su) {
  const float gr[kChunkSteps] = {gpv[0].x, gpv[0].z, gpv[1].x, gpv[1].z};
  const float gu[kChunkSteps] = {gpv[0].y, gpv[0].w, gpv[1].y, gpv[1].w};
  fold_sums(gr, gu, sr, su);
}

// s_a and the linear's row scale s_a * s_b from the two sums.
__device__ __forceinline__ void pair_scale(float sr, float su, int D, float eps, bool two, float& s_a,
                                           float& scale) {
#pragma clang fp contract(off)
  s_a = two ? 1.0f / sqrtf(sr / (float)D + eps) : 1.0f;
  const float s_b = 1.0f / sqrtf(((s_a * s_a) * su) / (float)D + eps);
  scale = s_a * s_b;
}

__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}

}  // namespace wfd

// Host-side error reporting shared by every C-ABI entry point.
namespace wfd {
void set_error(const char* fmt, ...);
int launch_status(const char* what);

// Greedy argmax step: (ov, oi) replaces (bv, bi) if it ranks higher, or ranks
// the same with a lower index. NaN ranks above every number, as in
// torch.argmax, so a row holding a NaN yields its first NaN's index. The rank
// is a total order on (value, index), so merging in any order and grouping
// gives the same id: the first index of the largest value.
__device__ __forceinline__ void argmax_merge(float& bv, int& bi, float ov, int oi) {
  const bool onan = ov != ov, bnan = bv != bv;
  const bool take = onan ? (!bnan || oi < bi) : (!bnan && (ov > bv || (ov == bv && oi < bi)));
  if (take) {
    bv = ov;
    bi = oi;
  }
}

}  // namespace wfd
