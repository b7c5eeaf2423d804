// Row-invariant skinny linear layer: y[m, :] = x[m, :] @ W^T on MFMA.
//
// Replaces the nn.Linear calls of the block forwards (Wqkv, proj, the gated
// MLP, the adapter, lm_head; src/decoding/huginn_blocks.py:79,100-102,216,291
// and huginn_blocks_batch.py:149,160-161,299,345). At decode M = n is 1..~512
// rows while W is 4-128 MB, so the layer is a weight stream: each weight byte
// is read from HBM once per launch.
//
// Arithmetic contract (depends on K and the dtype only, never on n or on how
// the work is split): K is cut into P = K / KC chunks of 4 MFMA k-steps
// (KC = 128 bf16 / 64 fp32 elements); a chunk partial is the MFMA chain over
// its 4 steps starting from zero; y = epilogue(((0 + c_0) + c_1) + ... + c_{P-1})
// in fp32. Two kernels honour it bit for bit:
//
//  * wide (n <= 16): one 1024-thread workgroup per 16-column tile; its 16
//    waves take the chunks round-robin (all loads of a wave issued together),
//    park the chunk partials in LDS, and threads sum them in chunk order.
//    No cross-workgroup synchronization: the column tile's whole K is reduced
//    inside one workgroup.
//  * tile (n > 16): a workgroup owns 64 rows x 32 columns; each of its 4 waves
//    walks the chunks in order for one 16-row tile and two column tiles, with
//    a two-stage register pipeline (chunk p+1 in flight while chunk p runs on
//    MFMA). The waves of a workgroup read the same weight fragments, so the
//    weights stream from HBM once per 64 rows.
//
// So y[m] is bit-identical whatever n is and wherever row m sits -- the
// property that keeps wavefront decode token-identical to sequential decode.
//
// Epilogues: plain store (bf16 or fp32 out); SwiGLU, where tile 0 is the
// gate feature block and tile 1 the matching up block `pair_off` rows below
// it: out = silu(gate) * up; and QKV-RoPE-append, for the fused q|k|v
// projection: the output row is rounded to the element type, q and k heads are
// rotated by the row's position (interleaved pairs: columns 2j and 2j+1 sit in
// one 16-column tile, so the partner value is one lane shuffle away), q goes to
// q_out and k, v are written straight into the slot cache row flat_row[m]
// (src/decoding/huginn_blocks.py:77-87 + kv_cache.py:97-104 fused into the
// projection; the separate qkv_rope_append pass and its qkv round trip vanish).
#include "wfd_common.h"

namespace wfd {

constexpr int kWideWaves = 16;
constexpr int kWideMaxChunksPerWave = 3;
constexpr int kWideMaxRows = 16;
enum Epilogue : int { kEpiPlain = 0, kEpiSwiGLU = 1, kEpiRope = 2 };


// Operands of the QKV-RoPE-append epilogue (unused by the others).
struct RopeArgs {
  const int32_t* pos;       // [n] positions (clamped into the table)
  const float* cos_t;       // [rows, Dh/2]
  const float* sin_t;       // [rows, Dh/2]
  int tab_rows;
  const int64_t* flat_row;  // [n] slot-cache row of each token
  void* q_out;              // [n, H, Dh]
  void* k_cache;            // [rows, Hkv, Dh]
  void* v_cache;
  int H, Hkv, Dh;
};

template <typename T>
using LinTraits = Chunk<T>;


// Column start of tile t (0..NT-1) of column group g.
template <int NT, int EPI>
__device__ __forceinline__ int tile_col(int g, int t, int pair_off) {
  if (EPI == kEpiSwiGLU) return (t == 0 ? 0 : pair_off) + g * 16;
  return (g * NT + t) * 16;
}

template <typename TO, int EPI>
__device__ __forceinline__ void store_elem(TO* __restrict__ y, int64_t ldy, int row, int col, float v0, float v1) {
  if (EPI == kEpiSwiGLU)
    Elem<TO>::store(y + (int64_t)row * ldy + col, (v0 / (1.0f + expf(-v0))) * v1);
  else
    Elem<TO>::store(y + (int64_t)row * ldy + col, v0);
}

// Value v0 of output (row, col) and its RoPE partner v1 = value of column col ^ 1.
template <typename TO>
__device__ __forceinline__ void store_rope(const RopeArgs& ra, int row, int col, float v0, float v1) {
  const int head = col / ra.Dh;
  const int d = col - head * ra.Dh;
  TO* dst;
  float out;
  if (head >= ra.H + ra.Hkv) {
    dst = (TO*)ra.v_cache + ra.flat_row[row] * (int64_t)(ra.Hkv * ra.Dh) + (head - ra.H - ra.Hkv) * ra.Dh + d;
    out = v0;
  } else {
    int p = ra.pos[row];
    p = p < 0 ? 0 : (p >= ra.tab_rows ? ra.tab_rows - 1 : p);
    const int half = ra.Dh >> 1;
    const float c = ra.cos_t[(int64_t)p * half + (d >> 1)];
    const float s = ra.sin_t[(int64_t)p * half + (d >> 1)];
    const float xm = Elem<TO>::round(v0);
    const float xp = Elem<TO>::round(v1);
    out = (d & 1) ? fmaf(xp, s, xm * c) : fmaf(xm, c, -(xp * s));
    dst = head < ra.H ? (TO*)ra.q_out + ((int64_t)row * ra.H + head) * ra.Dh + d
                      : (TO*)ra.k_cache + ra.flat_row[row] * (int64_t)(ra.Hkv * ra.Dh) + (head - ra.H) * ra.Dh + d;
  }
  Elem<TO>::store(dst, out);
}

template <typename T, int NT>
__device__ __forceinline__ void load_w(u32x4 (&wf)[NT][kChunkSteps], const T* const (&wrow)[NT], int p) {
  constexpr int KSTEP = LinTraits<T>::KSTEP;
#pragma unroll
  for (int s = 0; s < kChunkSteps; ++s)
#pragma unroll
    for (int t = 0; t < NT; ++t) wf[t][s] = ld16(wrow[t] + (int64_t)(p * kChunkSteps + s) * KSTEP);
}

template <typename T>
__device__ __forceinline__ void load_x(u32x4 (&xf)[kChunkSteps], const T* xp, int p) {
  constexpr int KSTEP = LinTraits<T>::KSTEP;
#pragma unroll
  for (int s = 0; s < kChunkSteps; ++s) xf[s] = ld16(xp + (int64_t)(p * kChunkSteps + s) * KSTEP);
}

// Operand row of lane `col` in the 16-row tile starting at `base` (uniform
// over the wave): x_rows[base + col], read with uniform scalar loads, so the
// vector-memory counter tracks operand data only and no weight load waits for
// an index. Lanes at or past n take the tile's first row: every load stays in
// range and straight-line (a divergent guarded load costs a wait at the join),
// and their results are never stored -- MFMA rows never mix.
__device__ __forceinline__ int tile_row(const int32_t* __restrict__ x_rows, int base, int col, int n) {
  const int m = n - base < 16 ? n - base : 16;
  if (!x_rows) return base + (col < m ? col : 0);
  int r = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int v = x_rows[base + (j < m ? j : 0)];
    r = col == j ? v : r;
  }
  return r;
}

template <typename T, int NT>
__device__ __forceinline__ void chunk_mma(f32x4 (&acc)[NT], const u32x4 (&xf)[kChunkSteps],
                                          const u32x4 (&wf)[NT][kChunkSteps]) {
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < kChunkSteps; ++s)
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = mfma_step<T>(xf[s], wf[t][s], acc[t]);
}

// ---------------------------------------------------------------------------
// wide: grid (groups), 1024 threads; NT = 2 only for SwiGLU (gate + up tiles).
template <typename T, typename TO, int NT, int EPI, int MC>
__global__ __launch_bounds__(64 * kWideWaves) void linear_wide_kernel(
    const T* __restrict__ x, const int32_t* __restrict__ x_rows, int64_t ldx, const T* __restrict__ W,
    TO* __restrict__ y, int64_t ldy, int n, int K, int pair_off, const RopeArgs ra) {
  extern __shared__ f32x4 red[];  // [P][NT][64 lanes]
  constexpr int V = LinTraits<T>::V;
  const int P = K / LinTraits<T>::KC;
  const int g = blockIdx.x;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;

  const int xr = tile_row(x_rows, 0, col, n);
  const T* wrow[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) wrow[t] = W + (int64_t)(tile_col<NT, EPI>(g, t, pair_off) + col) * K + grp * V;
  const T* xp = x + (int64_t)xr * ldx + grp * V;

  // Every load below is unconditional; a wave past the last chunk re-reads
  // chunk P-1 and discards it.
  u32x4 wf[MC][NT][kChunkSteps];
  u32x4 xf[MC][kChunkSteps];
#pragma unroll
  for (int j = 0; j < MC; ++j) {
    const int p = wave + kWideWaves * j;
    const int pc = p < P ? p : P - 1;
    load_w<T, NT>(wf[j], wrow, pc);
    load_x<T>(xf[j], xp, pc);
  }
#pragma unroll
  for (int j = 0; j < MC; ++j) {
    const int p = wave + kWideWaves * j;
    if (p < P) {
      f32x4 acc[NT];
      chunk_mma<T, NT>(acc, xf[j], wf[j]);
#pragma unroll
      for (int t = 0; t < NT; ++t) red[(p * NT + t) * 64 + lane] = acc[t];
    }
  }
  __syncthreads();

  // threads 0..255: one (lane', r) output each; sum chunk partials in chunk order
  if (threadIdx.x < 256) {
    const int ln = threadIdx.x >> 2;
    const int r = threadIdx.x & 3;
    const int row = 4 * (ln >> 4) + r;
    const float* rf = reinterpret_cast<const float*>(red);
    float v[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) v[t] = 0.f;
    for (int p = 0; p < P; ++p)
#pragma unroll
      for (int t = 0; t < NT; ++t) v[t] += rf[((p * NT + t) * 64 + ln) * 4 + r];
    // column ln ^ 1 lives in thread threadIdx.x ^ 4 (all 256 threads take part)
    const float partner = EPI == kEpiRope ? __shfl_xor(v[0], 4, 64) : 0.f;
    if (row < n) {
      if (EPI == kEpiSwiGLU)
        store_elem<TO, EPI>(y, ldy, row, g * 16 + (ln & 15), v[0], v[NT - 1]);
      else if (EPI == kEpiRope)
        store_rope<TO>(ra, row, g * 16 + (ln & 15), v[0], partner);
      else
        store_elem<TO, EPI>(y, ldy, row, g * 16 + (ln & 15), v[0], 0.f);
    }
  }
}

// ---------------------------------------------------------------------------
// tile: grid (ceil(n/64), ceil(groups/NB)), 256 threads; wave = 16-row tile,
// NB column groups per workgroup.
template <typename T, typename TO, int NT, int EPI, int NB>
__global__ __launch_bounds__(256) void linear_tile_kernel(const T* __restrict__ x, const int32_t* __restrict__ x_rows,
                                                          int64_t ldx, const T* __restrict__ W, TO* __restrict__ y,
                                                          int64_t ldy, int n, int K, int pair_off, int groups,
                                                          const RopeArgs ra) {
  constexpr int V = LinTraits<T>::V;
  constexpr int NC = NB * NT;  // weight tiles per wave
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int row0 = (blockIdx.x * 4 + wave) * 16;
  if (row0 >= n) return;  // no barriers in this kernel
  const int P = K / LinTraits<T>::KC;
  const int xr = tile_row(x_rows, row0, col, n);

  const T* wrow[NC];
  bool gok[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int g = blockIdx.y * NB + b;
    gok[b] = g < groups;
    const int gg = gok[b] ? g : 0;
#pragma unroll
    for (int t = 0; t < NT; ++t) wrow[b * NT + t] = W + (int64_t)(tile_col<NT, EPI>(gg, t, pair_off) + col) * K + grp * V;
  }
  const T* xp = x + (int64_t)xr * ldx + grp * V;

  // two-stage register pipeline; every load is unconditional (the stage past
  // the last chunk re-reads chunk P-1 and is never used)
  f32x4 tot[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) tot[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 wa[NC][kChunkSteps], wb[NC][kChunkSteps], xa[kChunkSteps], xb[kChunkSteps];
  load_w<T, NC>(wa, wrow, 0);
  load_x<T>(xa, xp, 0);
  for (int p = 0; p < P; p += 2) {
    const int p1 = p + 1 < P ? p + 1 : P - 1;
    load_w<T, NC>(wb, wrow, p1);
    load_x<T>(xb, xp, p1);
    f32x4 acc[NC];
    chunk_mma<T, NC>(acc, xa, wa);
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) tot[c][r] += acc[c][r];
    if (p + 1 >= P) break;
    const int p2 = p + 2 < P ? p + 2 : P - 1;
    load_w<T, NC>(wa, wrow, p2);
    load_x<T>(xa, xp, p2);
    chunk_mma<T, NC>(acc, xb, wb);
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) tot[c][r] += acc[c][r];
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (!gok[b]) continue;
    const int g = blockIdx.y * NB + b;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int orow = row0 + 4 * grp + r;
      // column col ^ 1 lives in lane ^ 1 (the whole wave takes part)
      const float partner = EPI == kEpiRope ? __shfl_xor(tot[b * NT][r], 1, 64) : 0.f;
      if (orow >= n) continue;
      if (EPI == kEpiRope)
        store_rope<TO>(ra, orow, g * 16 + col, tot[b * NT][r], partner);
      else if (EPI == kEpiSwiGLU)
        store_elem<TO, EPI>(y, ldy, orow, g * 16 + col, tot[b * NT][r], tot[b * NT + NT - 1][r]);
      else
        store_elem<TO, EPI>(y, ldy, orow, tile_col<NT, EPI>(g, 0, pair_off) + col, tot[b * NT][r], 0.f);
    }
  }
}

template <typename T, typename TO, int NT, int EPI>
static void launch_linear(const void* x, const int32_t* xr, int64_t ldx, const void* W, void* y, int64_t ldy, int n,
                          int N, int K, int pair_off, const RopeArgs& ra, hipStream_t st) {
  const int groups = (EPI == kEpiSwiGLU) ? pair_off / 16 : N / 16;
  const int P = K / LinTraits<T>::KC;
  const size_t lds = (size_t)P * NT * 64 * sizeof(f32x4);
  const int mc = (P + kWideWaves - 1) / kWideWaves;  // chunks per wave
  const bool wide = n <= kWideMaxRows && mc <= kWideMaxChunksPerWave && lds <= 65536 && (NT == 1 || mc == 1);
  if (wide && mc == 1) {
    hipLaunchKernelGGL((linear_wide_kernel<T, TO, NT, EPI, 1>), dim3(groups), dim3(64 * kWideWaves), lds, st,
                       (const T*)x, xr, ldx, (const T*)W, (TO*)y, ldy, n, K, pair_off, ra);
  } else if (wide && mc == 2) {
    hipLaunchKernelGGL((linear_wide_kernel<T, TO, 1, EPI, 2>), dim3(groups), dim3(64 * kWideWaves), lds, st,
                       (const T*)x, xr, ldx, (const T*)W, (TO*)y, ldy, n, K, pair_off, ra);
  } else if (wide) {
    hipLaunchKernelGGL((linear_wide_kernel<T, TO, 1, EPI, 3>), dim3(groups), dim3(64 * kWideWaves), lds, st,
                       (const T*)x, xr, ldx, (const T*)W, (TO*)y, ldy, n, K, pair_off, ra);
  } else {
    constexpr int NB = (NT == 1) ? 2 : 1;
    hipLaunchKernelGGL((linear_tile_kernel<T, TO, NT, EPI, NB>), dim3((n + 63) / 64, (groups + NB - 1) / NB),
                       dim3(256), 0, st, (const T*)x, xr, ldx, (const T*)W, (TO*)y, ldy, n, K, pair_off, groups, ra);
  }
}

}  // namespace wfd

extern "C" {

int wfd_linear_k_multiple(int dtype) {
  using namespace wfd;
  return dtype == kBF16 ? LinTraits<bf16_t>::KC : LinTraits<float>::KC;
}

int wfd_linear(const void* x, const int32_t* x_rows, int64_t ldx, const void* W, void* y, int64_t ldy, int n, int N,
               int K, int dtype, int out_dtype, int epilogue, int pair_off, hipStream_t stream) {
  using namespace wfd;
  if (n < 0 || N <= 0 || K <= 0 || ldx < K) {
    set_error("wfd_linear: bad shape n=%d N=%d K=%d ldx=%lld", n, N, K, (long long)ldx);
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!x || !W || !y) {
    set_error("wfd_linear: null pointer argument");
    return kBadArg;
  }
  const int kmul = wfd_linear_k_multiple(dtype);
  if (K % kmul != 0 || N % 16 != 0) {
    set_error("wfd_linear: K=%d must be a multiple of %d and N=%d of 16", K, kmul, N);
    return kUnsupported;
  }
  if (epilogue == kEpiSwiGLU) {
    if (pair_off <= 0 || pair_off % 16 != 0 || N != 2 * pair_off || ldy < pair_off) {
      set_error("wfd_linear: swiglu needs N == 2*pair_off, pair_off %% 16 == 0 (N=%d pair_off=%d)", N, pair_off);
      return kBadArg;
    }
  } else if (epilogue == kEpiPlain) {
    if (ldy < N) {
      set_error("wfd_linear: ldy=%lld < N=%d", (long long)ldy, N);
      return kBadArg;
    }
  } else {
    set_error("wfd_linear: unknown epilogue %d", epilogue);
    return kUnsupported;
  }
  const RopeArgs ra{};
  if (dtype == kBF16 && out_dtype == kBF16) {
    if (epilogue == kEpiSwiGLU)
      launch_linear<bf16_t, bf16_t, 2, kEpiSwiGLU>(x, x_rows, ldx, W, y, ldy, n, N, K, pair_off, ra, stream);
    else
      launch_linear<bf16_t, bf16_t, 1, kEpiPlain>(x, x_rows, ldx, W, y, ldy, n, N, K, 0, ra, stream);
  } else if (dtype == kBF16 && out_dtype == kF32 && epilogue == kEpiPlain) {
    launch_linear<bf16_t, float, 1, kEpiPlain>(x, x_rows, ldx, W, y, ldy, n, N, K, 0, ra, stream);
  } else if (dtype == kF32 && out_dtype == kF32) {
    if (epilogue == kEpiSwiGLU)
      launch_linear<float, float, 2, kEpiSwiGLU>(x, x_rows, ldx, W, y, ldy, n, N, K, pair_off, ra, stream);
    else
      launch_linear<float, float, 1, kEpiPlain>(x, x_rows, ldx, W, y, ldy, n, N, K, 0, ra, stream);
  } else {
    set_error("wfd_linear: unsupported dtype=%d out_dtype=%d epilogue=%d", dtype, out_dtype, epilogue);
    return kUnsupported;
  }
  return launch_status("wfd_linear");
}

int wfd_linear_qkv_rope_append(const void* x, const int32_t* x_rows, int64_t ldx, const void* Wqkv, int n, int K,
                               const int32_t* pos, const float* rope_cos, const float* rope_sin, int rope_rows,
                               const int64_t* flat_row, void* q_out, void* k_cache, void* v_cache, int H, int Hkv,
                               int Dh, int dtype, hipStream_t stream) {
  using namespace wfd;
  if (n < 0 || K <= 0 || ldx < K || H <= 0 || Hkv <= 0 || H % Hkv != 0 || Dh <= 0 || Dh % 16 != 0 ||
      rope_rows <= 0) {
    set_error("wfd_linear_qkv_rope_append: bad shape n=%d K=%d H=%d Hkv=%d Dh=%d rope_rows=%d", n, K, H, Hkv, Dh,
              rope_rows);
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!x || !Wqkv || !pos || !rope_cos || !rope_sin || !flat_row || !q_out || !k_cache || !v_cache) {
    set_error("wfd_linear_qkv_rope_append: null pointer argument");
    return kBadArg;
  }
  const int kmul = wfd_linear_k_multiple(dtype);
  if (K % kmul != 0) {
    set_error("wfd_linear_qkv_rope_append: K=%d must be a multiple of %d", K, kmul);
    return kUnsupported;
  }
  const int N = (H + 2 * Hkv) * Dh;
  const RopeArgs ra{pos, rope_cos, rope_sin, rope_rows, flat_row, q_out, k_cache, v_cache, H, Hkv, Dh};
  if (dtype == kBF16)
    launch_linear<bf16_t, bf16_t, 1, kEpiRope>(x, x_rows, ldx, Wqkv, nullptr, 0, n, N, K, 0, ra, stream);
  else if (dtype == kF32)
    launch_linear<float, float, 1, kEpiRope>(x, x_rows, ldx, Wqkv, nullptr, 0, n, N, K, 0, ra, stream);
  else {
    set_error("wfd_linear_qkv_rope_append: unsupported dtype=%d", dtype);
    return kUnsupported;
  }
  return launch_status("wfd_linear_qkv_rope_append");
}

}  // extern "C"
