// Row-wise fused pieces of the recurrent-block forward and the slot-cache
// append, plus the small gathers the decode tick needs.
//
//  * add_rmsnorm: x' = rmsnorm(a + res) * w1, optionally h = rmsnorm(x') * w2.
//    The sandwich block's `norm_2(att + x)` followed by `norm_3(x)`, and
//    `norm_4(mlp + x)` followed by the next block's `norm_1`
//    (src/decoding/huginn_blocks.py:100-102, huginn_blocks_batch.py:159-161),
//    in one pass; with res == nullptr it is a plain RMSNorm (ln_f, norm_1).
//  * qkv_rope_append: split the fused QKV row, rotate q and k by the
//    position's RoPE angles (interleaved pairs), write q out and append k, v
//    to the slot cache at flat_row[i] (huginn_blocks.py:77-87 + the cache
//    write of kv_cache.py:97-104 / batch_kv_cache.py:61-73 /
//    graph_blocks.py:172-176, fused).
//  * kv_append: the bare slot-cache append (same indexing, no rotation).
//  * embed, copy_rows, argmax: token embedding gather (x emb_scale), row
//    gather/scatter (initial loop state, wave-state pool), greedy argmax
//    (acceptance.py:40-44) on device. argmax can also drop each id into a
//    device token ring and embed can take its ids from there, so a decode
//    loop feeds sampled tokens back without a host round trip.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "wfd_common.h"

namespace wfd {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return kLaunch;
  }
  return kOk;
}

constexpr int kRowThreads = 256;
constexpr int kNormMaxD = 4096;
constexpr int kNormRowsPerCuLaunch = 1024;  // rows from which the norm packs 4 rows per workgroup

// One wave per row, 16-byte vector loads. The row is cut into the linear
// layer's K chunks (KC elements); lane (j = lane / 16, c = lane % 16) holds,
// per round r, chunk p = 16 r + c exactly as an MFMA A-operand lane holds it
// (4 steps x V elements of lane group j), and the sum of squares is reduced in
// the library's one order (chunk_sumsq, then chunks in order). Every load is
// unconditional, and the residual / second-norm variants are compile-time, so
// no load sits behind a data-dependent branch (whose join would wait for it).
//
// Where the row `a` comes from (SRC):
//  * kSrcRows: rows of `a` (a_rows[i] or i).
//  * kSrcSplit: the fp32 slice partials of a split-K linear
//    (wfd_linear_partials: slice q of row i at part + q * slice_stride + i * D),
//    added in slice order from zero -- the linear's arithmetic contract -- and
//    rounded to T as the linear's store would.
//  * kSrcEmbed: the embedding row table[id_i] * scale rounded to T, id_i =
//    ids[i] or, for a negative id with a ring, the device token ring's entry
//    -(id + 1) (wfd_embed's arithmetic); each row's wave also copies row
//    cp_src_rows[i] of cp_src to row cp_dst_rows[i] of cp_dst (cp_width
//    elements; the prelude's initial loop state).
// With a_out the resolved row is stored there (the adapter's output and the
// embedding are their block's residual stream); the rest is the plain
// kernel's math on the same values.
enum : int { kSrcRows = 0, kSrcSplit = 1, kSrcEmbed = 2 };
constexpr int kSplitMaxSlices = 4;  // the linear's K slices (at most 4)

struct SrcArgs {
  const float* part;  // kSrcSplit
  int64_t slice_stride;
  int nslices;
  const int64_t* ids;  // kSrcEmbed
  const int64_t* ring;
  int64_t ring_len;
  const void* table;
  float scale;
  int vocab;
  const void* cp_src;
  const int32_t* cp_src_rows;
  int64_t cp_lds;
  void* cp_dst;
  const int32_t* cp_dst_rows;
  int64_t cp_ldd;
  int cp_width;
  void* a_out;  // kSrcSplit, kSrcEmbed
  int64_t lda_out;
};

template <typename T, bool RES, bool TWO, int MAXR, int SRC>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(
    const T* __restrict__ a, const int32_t* __restrict__ a_rows, int64_t lda, const T* __restrict__ res,
    int64_t ldr, const T* __restrict__ w1, const T* __restrict__ w2, T* __restrict__ x_out,
    const int32_t* __restrict__ out_rows, int64_t ldo, T* __restrict__ h_out, int64_t ldh, int n, int D, float eps,
    const SrcArgs sp) {
  constexpr bool SPLIT = SRC == kSrcSplit;
  constexpr bool KEEP = SRC != kSrcRows;  // a row resolved here, storable to a_out
  constexpr int V = Chunk<T>::V;
  constexpr int KSTEP = Chunk<T>::KSTEP;
  constexpr int KC = Chunk<T>::KC;
  const int i = blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = lane & 15;
  const int j = lane >> 4;
  if (i >= n) return;  // no barriers below
  const int P = D / KC;
  const int64_t ar = SRC == kSrcRows && a_rows ? a_rows[i] : i;
  [[maybe_unused]] const T* erow = nullptr;  // kSrcEmbed: the table row
  if constexpr (SRC == kSrcEmbed) {
    int64_t id = sp.ids[i];
    if (id < 0 && sp.ring) {  // a token handle: the id sits in the device token ring
      const int64_t slot = -id - 1;
      id = slot < sp.ring_len ? sp.ring[slot] : 0;
    }
    id = id < 0 ? 0 : (id >= sp.vocab ? sp.vocab - 1 : id);
    erow = (const T*)sp.table + id * D;
    if (sp.cp_src) {  // the side copy, independent of the row's math
      const int64_t sr = sp.cp_src_rows ? sp.cp_src_rows[i] : i;
      const int64_t dr = sp.cp_dst_rows ? sp.cp_dst_rows[i] : i;
      for (int e = lane * V; e < sp.cp_width; e += 64 * V)
        *reinterpret_cast<u32x4*>((T*)sp.cp_dst + dr * sp.cp_ldd + e) = ld16((const T*)sp.cp_src + sr * sp.cp_lds + e);
    }
  }
  // every load is unconditional: a lane past the last chunk re-reads chunk
  // P-1 (its sum is never used, nothing is stored for it)
  float v[MAXR][kChunkSteps][V];
  u32x4 wa[MAXR][kChunkSteps], wb[MAXR][kChunkSteps];
  [[maybe_unused]] u32x4 wr[KEEP ? MAXR : 1][KEEP ? kChunkSteps : 1];
#pragma unroll
  for (int r = 0; r < MAXR; ++r) {
    const int p = r * 16 + c < P ? r * 16 + c : P - 1;
#pragma unroll
    for (int s = 0; s < kChunkSteps; ++s) {
      const int64_t off = (int64_t)p * KC + s * KSTEP + j * V;
      if constexpr (SPLIT) {
        // branch-free, so every load can be issued before the first add: a
        // slice past nslices re-reads slice 0 and adds +0 in its place (the
        // sum starts at +0 and so is never -0: adding +0 leaves its bits)
        float sum[V];
#pragma unroll
        for (int e = 0; e < V; ++e) sum[e] = 0.f;
#pragma unroll
        for (int q = 0; q < kSplitMaxSlices; ++q) {
          const bool live = q < sp.nslices;
          const float* src = sp.part + (live ? q : 0) * sp.slice_stride + (int64_t)i * D + off;
#pragma unroll
          for (int h = 0; h < V / 4; ++h) {
            const u32x4 w = ld16(src + 4 * h);
#pragma unroll
            for (int e = 0; e < 4; ++e) sum[4 * h + e] += live ? __uint_as_float(w[e]) : 0.f;
          }
        }
#pragma unroll
        for (int e = 0; e < V; ++e) v[r][s][e] = Elem<T>::round(sum[e]);
      } else if constexpr (SRC == kSrcEmbed) {
        Elem<T>::unpack(ld16(erow + off), v[r][s]);
#pragma unroll
        for (int e = 0; e < V; ++e) v[r][s][e] = Elem<T>::round(v[r][s][e] * sp.scale);
      } else {
        Elem<T>::unpack(ld16(a + ar * lda + off), v[r][s]);
      }
      wa[r][s] = ld16(w1 + off);
      if constexpr (TWO) wb[r][s] = ld16(w2 + off);
      if constexpr (RES && KEEP) {
        wr[r][s] = ld16(res + (int64_t)i * ldr + off);  // added after a_out is stored
      } else if constexpr (RES) {
        float q[V];
        Elem<T>::unpack(ld16(res + (int64_t)i * ldr + off), q);
#pragma unroll
        for (int e = 0; e < V; ++e) v[r][s][e] += q[e];
      }
    }
  }
  if constexpr (KEEP) {
    if (sp.a_out) {  // the resolved rows, when the caller keeps them
#pragma unroll
      for (int r = 0; r < MAXR; ++r)
#pragma unroll
        for (int s = 0; s < kChunkSteps; ++s)
          if (r * 16 + c < P)
            *reinterpret_cast<u32x4*>((T*)sp.a_out + (int64_t)i * sp.lda_out + (int64_t)(r * 16 + c) * KC +
                                      s * KSTEP + j * V) = Elem<T>::pack(v[r][s]);
    }
    if constexpr (RES) {
#pragma unroll
      for (int r = 0; r < MAXR; ++r)
#pragma unroll
        for (int s = 0; s < kChunkSteps; ++s) {
          float q[V];
          Elem<T>::unpack(wr[r][s], q);
#pragma unroll
          for (int e = 0; e < V; ++e) v[r][s][e] += q[e];
        }
    }
  }
  // first norm
  float cp[MAXR];
#pragma unroll
  for (int r = 0; r < MAXR; ++r) cp[r] = chunk_sumsq<V>(v[r]);
  float ss = 0.f;
#pragma unroll
  for (int r = 0; r < MAXR; ++r)
    for (int q = 0; q < 16 && r * 16 + q < P; ++q) ss += __shfl(cp[r], q, 64);
  float inv = rms_inv(ss, D, eps);
  const int64_t orow = out_rows ? out_rows[i] : i;
#pragma unroll
  for (int r = 0; r < MAXR; ++r) {
    const int p = r * 16 + c;
#pragma unroll
    for (int s = 0; s < kChunkSteps; ++s) {
      float w[V];
      Elem<T>::unpack(wa[r][s], w);
#pragma unroll
      for (int e = 0; e < V; ++e) v[r][s][e] = v[r][s][e] * inv * w[e];
      const u32x4 pk = Elem<T>::pack(v[r][s]);
      Elem<T>::unpack(pk, v[r][s]);  // continue from the rounded values
      if (x_out && p < P) *reinterpret_cast<u32x4*>(x_out + orow * ldo + (int64_t)p * KC + s * KSTEP + j * V) = pk;
    }
  }
  if constexpr (TWO) {
    // second norm, from the rounded first result (== a separate rmsnorm of x_out)
#pragma unroll
    for (int r = 0; r < MAXR; ++r) cp[r] = chunk_sumsq<V>(v[r]);
    ss = 0.f;
#pragma unroll
    for (int r = 0; r < MAXR; ++r)
      for (int q = 0; q < 16 && r * 16 + q < P; ++q) ss += __shfl(cp[r], q, 64);
    inv = rms_inv(ss, D, eps);
#pragma unroll
    for (int r = 0; r < MAXR; ++r) {
      const int p = r * 16 + c;
#pragma unroll
      for (int s = 0; s < kChunkSteps; ++s) {
        float w[V];
        Elem<T>::unpack(wb[r][s], w);
        float h[V];
#pragma unroll
        for (int e = 0; e < V; ++e) h[e] = v[r][s][e] * inv * w[e];
        if (p < P)
          *reinterpret_cast<u32x4*>(h_out + (int64_t)i * ldh + (int64_t)p * KC + s * KSTEP + j * V) =
              Elem<T>::pack(h);
      }
    }
  }
}

template <typename T, int MAXR, int SRC>
static void launch_norm_r(const void* a, const int32_t* a_rows, int64_t lda, const void* res, int64_t ldr,
                          const void* w1, const void* w2, void* x_out, const int32_t* out_rows, int64_t ldo,
                          void* h_out, int64_t ldh, int n, int D, float eps, const SrcArgs& sp,
                          hipStream_t stream) {
  // one row (wave) per workgroup unless there are rows enough to fill every
  // CU four times over: a CU streams its waves' rows at a bounded rate, so a
  // few hundred rows finish sooner spread one per CU
  const int rpw = n >= kNormRowsPerCuLaunch ? 4 : 1;
  const dim3 grid((n + rpw - 1) / rpw), block(64 * rpw);
  const T *at = (const T*)a, *rt = (const T*)res, *w1t = (const T*)w1, *w2t = (const T*)w2;
  T *xo = (T*)x_out, *ho = (T*)h_out;
  if (res && w2)
    hipLaunchKernelGGL((add_rmsnorm_kernel<T, true, true, MAXR, SRC>), grid, block, 0, stream, at, a_rows, lda, rt,
                       ldr, w1t, w2t, xo, out_rows, ldo, ho, ldh, n, D, eps, sp);
  else if (res)
    hipLaunchKernelGGL((add_rmsnorm_kernel<T, true, false, MAXR, SRC>), grid, block, 0, stream, at, a_rows, lda, rt,
                       ldr, w1t, w2t, xo, out_rows, ldo, ho, ldh, n, D, eps, sp);
  else if (w2)
    hipLaunchKernelGGL((add_rmsnorm_kernel<T, false, true, MAXR, SRC>), grid, block, 0, stream, at, a_rows, lda, rt,
                       ldr, w1t, w2t, xo, out_rows, ldo, ho, ldh, n, D, eps, sp);
  else
    hipLaunchKernelGGL((add_rmsnorm_kernel<T, false, false, MAXR, SRC>), grid, block, 0, stream, at, a_rows, lda, rt,
                       ldr, w1t, w2t, xo, out_rows, ldo, ho, ldh, n, D, eps, sp);
}

// Rounds of 16 chunks per lane: a row of up to 16 chunks needs one (the usual
// d_model), wider rows up to kNormMaxD take the general form.
template <typename T, int SRC>
static void launch_norm_t(const void* a, const int32_t* a_rows, int64_t lda, const void* res, int64_t ldr,
                          const void* w1, const void* w2, void* x_out, const int32_t* out_rows, int64_t ldo,
                          void* h_out, int64_t ldh, int n, int D, float eps, const SrcArgs& sp, hipStream_t stream) {
  if (D <= 16 * Chunk<T>::KC)
    launch_norm_r<T, 1, SRC>(a, a_rows, lda, res, ldr, w1, w2, x_out, out_rows, ldo, h_out, ldh, n, D, eps, sp,
                             stream);
  else
    launch_norm_r<T, kNormMaxD / (16 * Chunk<T>::KC), SRC>(a, a_rows, lda, res, ldr, w1, w2, x_out, out_rows, ldo,
                                                            h_out, ldh, n, D, eps, sp, stream);
}

template <int SRC>
static void launch_add_rmsnorm(int dtype, const void* a, const int32_t* a_rows, int64_t lda, const void* res,
                               int64_t ldr, const void* w1, const void* w2, void* x_out, const int32_t* out_rows,
                               int64_t ldo, void* h_out, int64_t ldh, int n, int D, float eps, const SrcArgs& sp,
                               hipStream_t stream) {
  if (dtype == kBF16)
    launch_norm_t<bf16_t, SRC>(a, a_rows, lda, res, ldr, w1, w2, x_out, out_rows, ldo, h_out, ldh, n, D, eps, sp,
                               stream);
  else
    launch_norm_t<float, SRC>(a, a_rows, lda, res, ldr, w1, w2, x_out, out_rows, ldo, h_out, ldh, n, D, eps, sp,
                              stream);
}

// Folded norm pairs, the row form (wfd_norm_prep; wfd_prep_t in wfd.h). One
// wave per row, the lane layout of add_rmsnorm_kernel: lane L = c + 16 j
// holds, at step s, the elements of chunk c at s KSTEP + j V -- for bf16 one
// whole 8-column group, for fp32 half of one (the other half in lane L ^ 16).
// Each element is wfd_linear_prep's epilogue value (prep_value), each group
// sum the same tree, and the lane adds its groups in step order before the
// butterfly -- the order a consumer adds the group sums wfd_linear_prep
// stores (fold_slot), so the scales are equal bit for bit. SPLIT: y is the
// in-order slice sum of wfd_linear_partials (the linear's output before its
// rounding); else y = a[i] (already rounded). r (when kept) and A are stored
// as soon as they are formed, the scales after the sums; XOUT keeps r for
// h = round((r * s_a) * wa), the first norm's output, written to rows h_rows.
template <typename T, bool SPLIT, bool RES, bool XOUT>
__global__ __launch_bounds__(256) void norm_prep_kernel(const T* __restrict__ a, int64_t lda,
                                                        const float* __restrict__ part, int64_t slice_stride,
                                                        int nslices, const wfd_prep_t pp, int two, float eps,
                                                        float* __restrict__ scale_out, float* __restrict__ s_out,
                                                        T* __restrict__ h_out, const int32_t* __restrict__ h_rows,
                                                        int64_t ldh, int n, int D) {
  constexpr int V = Chunk<T>::V;
  constexpr int KSTEP = Chunk<T>::KSTEP;
  constexpr int KC = Chunk<T>::KC;
  const int i = blockIdx.x * (blockDim.x >> 6) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int c = lane & 15;
  const int j = lane >> 4;
  if (i >= n) return;  // no barriers below
  const int P = D / KC;
  const int p = c < P ? c : P - 1;  // lanes past the last chunk re-read it (their values are never used)
  const bool live = fold_lane_live<T>(lane, P);
  const T* wa_t = (const T*)pp.wa;
  const T* wb_t = (const T*)pp.wb;
  const bool prep = pp.a_out != nullptr;  // uniform
  [[maybe_unused]] float r[kChunkSteps][V];
  float gr[kChunkSteps], gu[kChunkSteps];
  float s_in = 1.f;
  if constexpr (RES) {
    if (pp.s_in) s_in = pp.s_in[i];
  }
  // every load of the row first, then the arithmetic and the stores: the
  // stores cannot be shown not to alias the loads, so loads issued after one
  // would wait for it, one HBM round trip per step
  constexpr int YL = SPLIT ? kSplitMaxSlices * (V / 4) : 1;
  const u32x4 one = Elem<T>::pack_ones();
  u32x4 yraw[kChunkSteps][YL], rraw[kChunkSteps], wiraw[kChunkSteps], waraw[kChunkSteps], wbraw[kChunkSteps];
#pragma unroll
  for (int s = 0; s < kChunkSteps; ++s) {
    const int64_t off = (int64_t)p * KC + s * KSTEP + j * V;
    if constexpr (SPLIT) {
#pragma unroll
      for (int q = 0; q < kSplitMaxSlices; ++q) {
        const float* src = part + q * slice_stride + (int64_t)i * D + off;
#pragma unroll
        for (int h = 0; h < V / 4; ++h) yraw[s][q * (V / 4) + h] = q < nslices ? ld16(src + 4 * h) : u32x4{0, 0, 0, 0};
      }
    } else {
      yraw[s][0] = ld16(a + (int64_t)i * lda + off);
    }
    rraw[s] = wiraw[s] = one;
    if constexpr (RES) {
      rraw[s] = ld16((const T*)pp.r_in + (int64_t)i * pp.ld_in + off);
      if (pp.w_in) wiraw[s] = ld16((const T*)pp.w_in + off);
    }
    waraw[s] = wa_t ? ld16(wa_t + off) : one;
    wbraw[s] = prep ? ld16(wb_t + off) : one;
  }
#pragma unroll
  for (int s = 0; s < kChunkSteps; ++s) {
    const int64_t off = (int64_t)p * KC + s * KSTEP + j * V;
    float y[V];
    if constexpr (SPLIT) {
      // slices in order from +0 (slices past nslices load as +0)
#pragma unroll
      for (int e = 0; e < V; ++e) y[e] = 0.f;
#pragma unroll
      for (int q = 0; q < kSplitMaxSlices; ++q) {
#pragma unroll
        for (int h = 0; h < V / 4; ++h) {
#pragma unroll
          for (int e = 0; e < 4; ++e) y[4 * h + e] += __uint_as_float(yraw[s][q * (V / 4) + h][e]);
        }
      }
    } else {
      Elem<T>::unpack(yraw[s][0], y);
    }
    float rin[V], win[V], wa[V], wb[V];
    Elem<T>::unpack(rraw[s], rin);
    Elem<T>::unpack(wiraw[s], win);
    Elem<T>::unpack(waraw[s], wa);
    Elem<T>::unpack(wbraw[s], wb);
    float rv[V], Av[V], sr[V], su[V];
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const PrepVal pv = prep_value<T>(y[e], RES, rin[e], s_in, win[e], wa[e], wb[e]);
      rv[e] = pv.r;
      Av[e] = pv.A;
      sr[e] = pv.sr;
      su[e] = pv.su;
    }
    if constexpr (XOUT) {
#pragma unroll
      for (int e = 0; e < V; ++e) r[s][e] = rv[e];
    }
    if (c < P) {
      if (pp.r_out) *reinterpret_cast<u32x4*>((T*)pp.r_out + (int64_t)i * pp.ld_out + off) = Elem<T>::pack(rv);
      if (prep) *reinterpret_cast<u32x4*>((T*)pp.a_out + (int64_t)i * pp.ld_a + off) = Elem<T>::pack(Av);
    }
    // the group's tree: ((c0+c1)+(c2+c3))+((c4+c5)+(c6+c7))
    float tr = tree4(sr[0], sr[1], sr[2], sr[3]);
    float tu = tree4(su[0], su[1], su[2], su[3]);
    if constexpr (V == 8) {
      tr = add_rn(tr, tree4(sr[4], sr[5], sr[6], sr[7]));
      tu = add_rn(tu, tree4(su[4], su[5], su[6], su[7]));
    } else {  // the group's other half sits in lane L ^ 16
      tr = add_rn(tr, __shfl_xor(tr, 16, 64));
      tu = add_rn(tu, __shfl_xor(tu, 16, 64));
    }
    gr[s] = live ? tr : 0.f;
    gu[s] = live ? tu : 0.f;
  }
  float srow, surow;
  fold_sums(gr, gu, srow, surow);
  float s_a, scale;
  pair_scale(srow, surow, D, eps, two != 0, s_a, scale);
  if (prep && lane == 0) {
    scale_out[i] = scale;
    if (s_out) s_out[i] = s_a;
  }
  if constexpr (XOUT) {
    const int64_t orow = h_rows ? h_rows[i] : i;
#pragma unroll
    for (int s = 0; s < kChunkSteps; ++s) {
      const int64_t off = (int64_t)p * KC + s * KSTEP + j * V;
      float wa[V], h[V];
      Elem<T>::unpack(waraw[s], wa);
#pragma unroll
      for (int e = 0; e < V; ++e) h[e] = norm_value<T>(r[s][e], s_a, wa[e]);
      if (c < P) *reinterpret_cast<u32x4*>(h_out + orow * ldh + off) = Elem<T>::pack(h);
    }
  }
}

template <typename T, bool SPLIT, bool RES, bool XOUT>
static void launch_norm_prep_t(const void* a, int64_t lda, const float* part, int64_t slice_stride, int nslices,
                               const wfd_prep_t& pp, int two, float eps, float* scale_out, float* s_out, void* h_out,
                               const int32_t* h_rows, int64_t ldh, int n, int D, hipStream_t stream) {
  const int rpw = n >= kNormRowsPerCuLaunch ? 4 : 1;  // as add_rmsnorm: rows spread one per CU below 1024
  const dim3 grid((n + rpw - 1) / rpw), block(64 * rpw);
  hipLaunchKernelGGL((norm_prep_kernel<T, SPLIT, RES, XOUT>), grid, block, 0, stream, (const T*)a, lda, part,
                     slice_stride, nslices, pp, two, eps, scale_out, s_out, (T*)h_out, h_rows, ldh, n, D);
}

template <typename T>
static void launch_norm_prep(const void* a, int64_t lda, const float* part, int64_t slice_stride, int nslices,
                             const wfd_prep_t& pp, int two, float eps, float* scale_out, float* s_out, void* h_out,
                             const int32_t* h_rows, int64_t ldh, int n, int D, hipStream_t stream) {
#define WFD_NP(SP, RS, FI)                                                                                         \
  launch_norm_prep_t<T, SP, RS, FI>(a, lda, part, slice_stride, nslices, pp, two, eps, scale_out, s_out, h_out, \
                                    h_rows, ldh, n, D, stream)
  const bool sp = part != nullptr, rs = pp.r_in != nullptr, fi = h_out != nullptr;
  if (sp && rs && fi) WFD_NP(true, true, true);
  else if (sp && rs) WFD_NP(true, true, false);
  else if (sp && fi) WFD_NP(true, false, true);
  else if (sp) WFD_NP(true, false, false);
  else if (rs && fi) WFD_NP(false, true, true);
  else if (rs) WFD_NP(false, true, false);
  else if (fi) WFD_NP(false, false, true);
  else WFD_NP(false, false, false);
#undef WFD_NP
}

template <typename T>
__global__ __launch_bounds__(kRowThreads) void qkv_rope_append_kernel(
    const T* __restrict__ qkv, int64_t ldq, const int32_t* __restrict__ pos, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, int tab_rows, const int64_t* __restrict__ flat_row, T* __restrict__ q_out,
    T* __restrict__ kc, T* __restrict__ vc, int64_t block_rows, int H, int Hkv, int Dh) {
  const int i = blockIdx.x;
  const int half = Dh >> 1;
  int p = pos[i];
  p = p < 0 ? 0 : (p >= tab_rows ? tab_rows - 1 : p);
  const int64_t fr = flat_row[i];
  const T* src = qkv + (int64_t)i * ldq;
  const int npairs = (H + Hkv) * half;
  for (int idx = threadIdx.x; idx < npairs; idx += kRowThreads) {
    const int head = idx / half;
    const int j = idx - head * half;
    const float x0 = Elem<T>::load(src + head * Dh + 2 * j);
    const float x1 = Elem<T>::load(src + head * Dh + 2 * j + 1);
    const float c = cos_t[(int64_t)p * half + j];
    const float s = sin_t[(int64_t)p * half + j];
    const float y0 = fmaf(x0, c, -(x1 * s));
    const float y1 = fmaf(x0, s, x1 * c);
    T* dst = head < H ? q_out + ((int64_t)i * H + head) * Dh + 2 * j
                      : kc + kv_offset(fr, head - H, Hkv, Dh, block_rows) + 2 * j;
    Elem<T>::store(dst, y0);
    Elem<T>::store(dst + 1, y1);
  }
  const T* vsrc = src + (int64_t)(H + Hkv) * Dh;
  for (int e = threadIdx.x; e < Hkv * Dh; e += kRowThreads) {
    const int h = e / Dh;
    vc[kv_offset(fr, h, Hkv, Dh, block_rows) + (e - h * Dh)] = vsrc[e];
  }
}

template <typename T>
__global__ __launch_bounds__(kRowThreads) void kv_append_kernel(const T* __restrict__ k, const T* __restrict__ v,
                                                                T* __restrict__ kc, T* __restrict__ vc,
                                                                int64_t block_rows,
                                                                const int64_t* __restrict__ flat_row, int Hkv,
                                                                int Dh) {
  const int i = blockIdx.x;
  const int64_t fr = flat_row[i];
  const int row_elems = Hkv * Dh;
  for (int e = threadIdx.x; e < row_elems; e += kRowThreads) {
    const int h = e / Dh;
    const int64_t dst = kv_offset(fr, h, Hkv, Dh, block_rows) + (e - h * Dh);
    kc[dst] = k[(int64_t)i * row_elems + e];
    vc[dst] = v[(int64_t)i * row_elems + e];
  }
}

template <typename T>
__global__ __launch_bounds__(kRowThreads) void embed_kernel(const int64_t* __restrict__ ids,
                                                            const int64_t* __restrict__ ring, int64_t ring_len,
                                                            const T* __restrict__ table, float scale,
                                                            T* __restrict__ out, int64_t ldo, int Vocab, int D) {
  const int i = blockIdx.x;
  int64_t id = ids[i];
  if (id < 0 && ring) {  // a token handle: the id sits in the device token ring
    const int64_t slot = -id - 1;
    id = slot < ring_len ? ring[slot] : 0;
  }
  id = id < 0 ? 0 : (id >= Vocab ? Vocab - 1 : id);
  for (int e = threadIdx.x; e < D; e += kRowThreads) {
    float x = Elem<T>::load(table + id * D + e);
    if (scale != 1.0f) x *= scale;
    Elem<T>::store(out + (int64_t)i * ldo + e, x);
  }
}

template <typename T>
__global__ __launch_bounds__(kRowThreads) void copy_rows_kernel(const T* __restrict__ src,
                                                                const int32_t* __restrict__ src_rows, int64_t lds,
                                                                T* __restrict__ dst, const int32_t* __restrict__ dst_rows,
                                                                int64_t ldd, int width) {
  const int i = blockIdx.x;
  const int64_t sr = src_rows ? src_rows[i] : i;
  const int64_t dr = dst_rows ? dst_rows[i] : i;
  for (int e = threadIdx.x; e < width; e += kRowThreads) dst[dr * ldd + e] = src[sr * lds + e];
}

constexpr int kArgThreads = 1024;
constexpr int kArgUnroll = 8;  // a 32000-entry row: 8000 16-byte loads over 1024 threads

// Row i's id ix: out[i], the accept flag, the token ring.
__device__ __forceinline__ void argmax_finish(int i, int ix, int64_t* __restrict__ out, int64_t* __restrict__ ring,
                                              const int32_t* __restrict__ ring_rows, int64_t ring_len,
                                              const int64_t* __restrict__ expect, int32_t* __restrict__ accept) {
  out[i] = (int64_t)ix;
  if (accept) {
    // greedy acceptance on the device: the token speculated at the next
    // position is a plain id (>= 0) or a ring handle -(slot + 1) written by
    // an earlier pass; anything else is "nothing to compare" (reads 0)
    const int64_t e = expect[i];
    int64_t want = -1;
    if (e >= 0)
      want = e;
    else if (ring && e >= -ring_len)
      want = ring[-e - 1];
    accept[i] = want == (int64_t)ix ? 1 : 0;
  }
  if (ring) {
    const int32_t r = ring_rows[i];
    if (r >= 0 && r < ring_len) ring[r] = (int64_t)ix;
  }
}

// One 1024-thread workgroup per row; first index wins ties (as torch.argmax).
__global__ __launch_bounds__(kArgThreads) void argmax_kernel(const float* __restrict__ logits, int64_t ld,
                                                            int64_t* __restrict__ out, int64_t* __restrict__ ring,
                                                            const int32_t* __restrict__ ring_rows, int64_t ring_len,
                                                            const int64_t* __restrict__ expect,
                                                            int32_t* __restrict__ accept, int Vocab) {
  __shared__ float sv[kArgThreads / 64];
  __shared__ int si[kArgThreads / 64];
  const int i = blockIdx.x;
  const float* row = logits + (int64_t)i * ld;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  const int nv = ((ld & 3) == 0) ? Vocab / 4 : 0;  // 16-byte loads when rows stay aligned
  // kArgUnroll loads in flight per thread before the first compare (the row
  // was just written by other CUs: one round trip instead of one per load);
  // the merge is order-free (value, then lowest index)
  for (int q0 = threadIdx.x; q0 < nv; q0 += kArgThreads * kArgUnroll) {
    u32x4 w[kArgUnroll];
#pragma unroll
    for (int u = 0; u < kArgUnroll; ++u) {
      const int q = q0 + u * kArgThreads;
      w[u] = q < nv ? ld16(row + 4 * q) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kArgUnroll; ++u) {
      const int q = q0 + u * kArgThreads;
      if (q < nv) {
#pragma unroll
        for (int k = 0; k < 4; ++k) argmax_merge(best, bi, __uint_as_float(w[u][k]), 4 * q + k);
      }
    }
  }
  for (int e = 4 * nv + threadIdx.x; e < Vocab; e += kArgThreads) argmax_merge(best, bi, row[e], e);
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(best, m, 64);
    const int oi = __shfl_xor(bi, m, 64);
    argmax_merge(best, bi, ov, oi);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sv[0];
    int ix = si[0];
    for (int w = 1; w < kArgThreads / 64; ++w) argmax_merge(b, ix, sv[w], si[w]);
    argmax_finish(i, ix, out, ring, ring_rows, ring_len, expect, accept);
  }
}

// The same ids from the per-column-group bests a few-row linear leaves
// (val / idx[i * groups + s]): the merge is order-free, so merging the group
// bests gives the first index of the row's largest value, as over the row.
// One 256-thread workgroup per row.
constexpr int kArgGroupThreads = 256;
__global__ __launch_bounds__(kArgGroupThreads) void argmax_groups_kernel(
    const float* __restrict__ val, const int32_t* __restrict__ idx, int groups, int64_t* __restrict__ out,
    int64_t* __restrict__ ring, const int32_t* __restrict__ ring_rows, int64_t ring_len,
    const int64_t* __restrict__ expect, int32_t* __restrict__ accept) {
  __shared__ float sv[kArgGroupThreads / 64];
  __shared__ int si[kArgGroupThreads / 64];
  const int i = blockIdx.x;
  const float* v = val + (int64_t)i * groups;
  const int32_t* x = idx + (int64_t)i * groups;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  constexpr int U = 8;  // loads in flight per thread (2000 groups: one round)
  for (int s0 = threadIdx.x; s0 < groups; s0 += kArgGroupThreads * U) {
    float ov[U];
    int oi[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = s0 + u * kArgGroupThreads;
      ov[u] = s < groups ? v[s] : -INFINITY;
      oi[u] = s < groups ? x[s] : 0x7fffffff;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) argmax_merge(best, bi, ov[u], oi[u]);
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    const float ov = __shfl_xor(best, m, 64);
    const int oi = __shfl_xor(bi, m, 64);
    argmax_merge(best, bi, ov, oi);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sv[0];
    int ix = si[0];
    for (int w = 1; w < kArgGroupThreads / 64; ++w) argmax_merge(b, ix, sv[w], si[w]);
    argmax_finish(i, ix, out, ring, ring_rows, ring_len, expect, accept);
  }
}

// SwiGLU of rows laid out [gate (F) | up (F)]: out[i][j] = silu(gate) * up,
// silu(v) = v / (1 + e^-v), in fp32 from the stored (rounded) gate and up,
// rounded once -- the linear layer's SwiGLU epilogue for a gate|up product
// computed elsewhere (the prompt pass's library GEMM). One 16-byte vector of
// each half per thread.
template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(const T* __restrict__ gu, int64_t ldg, T* __restrict__ out,
                                                     int64_t ldo, int n, int F) {
  constexpr int V = Elem<T>::kVec;
  const int per_row = F / V;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)n * per_row) return;
  const int i = (int)(t / per_row);
  const int j = (int)(t - (int64_t)i * per_row) * V;
  float g[V], u[V], o[V];
  Elem<T>::unpack(ld16(gu + (int64_t)i * ldg + j), g);
  Elem<T>::unpack(ld16(gu + (int64_t)i * ldg + F + j), u);
#pragma unroll
  for (int e = 0; e < V; ++e) o[e] = (g[e] / (1.0f + expf(-g[e]))) * u[e];
  *reinterpret_cast<u32x4*>(out + (int64_t)i * ldo + j) = Elem<T>::pack(o);
}

}  // namespace wfd

extern "C" {

const char* wfd_last_error(void) { return wfd::g_err; }

int wfd_abi_version(void) { return 7; }

int wfd_add_rmsnorm(const void* a, const int32_t* a_rows, int64_t lda, const void* res, int64_t ldr, const void* w1,
                    const void* w2, void* x_out, const int32_t* out_rows, int64_t ldo, void* h_out, int64_t ldh, int n,
                    int D, float eps, int dtype, hipStream_t stream) {
  using namespace wfd;
  if (dtype != kBF16 && dtype != kF32) {
    set_error("wfd_add_rmsnorm: unsupported dtype %d", dtype);
    return kUnsupported;
  }
  const int kc = dtype == kBF16 ? Chunk<bf16_t>::KC : Chunk<float>::KC;
  if (n < 0 || D <= 0 || D > kNormMaxD || D % kc != 0) {
    set_error("wfd_add_rmsnorm: bad shape n=%d D=%d (D <= %d, multiple of %d)", n, D, kNormMaxD, kc);
    return kBadArg;
  }
  const int esz = dtype == kBF16 ? 2 : 4;
  if ((((uintptr_t)a | (uintptr_t)res | (uintptr_t)w1 | (uintptr_t)w2 | (uintptr_t)x_out | (uintptr_t)h_out) & 15) ||
      ((lda * esz) & 15) || (res && ((ldr * esz) & 15)) || (x_out && ((ldo * esz) & 15)) ||
      (h_out && ((ldh * esz) & 15))) {
    set_error("wfd_add_rmsnorm: rows must be 16-byte aligned");
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!a || !w1 || (w2 && !h_out) || (!w2 && !x_out)) {
    set_error("wfd_add_rmsnorm: null pointer argument");
    return kBadArg;
  }
  launch_add_rmsnorm<kSrcRows>(dtype, a, a_rows, lda, res, ldr, w1, w2, x_out, out_rows, ldo, h_out, ldh, n, D, eps,
                               SrcArgs{}, stream);
  return launch_status("wfd_add_rmsnorm");
}

int wfd_add_rmsnorm_split(const float* part, int64_t slice_stride, int nslices, void* a_out, int64_t lda_out,
                          const void* res, int64_t ldr, const void* w1, const void* w2, void* x_out,
                          const int32_t* out_rows, int64_t ldo, void* h_out, int64_t ldh, int n, int D, float eps,
                          int dtype, hipStream_t stream) {
  using namespace wfd;
  if (dtype != kBF16 && dtype != kF32) {
    set_error("wfd_add_rmsnorm_split: unsupported dtype %d", dtype);
    return kUnsupported;
  }
  const int kc = dtype == kBF16 ? Chunk<bf16_t>::KC : Chunk<float>::KC;
  if (n < 0 || D <= 0 || D > kNormMaxD || D % kc != 0 || nslices < 1 || nslices > kSplitMaxSlices ||
      slice_stride < (int64_t)n * D) {
    set_error("wfd_add_rmsnorm_split: bad shape n=%d D=%d nslices=%d slice_stride=%lld", n, D, nslices,
              (long long)slice_stride);
    return kBadArg;
  }
  const int esz = dtype == kBF16 ? 2 : 4;
  if ((((uintptr_t)part | (uintptr_t)a_out | (uintptr_t)res | (uintptr_t)w1 | (uintptr_t)w2 | (uintptr_t)x_out |
        (uintptr_t)h_out) & 15) || ((slice_stride * 4) & 15) || (a_out && ((lda_out * esz) & 15)) ||
      (res && ((ldr * esz) & 15)) || (x_out && ((ldo * esz) & 15)) || (h_out && ((ldh * esz) & 15))) {
    set_error("wfd_add_rmsnorm_split: rows must be 16-byte aligned");
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!part || !w1 || (w2 && !h_out) || (!w2 && !x_out)) {
    set_error("wfd_add_rmsnorm_split: null pointer argument");
    return kBadArg;
  }
  SrcArgs sp{};
  sp.part = part;
  sp.slice_stride = slice_stride;
  sp.nslices = nslices;
  sp.a_out = a_out;
  sp.lda_out = lda_out;
  launch_add_rmsnorm<kSrcSplit>(dtype, nullptr, nullptr, 0, res, ldr, w1, w2, x_out, out_rows, ldo, h_out, ldh, n, D,
                                eps, sp, stream);
  return launch_status("wfd_add_rmsnorm_split");
}

int wfd_norm_prep(const void* a, int64_t lda, const float* part, int64_t slice_stride, int nslices,
                  const wfd_prep_t* pp, int two, float eps, float* scale_out, float* s_out, void* h_out,
                  const int32_t* h_rows, int64_t ldh, int n, int D, int dtype, hipStream_t stream) {
  using namespace wfd;
  if (dtype != kBF16 && dtype != kF32) {
    set_error("wfd_norm_prep: unsupported dtype %d", dtype);
    return kUnsupported;
  }
  const int kc = dtype == kBF16 ? Chunk<bf16_t>::KC : Chunk<float>::KC;
  const int dmax = dtype == kBF16 ? fold_max_d<bf16_t>() : fold_max_d<float>();
  if (n < 0 || D <= 0 || D > dmax || D % kc != 0 ||
      (part && (nslices < 1 || nslices > kSplitMaxSlices || slice_stride < (int64_t)n * D))) {
    set_error("wfd_norm_prep: bad shape n=%d D=%d (a multiple of %d, at most %d) nslices=%d", n, D, kc, dmax,
              nslices);
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!pp || (!part && !a) || (!h_out && !pp->a_out) || (pp->a_out && (!pp->wb || !scale_out))) {
    set_error("wfd_norm_prep: null pointer argument (a or part; h_out or pp->a_out; the prep form needs pp->wb "
              "and scale_out)");
    return kBadArg;
  }
  if ((pp->wa != nullptr) != (two != 0)) {
    set_error("wfd_norm_prep: two must be set exactly when norm a's weight pp->wa is given");
    return kBadArg;
  }
  if ((a && lda < D) || (pp->r_in && pp->ld_in < D) || (pp->r_out && pp->ld_out < D) || (pp->a_out && pp->ld_a < D) ||
      (h_out && ldh < D)) {
    set_error("wfd_norm_prep: a row pitch is below D=%d", D);
    return kBadArg;
  }
  const int esz = dtype == kBF16 ? 2 : 4;
  if ((((uintptr_t)a | (uintptr_t)part | (uintptr_t)pp->r_in | (uintptr_t)pp->w_in | (uintptr_t)pp->r_out |
        (uintptr_t)pp->a_out | (uintptr_t)pp->wa | (uintptr_t)pp->wb | (uintptr_t)h_out) & 15) ||
      ((slice_stride * 4) & 15) || (a && ((lda * esz) & 15)) || (pp->r_in && ((pp->ld_in * esz) & 15)) ||
      (pp->r_out && ((pp->ld_out * esz) & 15)) || (pp->a_out && ((pp->ld_a * esz) & 15)) ||
      (h_out && ((ldh * esz) & 15))) {
    set_error("wfd_norm_prep: rows must be 16-byte aligned");
    return kBadArg;
  }
  if (dtype == kBF16)
    launch_norm_prep<bf16_t>(a, lda, part, slice_stride, nslices, *pp, two, eps, scale_out, s_out, h_out, h_rows, ldh,
                             n, D, stream);
  else
    launch_norm_prep<float>(a, lda, part, slice_stride, nslices, *pp, two, eps, scale_out, s_out, h_out, h_rows, ldh,
                            n, D, stream);
  return launch_status("wfd_norm_prep");
}

int wfd_embed_rmsnorm(const int64_t* ids, const int64_t* ring, int64_t ring_len, const void* table, float scale,
                      int vocab, const void* w1, void* x_out, int64_t ldx, void* h_out, int64_t ldh,
                      const void* cp_src, const int32_t* cp_src_rows, int64_t cp_lds, void* cp_dst,
                      const int32_t* cp_dst_rows, int64_t cp_ldd, int cp_width, int n, int D, float eps, int dtype,
                      hipStream_t stream) {
  using namespace wfd;
  if (dtype != kBF16 && dtype != kF32) {
    set_error("wfd_embed_rmsnorm: unsupported dtype %d", dtype);
    return kUnsupported;
  }
  const int kc = dtype == kBF16 ? Chunk<bf16_t>::KC : Chunk<float>::KC;
  const int esz = dtype == kBF16 ? 2 : 4;
  const int vec = 16 / esz;
  if (n < 0 || D <= 0 || D > kNormMaxD || D % kc != 0 || vocab <= 0 || ring_len < 0 ||
      (cp_src && (cp_width <= 0 || cp_width % vec || cp_lds < cp_width || cp_ldd < cp_width))) {
    set_error("wfd_embed_rmsnorm: bad shape n=%d D=%d vocab=%d cp_width=%d", n, D, vocab, cp_width);
    return kBadArg;
  }
  if ((((uintptr_t)table | (uintptr_t)w1 | (uintptr_t)x_out | (uintptr_t)h_out | (uintptr_t)cp_src |
        (uintptr_t)cp_dst) & 15) || (x_out && ((ldx * esz) & 15)) || ((ldh * esz) & 15) ||
      (cp_src && (((cp_lds * esz) & 15) || ((cp_ldd * esz) & 15)))) {
    set_error("wfd_embed_rmsnorm: rows must be 16-byte aligned");
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!ids || !table || !w1 || !h_out || (cp_src && !cp_dst)) {
    set_error("wfd_embed_rmsnorm: null pointer argument");
    return kBadArg;
  }
  SrcArgs sp{};
  sp.ids = ids;
  sp.ring = ring;
  sp.ring_len = ring_len;
  sp.table = table;
  sp.scale = scale;
  sp.vocab = vocab;
  sp.cp_src = cp_src;
  sp.cp_src_rows = cp_src_rows;
  sp.cp_lds = cp_lds;
  sp.cp_dst = cp_dst;
  sp.cp_dst_rows = cp_dst_rows;
  sp.cp_ldd = cp_ldd;
  sp.cp_width = cp_width;
  sp.a_out = x_out;
  sp.lda_out = ldx;
  // the norm's output is h; the embedded row is kept through a_out
  launch_add_rmsnorm<kSrcEmbed>(dtype, nullptr, nullptr, 0, nullptr, 0, w1, nullptr, h_out, nullptr, ldh, nullptr, 0,
                                n, D, eps, sp, stream);
  return launch_status("wfd_embed_rmsnorm");
}

int wfd_qkv_rope_append(const void* qkv, int64_t ldq, const int32_t* pos, const float* rope_cos,
                        const float* rope_sin, int rope_rows, const int64_t* flat_row, void* q_out, void* k_cache,
                        void* v_cache, int64_t kv_block_rows, int n, int H, int Hkv, int Dh, int dtype,
                        hipStream_t stream) {
  using namespace wfd;
  if (n < 0 || H <= 0 || Hkv <= 0 || Dh <= 0 || (Dh & 1) || rope_rows <= 0 || ldq < (int64_t)(H + 2 * Hkv) * Dh ||
      kv_block_rows < 0) {
    set_error("wfd_qkv_rope_append: bad shape n=%d H=%d Hkv=%d Dh=%d rope_rows=%d", n, H, Hkv, Dh, rope_rows);
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!qkv || !pos || !rope_cos || !rope_sin || !flat_row || !q_out || !k_cache || !v_cache) {
    set_error("wfd_qkv_rope_append: null pointer argument");
    return kBadArg;
  }
  if (dtype == kBF16)
    hipLaunchKernelGGL(qkv_rope_append_kernel<bf16_t>, dim3(n), dim3(kRowThreads), 0, stream, (const bf16_t*)qkv, ldq,
                       pos, rope_cos, rope_sin, rope_rows, flat_row, (bf16_t*)q_out, (bf16_t*)k_cache,
                       (bf16_t*)v_cache, kv_block_rows, H, Hkv, Dh);
  else if (dtype == kF32)
    hipLaunchKernelGGL(qkv_rope_append_kernel<float>, dim3(n), dim3(kRowThreads), 0, stream, (const float*)qkv, ldq,
                       pos, rope_cos, rope_sin, rope_rows, flat_row, (float*)q_out, (float*)k_cache, (float*)v_cache,
                       kv_block_rows, H, Hkv, Dh);
  else {
    set_error("wfd_qkv_rope_append: unsupported dtype %d", dtype);
    return kUnsupported;
  }
  return launch_status("wfd_qkv_rope_append");
}

int wfd_swiglu(const void* gu, int64_t ldg, void* out, int64_t ldo, int n, int F, int dtype, hipStream_t stream) {
  using namespace wfd;
  const int vec = dtype == kBF16 ? Elem<bf16_t>::kVec : Elem<float>::kVec;
  if (dtype != kBF16 && dtype != kF32) {
    set_error("wfd_swiglu: unsupported dtype %d", dtype);
    return kUnsupported;
  }
  if (n < 0 || F <= 0 || F % vec || ldg < 2 * (int64_t)F || ldo < F || ldg % vec || ldo % vec) {
    set_error("wfd_swiglu: bad shape n=%d F=%d ldg=%lld ldo=%lld (F and strides multiples of %d)", n, F,
              (long long)ldg, (long long)ldo, vec);
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!gu || !out || ((uintptr_t)gu & 15) || ((uintptr_t)out & 15)) {
    set_error("wfd_swiglu: null or unaligned pointer (16-byte alignment)");
    return kBadArg;
  }
  const int64_t threads = (int64_t)n * (F / vec);
  const dim3 grid((unsigned)((threads + 255) / 256));
  if (dtype == kBF16)
    hipLaunchKernelGGL(swiglu_kernel<bf16_t>, grid, dim3(256), 0, stream, (const bf16_t*)gu, ldg, (bf16_t*)out, ldo,
                       n, F);
  else
    hipLaunchKernelGGL(swiglu_kernel<float>, grid, dim3(256), 0, stream, (const float*)gu, ldg, (float*)out, ldo, n,
                       F);
  return launch_status("wfd_swiglu");
}

int wfd_kv_append(const void* k, const void* v, void* k_cache, void* v_cache, int64_t kv_block_rows,
                  const int64_t* flat_row, int n, int Hkv, int Dh, int dtype, hipStream_t stream) {
  using namespace wfd;
  if (n < 0 || Hkv <= 0 || Dh <= 0 || kv_block_rows < 0) {
    set_error("wfd_kv_append: bad shape n=%d Hkv=%d Dh=%d kv_block_rows=%lld", n, Hkv, Dh, (long long)kv_block_rows);
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!k || !v || !k_cache || !v_cache || !flat_row) {
    set_error("wfd_kv_append: null pointer argument");
    return kBadArg;
  }
  if (dtype == kBF16)
    hipLaunchKernelGGL(kv_append_kernel<bf16_t>, dim3(n), dim3(kRowThreads), 0, stream, (const bf16_t*)k,
                       (const bf16_t*)v, (bf16_t*)k_cache, (bf16_t*)v_cache, kv_block_rows, flat_row, Hkv, Dh);
  else if (dtype == kF32)
    hipLaunchKernelGGL(kv_append_kernel<float>, dim3(n), dim3(kRowThreads), 0, stream, (const float*)k,
                       (const float*)v, (float*)k_cache, (float*)v_cache, kv_block_rows, flat_row, Hkv, Dh);
  else {
    set_error("wfd_kv_append: unsupported dtype %d", dtype);
    return kUnsupported;
  }
  return launch_status("wfd_kv_append");
}

int wfd_embed(const int64_t* ids, const int64_t* ring, int64_t ring_len, const void* table, float scale, void* out,
              int64_t ldo, int n, int vocab, int D, int dtype, hipStream_t stream) {
  using namespace wfd;
  if (n < 0 || vocab <= 0 || D <= 0 || ldo < D) {
    set_error("wfd_embed: bad shape n=%d vocab=%d D=%d", n, vocab, D);
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!ids || !table || !out || (ring && ring_len <= 0)) {
    set_error("wfd_embed: null pointer argument (or empty ring)");
    return kBadArg;
  }
  if (dtype == kBF16)
    hipLaunchKernelGGL(embed_kernel<bf16_t>, dim3(n), dim3(kRowThreads), 0, stream, ids, ring, ring_len,
                       (const bf16_t*)table, scale, (bf16_t*)out, ldo, vocab, D);
  else if (dtype == kF32)
    hipLaunchKernelGGL(embed_kernel<float>, dim3(n), dim3(kRowThreads), 0, stream, ids, ring, ring_len,
                       (const float*)table, scale, (float*)out, ldo, vocab, D);
  else {
    set_error("wfd_embed: unsupported dtype %d", dtype);
    return kUnsupported;
  }
  return launch_status("wfd_embed");
}

int wfd_copy_rows(const void* src, const int32_t* src_rows, int64_t lds, void* dst, const int32_t* dst_rows,
                  int64_t ldd, int n, int width, int dtype, hipStream_t stream) {
  using namespace wfd;
  if (n < 0 || width <= 0 || lds < width || ldd < width) {
    set_error("wfd_copy_rows: bad shape n=%d width=%d", n, width);
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!src || !dst) {
    set_error("wfd_copy_rows: null pointer argument");
    return kBadArg;
  }
  if (dtype == kBF16)
    hipLaunchKernelGGL(copy_rows_kernel<uint16_t>, dim3(n), dim3(kRowThreads), 0, stream, (const uint16_t*)src,
                       src_rows, lds, (uint16_t*)dst, dst_rows, ldd, width);
  else if (dtype == kF32)
    hipLaunchKernelGGL(copy_rows_kernel<float>, dim3(n), dim3(kRowThreads), 0, stream, (const float*)src, src_rows,
                       lds, (float*)dst, dst_rows, ldd, width);
  else {
    set_error("wfd_copy_rows: unsupported dtype %d", dtype);
    return kUnsupported;
  }
  return launch_status("wfd_copy_rows");
}

int wfd_argmax(const float* logits, int64_t ld, int64_t* out, int64_t* ring, const int32_t* ring_rows,
               int64_t ring_len, const int64_t* expect, int32_t* accept, int n, int vocab, hipStream_t stream) {
  using namespace wfd;
  if (n < 0 || vocab <= 0 || ld < vocab) {
    set_error("wfd_argmax: bad shape n=%d vocab=%d", n, vocab);
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!logits || !out || (ring && (!ring_rows || ring_len <= 0)) || (!expect != !accept)) {
    set_error("wfd_argmax: null pointer argument (ring needs ring_rows and a length; expect and accept go together)");
    return kBadArg;
  }
  if (((uintptr_t)logits) & 15) {
    set_error("wfd_argmax: logits must be 16-byte aligned");
    return kBadArg;
  }
  hipLaunchKernelGGL(argmax_kernel, dim3(n), dim3(kArgThreads), 0, stream, logits, ld, out, ring, ring_rows,
                     ring_len, expect, accept, vocab);
  return launch_status("wfd_argmax");
}

int wfd_argmax_groups(const float* part_val, const int32_t* part_idx, int groups, int64_t* out, int64_t* ring,
                      const int32_t* ring_rows, int64_t ring_len, const int64_t* expect, int32_t* accept, int n,
                      hipStream_t stream) {
  using namespace wfd;
  if (n < 0 || groups <= 0) {
    set_error("wfd_argmax_groups: bad shape n=%d groups=%d", n, groups);
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!part_val || !part_idx || !out || (ring && (!ring_rows || ring_len <= 0)) || (!expect != !accept)) {
    set_error("wfd_argmax_groups: null pointer argument (ring needs ring_rows and a length; expect and accept go "
              "together)");
    return kBadArg;
  }
  hipLaunchKernelGGL(argmax_groups_kernel, dim3(n), dim3(kArgGroupThreads), 0, stream, part_val, part_idx, groups,
                     out, ring, ring_rows, ring_len, expect, accept);
  return launch_status("wfd_argmax_groups");
}

}  // extern "C"
