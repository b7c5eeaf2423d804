// Row-invariant skinny linear layer: y[m, :] = x[m, :] @ W^T on MFMA.
//
// Replaces the nn.Linear calls of the block forwards (Wqkv, proj, the gated
// MLP, the adapter, lm_head; src/decoding/huginn_blocks.py:79,100-102,216,291
// and huginn_blocks_batch.py:149,160-161,299,345). At decode M = n is 1..~512
// rows while W is 4-128 MB, so the layer is a weight stream: each weight byte
// is read from HBM once per launch.
//
// Work unit: a tile of 16 weight rows (the 16 output columns of one MFMA).
// For the gated MLP a tile holds 8 gate rows and the 8 matching up rows, so a
// launch has N/16 tiles whatever the epilogue -- enough workgroups to keep
// every CU streaming (pairing a 16-row gate tile with its 16-row up tile
// halves the grid and leaves the chip underfed at the 11264 x 2048 MLP input).
//
// Arithmetic contract (depends on K and the dtype only, never on n or on how
// the work is split): K is cut into P = K / KC chunks of 4 MFMA k-steps
// (KC = 128 bf16 / 64 fp32 elements); the chunks into at most 4 consecutive
// slices of Q = ceil(P / 4) chunks, and each slice into at most 4 consecutive
// sub-slices of R = ceil(Q / 4) chunks. A chunk partial is the MFMA chain over
// its 4 steps starting from zero; a sub-slice sum is ((0 + c_a) + c_a+1) + ...
// over its chunks in order, a slice sum ((0 + u_0) + u_1) + ... over its
// sub-slices in order, and y = epilogue(((0 + s_0) + s_1) + ...) over the
// slices in order, all in fp32. The slices let a many-row launch split K
// across workgroups (wfd_linear_partials writes the slice sums; the consumer
// adds them in slice order); the sub-slices (at most 16) let a few-row launch
// give each wave one run of chunks to sum in registers. Every sum starts at
// +0 and so is never -0: adding a +0 for an empty (sub-)slice leaves its bits.
// Five kernels honour the contract bit for bit:
//
//  * wide (n <= 16): one 16-wave workgroup per tile (or column half of a
//    tile), 8 waves when there are more than 512 tiles; wave w sums sub-slice
//    w (and w + 8 with 8 waves) in registers (all loads of a wave issued
//    together), parks it in LDS, and threads add the 16 sub-slice sums in
//    contract order. No cross-workgroup synchronization: a tile's whole K is
//    reduced inside one workgroup.
//  * tile (n > 16, few row-block x tile pairs): a workgroup owns 64 rows of x
//    and 2 tiles; each of its 4 waves walks the chunks in order for one
//    16-row block of x and both tiles, with a two-stage register pipeline.
//  * gemm (n > 16, many pairs): 64 rows x 2 or 4 tiles per workgroup, the
//    tiles' weights staged once in LDS for the 4 waves, weights and x loaded
//    two chunks ahead, an XCD-aware grid.
//  * stream (n > 16, at most 256 tiles): 64 rows x 1 or 2 tiles per
//    workgroup, weights and x moved global -> LDS by direct-to-LDS loads
//    through a 4-stage ring (3 chunks in flight without registers).
//  * gemm, slice form (wfd_linear_partials): the gemm kernel over one slice
//    of K per workgroup (grid y = slice), storing fp32 slice partials.
//
// So y[m] is bit-identical whatever n is and wherever row m sits -- the
// property that keeps wavefront decode token-identical to sequential decode.
//
// x operand: every kernel reads a 16-row block's chunk with coalesced loads
// of whole 256-byte row segments and turns them into MFMA fragments through
// the wave's LDS (xc_offsets below): a fragment load would touch 16 rows x 64
// bytes per instruction.
//
// Weight layout ("packed", made once by wfd_linear_pack): W is stored in MFMA
// fragment order, tile by tile -- for tile g, chunk p, step s the 64 lanes'
// 16-byte B fragments sit back to back, so every weight load instruction of a
// wave reads 1 KB of contiguous memory (row-major W would make each
// instruction touch 16 rows x 64 B). SwiGLU gate/up rows are paired into
// tiles by the packing.
//
// Epilogues: plain store (bf16 or fp32 out); SwiGLU, out = silu(gate) * up
// from columns c and c + 8 of a tile (one lane shuffle apart); and
// QKV-RoPE-append, for the fused q|k|v projection: the output row is rounded
// to the element type, q and k heads are rotated by the row's position
// (interleaved pairs: columns 2j and 2j+1 sit in one tile, so the partner
// value is one lane shuffle away), q goes to q_out and k, v are written
// straight into the slot cache row flat_row[m] (src/decoding/huginn_blocks.py:77-87
// + kv_cache.py:97-104 fused into the projection; the separate qkv_rope_append
// pass and its qkv round trip vanish).
#include <type_traits>

#include "wfd_common.h"

namespace wfd {

constexpr int kWideWaves = 16;
constexpr int kWideMaxChunksPerWave = 3;
constexpr int kWideMaxRows = 16;
constexpr int kHalfTileMax = 256;  // wide launches of at most this many tiles use half tiles
constexpr int kResidentWide = 512;  // 1024-thread workgroups resident at once (two per CU)
// (64-row block, weight tile) pairs up to which a many-row launch lets each
// wave stream its own weights (tile kernel) rather than share them through
// LDS (gemm kernel): measured crossover on the 2048-d model's projections
constexpr int kGemmMinBlockTiles = 512;
// Launches of at most this many weight tiles (2048 output columns) use the
// stream kernel, with this many LDS stages
constexpr int kStreamMaxTiles = 256;
constexpr int kStreamStages = 4;
// kEpiPrep: a d_model-output linear whose epilogue prepares the residual
// stream of a folded norm pair (wfd_prep_t), few-row launches only
enum Epilogue : int { kEpiPlain = 0, kEpiSwiGLU = 1, kEpiRope = 2, kEpiPrep = 3 };

// K slices and sub-slices of the arithmetic contract (see the header): at most
// 4 slices of Q = ceil(P / 4) chunks, each of at most 4 sub-slices of
// R = ceil(Q / 4) = ceil(P / 16) chunks.
constexpr int kSlices = 4;
constexpr int kSubSlices = 4;  // per slice
__host__ __device__ constexpr int slice_chunks(int P) { return (P + kSlices - 1) / kSlices; }
__host__ __device__ constexpr int slice_count(int P) { return (P + slice_chunks(P) - 1) / slice_chunks(P); }
__host__ __device__ constexpr int sub_chunks(int P) { return (slice_chunks(P) + kSubSlices - 1) / kSubSlices; }

// Where a kernel that walks chunks in order (from the start of a slice)
// closes a sub-slice or a slice: a running boundary, not a modulo (a chunk
// loop that tests p % Q pays an integer division per chunk).
struct SliceWalk {
  int P, Q, R, nsl, nsub;
  __device__ __forceinline__ SliceWalk(int P_, int p0)
      : P(P_), Q(slice_chunks(P_)), R(sub_chunks(P_)), nsl(p0 + slice_chunks(P_)), nsub(p0 + sub_chunks(P_)) {}
  // after chunk p: 0 inside a sub-slice, 1 a sub-slice ended, 2 a slice ended
  __device__ __forceinline__ int end(int p) {
    const int e = p + 1;
    if (e == nsl || e == P) {
      nsl += Q;
      nsub = e + R;
      return 2;
    }
    if (e == nsub) {
      nsub += R;
      return 1;
    }
    return 0;
  }
};

// Chunk partials into the contract's running sums: sub-slice, slice, total.
template <int NT>
__device__ __forceinline__ void contract_add(f32x4 (&sub)[NT], f32x4 (&sl)[NT], f32x4 (&tot)[NT],
                                             const f32x4 (&acc)[NT], int lvl) {
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) sub[t][r] += acc[t][r];
  if (lvl >= 1) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) sl[t][r] += sub[t][r];
      sub[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  if (lvl == 2) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int r = 0; r < 4; ++r) tot[t][r] += sl[t][r];
      sl[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
}

// Operands of the QKV-RoPE-append epilogue (unused by the others).
struct RopeArgs {
  const int32_t* pos;       // [n] positions (clamped into the table)
  const float* cos_t;       // [rows, Dh/2]
  const float* sin_t;       // [rows, Dh/2]
  int tab_rows;
  const int64_t* flat_row;  // [n] slot-cache row of each token
  void* q_out;              // [n, H, Dh]
  void* k_cache;            // slot cache, laid out as kv_offset() describes
  void* v_cache;
  int64_t block_rows;       // cache layout (kv_offset)
  int H, Hkv, Dh;
};

// Optional output of the few-row kernel (plain epilogue, fp32 y): per row m
// and column group s (the workgroup: a tile, or half a tile), the first
// largest value of y[m, group s] and its column at val / idx[m * groups + s].
struct TileArgmax {
  float* val;
  int32_t* idx;
};

template <typename T>
using LinTraits = Chunk<T>;

// Weight row behind column c (0..15) of tile g. A SwiGLU tile holds gate rows
// 8g..8g+7 in columns 0-7 and the matching up rows (pair_off below) in 8-15.
template <int EPI>
__device__ __forceinline__ int weight_row(int g, int c, int pair_off) {
  if (EPI == kEpiSwiGLU) return c < 8 ? 8 * g + c : pair_off + 8 * g + (c - 8);
  return 16 * g + c;
}

// The table operands of one output (row, col) of the QKV-RoPE-append
// epilogue: its rotation (cos, sin at the row's position; identity for v
// heads) and, for k / v heads, the row's slot-cache row. Loaded apart from the
// stores: a store may alias the tables as far as the compiler knows, so a
// load placed after one would wait for it -- kernels gather every operand of
// their outputs first (or at launch), then store.
struct RopePre {
  float c, s;
  int64_t ro;  // k / v heads: the cache offset of the row's kv head 0
};

// Head and in-head column of column 0 of tile g: uniform over the tile
// (Dh % 16 == 0), so one scalar division per tile rather than one per lane.
__device__ __forceinline__ int tile_head(const RopeArgs& ra, int g, int& dbase) {
  const int c0 = __builtin_amdgcn_readfirstlane(16 * g);
  const int head = c0 / ra.Dh;
  dbase = c0 - head * ra.Dh;
  return head;
}

// kv_offset(row, h) = kv_offset(row, 0) + h * kv_head_stride: the division
// by the block size is paid once per row, not once per stored element.
__device__ __forceinline__ int64_t kv_head_stride(const RopeArgs& ra) {
  return ra.block_rows > 1 ? ra.block_rows * ra.Dh : (int64_t)ra.Dh;
}

__device__ __forceinline__ int64_t rope_row_off(const RopeArgs& ra, int row) {
  return kv_offset(ra.flat_row[row], 0, ra.Hkv, ra.Dh, ra.block_rows);
}

__device__ __forceinline__ int rope_row_pos(const RopeArgs& ra, int row) {
  const int p = ra.pos[row];
  return p < 0 ? 0 : (p >= ra.tab_rows ? ra.tab_rows - 1 : p);
}

// The rotation of output (head, in-head column d) of a row at table position
// p; `ro` = the row's rope_row_off, carried for the store.
__device__ __forceinline__ RopePre rope_pre(const RopeArgs& ra, int p, int head, int d, int64_t ro) {
  RopePre o{1.f, 0.f, ro};
  if (head < ra.H + ra.Hkv) {
    const int half = ra.Dh >> 1;
    o.c = ra.cos_t[(int64_t)p * half + (d >> 1)];
    o.s = ra.sin_t[(int64_t)p * half + (d >> 1)];
  }
  return o;
}

// Value v0 of output (row, head, in-head column d) and its RoPE partner v1 =
// the value of column d ^ 1.
template <typename TO>
__device__ __forceinline__ void store_rope(const RopeArgs& ra, const RopePre& o, int row, int head, int d, float v0,
                                           float v1) {
  TO* dst;
  float out;
  if (head >= ra.H + ra.Hkv) {
    dst = (TO*)ra.v_cache + o.ro + (head - ra.H - ra.Hkv) * kv_head_stride(ra) + d;
    out = v0;
  } else {
    const float xm = Elem<TO>::round(v0);
    const float xp = Elem<TO>::round(v1);
    out = (d & 1) ? fmaf(xp, o.s, xm * o.c) : fmaf(xm, o.c, -(xp * o.s));
    dst = head < ra.H ? (TO*)ra.q_out + ((int64_t)row * ra.H + head) * ra.Dh + d
                      : (TO*)ra.k_cache + o.ro + (head - ra.H) * kv_head_stride(ra) + d;
  }
  Elem<TO>::store(dst, out);
}

// Operands of the QKV-RoPE-append epilogue for a lane's rows row4 .. row4 + 3
// (rows past n read row 0's, never stored) in two parts: per row, the table
// position and the cache offset of kv head 0, gathered at launch (their load
// round trip overlaps the main loop; 3 VGPRs a row); per output of tiles
// g0 .. g0 + NT - 1 (past the last tile: the last one's) at column col, the
// cos / sin pair, gathered after the main loop from the rows' positions (one
// round trip, and no table registers held through the loop). Loaded apart
// from the stores: a store may alias the tables as far as the compiler
// knows, so a load placed after one would wait for it. A no-op for the other
// epilogues.
struct RopeRows {
  int p[4];
  int64_t ro[4];
};

template <int EPI>
__device__ __forceinline__ void gather_rope_rows(RopeRows& rr, const RopeArgs& ra, int row4, int n) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    rr.p[r] = 0;
    rr.ro[r] = 0;
    if constexpr (EPI == kEpiRope) {
      const int row = row4 + r < n ? row4 + r : 0;
      rr.p[r] = rope_row_pos(ra, row);
      rr.ro[r] = rope_row_off(ra, row);
    }
  }
}

template <int EPI, int NT>
__device__ __forceinline__ void gather_rope(RopePre (&rp)[NT][4], const RopeArgs& ra, const RopeRows& rr, int g0,
                                            int tiles, int col) {
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    int dbase = 0, head = 0;
    if constexpr (EPI == kEpiRope) head = tile_head(ra, g0 + t < tiles ? g0 + t : tiles - 1, dbase);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      rp[t][r] = RopePre{1.f, 0.f, 0};
      if constexpr (EPI == kEpiRope) rp[t][r] = rope_pre(ra, rr.p[r], head, dbase + col, rr.ro[r]);
    }
  }
}

// A lane's rows row4 .. row4 + 3 of a folded norm pair's per-row scales
// (rows past n read row 0's; 1 without scales).
__device__ __forceinline__ void load_row_scales(float (&rsv)[4], const float* __restrict__ rscale, int row4, int n) {
#pragma unroll
  for (int r = 0; r < 4; ++r) rsv[r] = rscale ? rscale[row4 + r < n ? row4 + r : 0] : 1.f;
}

// Store of output (row, column c of tile g); `partner` is the value of column
// c ^ 1 (RoPE) or c ^ 8 (SwiGLU: the up value of gate column c < 8). Every
// lane fetches its partner before any lane branches here.
template <typename TO, int EPI>
__device__ __forceinline__ void store_out(TO* __restrict__ y, int64_t ldy, const RopeArgs& ra, int row, int g, int c,
                                          float v, float partner, const RopePre& rp) {
  if (EPI == kEpiSwiGLU) {
    if (c < 8) Elem<TO>::store(y + (int64_t)row * ldy + 8 * g + c, (v / (1.0f + expf(-v))) * partner);
  } else if (EPI == kEpiRope) {
    int dbase;
    const int head = tile_head(ra, g, dbase);
    store_rope<TO>(ra, rp, row, head, dbase + c, v, partner);
  } else {
    Elem<TO>::store(y + (int64_t)row * ldy + 16 * g + c, v);
  }
}

// Packed weights: element offset of lane `lane`'s fragment of (tile g, chunk
// p, step 0); step s adds s * 64 * V.
template <typename T>
__device__ __forceinline__ int64_t packed_off(int g, int p, int P, int lane) {
  return (((int64_t)g * P + p) * kChunkSteps * 64 + lane) * Chunk<T>::V;
}

template <typename T, int NT>
__device__ __forceinline__ void load_w(u32x4 (&wf)[NT][kChunkSteps], const T* const (&wtile)[NT], int P, int p,
                                       int lane) {
#pragma unroll
  for (int s = 0; s < kChunkSteps; ++s)
#pragma unroll
    for (int t = 0; t < NT; ++t)
      wf[t][s] = ld16(wtile[t] + packed_off<T>(0, p, P, lane) + (int64_t)s * 64 * Chunk<T>::V);
}

// Packing: one thread per 16-byte fragment, in packed order.
template <typename T, int EPI>
__global__ __launch_bounds__(256) void linear_pack_kernel(const T* __restrict__ W, T* __restrict__ Wp, int K,
                                                          int pair_off, int64_t nfrag) {
  constexpr int V = Chunk<T>::V;
  const int64_t f = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (f >= nfrag) return;
  const int P = K / Chunk<T>::KC;
  const int lane = (int)(f % 64);
  const int s = (int)((f / 64) % kChunkSteps);
  const int64_t gp = f / (64 * kChunkSteps);
  const int p = (int)(gp % P);
  const int g = (int)(gp / P);
  const int row = weight_row<EPI>(g, lane & 15, pair_off);
  const int64_t k = (int64_t)p * Chunk<T>::KC + s * Chunk<T>::KSTEP + (lane >> 4) * V;
  *reinterpret_cast<u32x4*>(Wp + f * V) = ld16(W + (int64_t)row * K + k);
}

// Coalesced x operand. An MFMA A fragment gives lane l row l % 16 and the
// 16-byte piece 4 s + l / 16 of that row's 256-byte chunk segment at step s,
// so a fragment load touches 16 rows x 64 bytes per instruction, which the
// memory pipeline serves at less than half the rate of whole segments (an
// L2-resident probe: ~55 against ~125 GB/s per CU). Instead a 16-row block's
// chunk is read as 4 loads of 4 whole segments -- load s: row r = 4 s + l / 16,
// piece (l % 16) ^ r -- stored to the wave's 4 KB of LDS as loaded (unit
// 64 s + l), and read back as fragments: lane l at step s reads unit
// 16 r' + ((4 s + l / 16) ^ r'), r' = l % 16, which holds row r', piece
// 4 s + l / 16. The XOR spreads both the stores and the fragment reads over
// all LDS banks. The fragments carry the same values in the same lanes as a
// direct fragment load, so the MFMAs and every bit of the result are the same.
constexpr int kXcUnits = 16 * 16;  // 16-byte units of a wave's LDS block: 16 rows x 16 pieces

// Byte offsets (chunk 0) of lane `lane`'s 4 coalesced loads for the 16-row
// block at `base` (kBufInvalid for rows at or past n: zeros, no traffic).
// Rows come from x_rows[base + r] when given, read with uniform scalar loads.
template <typename T>
__device__ __forceinline__ void xc_offsets(uint32_t (&off)[kChunkSteps], const int32_t* __restrict__ x_rows,
                                           int64_t ldx, int base, int lane, int n) {
  const int m = n - base < 16 ? n - base : 16;
  int rv[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) rv[j] = base + j;
  if (x_rows && m > 0) {
#pragma unroll
    for (int j = 0; j < 16; ++j) rv[j] = x_rows[base + (j < m ? j : 0)];
  }
#pragma unroll
  for (int s = 0; s < kChunkSteps; ++s) {
    const int r = 4 * s + (lane >> 4);
    int row = rv[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) row = r == j ? rv[j] : row;
    const int q = (lane & 15) ^ r;
    off[s] = r < m ? (uint32_t)(((int64_t)row * ldx + q * Chunk<T>::V) * sizeof(T)) : kBufInvalid;
  }
}

template <typename T>
__device__ __forceinline__ void load_xc(u32x4 (&xc)[kChunkSteps], __amdgpu_buffer_rsrc_t xr,
                                        const uint32_t (&off)[kChunkSteps], int p) {
  const uint32_t co = (uint32_t)(p * Chunk<T>::KC * sizeof(T));  // kBufInvalid + co stays out of range
#pragma unroll
  for (int s = 0; s < kChunkSteps; ++s) xc[s] = buf_ld16(xr, off[s] + co);
}

// Other lanes read what a lane stored: keep the compiler from moving LDS
// accesses across this point (the LDS executes one wave's accesses in order).
__device__ __forceinline__ void lds_order() { asm volatile("" ::: "memory"); }

__device__ __forceinline__ void xc_store(u32x4* __restrict__ xl, const u32x4 (&xc)[kChunkSteps], int lane) {
  lds_order();  // after the previous chunk's fragment reads
#pragma unroll
  for (int s = 0; s < kChunkSteps; ++s) xl[64 * s + lane] = xc[s];
  lds_order();  // before this chunk's fragment reads
}

__device__ __forceinline__ u32x4 xc_frag(const u32x4* __restrict__ xl, int st, int lane) {
  const int r = lane & 15;
  return xl[16 * r + ((4 * st + (lane >> 4)) ^ r)];
}

__device__ __forceinline__ void xc_frags(u32x4 (&xf)[kChunkSteps], const u32x4* __restrict__ xl, int lane) {
#pragma unroll
  for (int st = 0; st < kChunkSteps; ++st) xf[st] = xc_frag(xl, st, lane);
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
// wide: grid (tiles << HALF), WW waves (16, or 8 for launches of more tiles
// than 1024-thread workgroups can keep resident at once: two per CU). Wave w
// owns sub-slice w of the contract (with 8 waves also w + 8): RM >= R chunks
// per sub-slice, summed in chunk order in registers, so each wave parks one
// f32x4 per sub-slice in LDS and the tile's 16 sub-slice sums are added by
// threads 0..255 in contract order (the chunk layout over waves changes no
// bits). HALF: two workgroups per tile, each owning 8 of its 16 columns (its
// other lanes load zero weights through an invalid buffer offset: no memory
// traffic), so a 2048-column projection spreads over 256 workgroups instead
// of 128. The MFMA output of a column does not depend on the other columns'
// operands, so both forms give the same bits.
// The consumer side of a folded norm pair in the few-row kernel (rs.part: each
// row's group sums, reduced by the row's wave; rs.scale: the scales
// precomputed): issued first, so their loads are the oldest of the launch.

// The producer side (EPI == kEpiPrep): thread (ln, r) of the epilogue owns
// output (row 4 (ln / 16) + r, column 16 g + ln % 16); the operands of its
// element, fetched at launch.
struct PrepPre {
  float rin, sin, win, wa, wb;
};

template <typename T, typename TO, int EPI, int RM, bool HALF, int WW>
__global__ __launch_bounds__(64 * WW) __attribute__((amdgpu_waves_per_eu(WW == 8 && EPI != kEpiRope ? 6 : 1))) void linear_wide_kernel(
    const T* __restrict__ x, const int32_t* __restrict__ x_rows, int64_t ldx, const T* __restrict__ W,
    TO* __restrict__ y, int64_t ldy, int n, int K, int pair_off, const RopeArgs ra, const TileArgmax am,
    const wfd_rowscale_t rs, const wfd_prep_t pp) {
  constexpr int KPW = kSlices * kSubSlices / WW;  // sub-slices per wave
  static_assert(KPW * WW == kSlices * kSubSlices, "16 or 8 waves");
  __shared__ f32x4 red[kSlices * kSubSlices][64];  // sub-slice sums [sub-slice][lane]
  __shared__ __align__(16) u32x4 xl[WW][kXcUnits];  // each wave's x chunk (coalesced load -> fragments)
  __shared__ float rsc[kWideMaxRows];               // the rows' scales (rs.part)
  // folded norm pair, consumer side: row `wave`'s group sums (rs.part) or
  // this epilogue thread's row scale (rs.scale), loaded before anything else
  const bool by_part = EPI != kEpiPrep && rs.part != nullptr;
  constexpr int RPW = kWideMaxRows / WW;  // rows whose sums a wave reduces: wave, wave + WW
  // 16 waves: the group sums are loaded at launch, ahead of the main loop's
  // loads (behind them, the launch at 8 rows took 9.4 against 8.7 us), and
  // held through its MFMAs; 8 waves (three workgroups per CU by LDS, a
  // register budget of 80, which even one early row per wave would exceed)
  // load them after the loop, one more round trip
  constexpr bool kEarlyGroups = WW == kWideWaves;
  float4 gpv[RPW][2];
  float esc = 1.f;
  auto load_groups = [&](int q0, int q1) {
    const int wv = threadIdx.x >> 6;
    const int PD = rs.D / LinTraits<T>::KC;  // chunks of a row of r
#pragma unroll
    for (int q = q0; q < q1; ++q) {
      const int rw = wv + WW * q;
      if (by_part && rw < n)  // uniform over the wave
        fold_load<T>(gpv[q], reinterpret_cast<const float2*>(rs.part) + (int64_t)rw * kFoldSlots,
                     threadIdx.x & 63, PD);
    }
  };
  {
    if constexpr (kEarlyGroups) load_groups(0, RPW);
    if (EPI != kEpiPrep && rs.scale != nullptr && threadIdx.x < 256) {
      const int orow = 4 * ((threadIdx.x >> 2) >> 4) + (threadIdx.x & 3);
      esc = rs.scale[orow < n ? orow : 0];
    }
  }
  constexpr int V = LinTraits<T>::V;
  const int P = K / LinTraits<T>::KC;
  const int Q = slice_chunks(P);
  const int R = sub_chunks(P);
  const int g = HALF ? blockIdx.x >> 1 : blockIdx.x;
  const int half = HALF ? (int)(blockIdx.x & 1) : 0;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;

  uint32_t xoff[kChunkSteps];
  xc_offsets<T>(xoff, x_rows, ldx, 0, lane, n);
  const __amdgpu_buffer_rsrc_t xrs = buf_rsrc(x);
  const T* const wtile[1] = {W + packed_off<T>(g, 0, P, 0)};
  const __amdgpu_buffer_rsrc_t wrs = buf_rsrc(wtile[0]);
  // the RoPE epilogue's table operands of this thread's output, fetched at
  // launch so the epilogue waits on no load
  RopePre rp{1.f, 0.f, 0};
  if constexpr (EPI == kEpiRope) {
    if (threadIdx.x < 256) {
      const int orow = 4 * ((threadIdx.x >> 2) >> 4) + (threadIdx.x & 3);
      const int row = orow < n ? orow : 0;
      int dbase;
      const int head = tile_head(ra, g, dbase);
      rp = rope_pre(ra, rope_row_pos(ra, row), head, dbase + ((threadIdx.x >> 2) & 15), rope_row_off(ra, row));
    }
  }
  PrepPre pq{0.f, 1.f, 1.f, 1.f, 1.f};
  if constexpr (EPI == kEpiPrep) {
    if (threadIdx.x < 256) {
      const int orow = 4 * ((threadIdx.x >> 2) >> 4) + (threadIdx.x & 3);
      const int row = orow < n ? orow : 0;
      const int k = 16 * g + ((threadIdx.x >> 2) & 15);
      if (pp.r_in) pq.rin = Elem<T>::load((const T*)pp.r_in + (int64_t)row * pp.ld_in + k);
      if (pp.s_in) pq.sin = pp.s_in[row];
      if (pp.w_in) pq.win = Elem<T>::load((const T*)pp.w_in + k);
      if (pp.wa) pq.wa = Elem<T>::load((const T*)pp.wa + k);
      pq.wb = Elem<T>::load((const T*)pp.wb + k);
    }
  }

  // Sub-slice k = 4 q + u covers chunks [c0, c1) of slice q; an empty one
  // (past the last chunk) sums to +0. Every load is unconditional: a chunk
  // slot past the sub-slice's end re-reads chunk P-1 and is not added.
  int c0[KPW], c1[KPW];
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    const int k = wave + WW * i;
    const int q = k / kSubSlices, u = k % kSubSlices;
    const int se = (q + 1) * Q < P ? (q + 1) * Q : P;
    c0[i] = q * Q + u * R;
    c1[i] = c0[i] + R < se ? c0[i] + R : se;
  }
  u32x4 wf[KPW][RM][1][kChunkSteps];
  u32x4 xf[KPW][RM][kChunkSteps];
#pragma unroll
  for (int i = 0; i < KPW; ++i)
#pragma unroll
    for (int j = 0; j < RM; ++j) {
      const int p = c0[i] + j;
      const int pc = p < c1[i] ? p : P - 1;
      if (HALF) {
        const bool mine = (col >> 3) == half;
#pragma unroll
        for (int s2 = 0; s2 < kChunkSteps; ++s2) {
          const uint32_t off = (uint32_t)((packed_off<T>(0, pc, P, lane) + (int64_t)s2 * 64 * V) * sizeof(T));
          wf[i][j][0][s2] = buf_ld16(wrs, mine ? off : kBufInvalid);
        }
      } else {
        load_w<T, 1>(wf[i][j], wtile, P, pc, lane);
      }
      load_xc<T>(xf[i][j], xrs, xoff, pc);
    }
#pragma unroll
  for (int i = 0; i < KPW; ++i) {
    f32x4 sub = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < RM; ++j) {
      if (c0[i] + j < c1[i]) {  // uniform
        // the chunk's x fragments through the wave's LDS block
        u32x4 xa[kChunkSteps];
        xc_store(xl[wave], xf[i][j], lane);
        xc_frags(xa, xl[wave], lane);
        f32x4 acc[1];
        chunk_mma<T, 1>(acc, xa, wf[i][j]);
#pragma unroll
        for (int r = 0; r < 4; ++r) sub[r] += acc[0][r];
      }
    }
    red[wave + WW * i][lane] = sub;
  }
  if constexpr (!kEarlyGroups) load_groups(0, RPW);
#pragma unroll
  for (int q = 0; q < RPW; ++q) {
    const int rw = wave + WW * q;
    if (by_part && rw < n) {  // row rw's scale from its group sums (uniform over the wave)
      float sr, su;
      fold_sums4(gpv[q], sr, su);
      float s_a, scale;
      pair_scale(sr, su, rs.D, rs.eps, rs.two != 0, s_a, scale);
      if (lane == 0) {
        rsc[rw] = scale;
        if (rs.s_out && blockIdx.x == 0) rs.s_out[rw] = s_a;
      }
    }
  }
  __syncthreads();

  // threads 0..255: one (lane', r) output each, the 16 sub-slice sums added
  // sub-slice by sub-slice within each slice, then slice by slice
  if (threadIdx.x < 256) {
    const int ln = threadIdx.x >> 2;
    const int r = threadIdx.x & 3;
    const int row = 4 * (ln >> 4) + r;
    float us[kSlices * kSubSlices];
#pragma unroll
    for (int k = 0; k < kSlices * kSubSlices; ++k) us[k] = red[k][ln][r];
    float v = 0.f;
#pragma unroll
    for (int q = 0; q < kSlices; ++q) {
      float sl = 0.f;
#pragma unroll
      for (int u = 0; u < kSubSlices; ++u) sl += us[q * kSubSlices + u];
      v += sl;
    }
    if (by_part) v = mul_rn(v, rsc[row < n ? row : 0]);  // a folded norm pair's row scale
    else if (EPI != kEpiPrep && rs.scale != nullptr) v = mul_rn(v, esc);
    const bool mine = !HALF || ((ln & 15) >> 3) == half;
    if constexpr (EPI == kEpiPrep) {
      // the residual stream, the next linear's operand and the row's sums per
      // 8-column group: the group's columns are threads ^ 4, ^ 8, ^ 16 (column
      // bits 0, 1, 2), added as ((c0+c1)+(c2+c3))+((c4+c5)+(c6+c7))
      const PrepVal pv = prep_value<T>(v, pp.r_in != nullptr, pq.rin, pq.sin, pq.win, pq.wa, pq.wb);
      float tr = pv.sr, tu = pv.su;
#pragma unroll
      for (int m = 4; m <= 16; m <<= 1) {
        tr = add_rn(tr, __shfl_xor(tr, m, 64));
        tu = add_rn(tu, __shfl_xor(tu, m, 64));
      }
      if (row < n && mine) {
        const int k = 16 * g + (ln & 15);
        if (pp.r_out) Elem<T>::store((T*)pp.r_out + (int64_t)row * pp.ld_out + k, pv.r);
        if (pp.a_out) Elem<T>::store((T*)pp.a_out + (int64_t)row * pp.ld_a + k, pv.A);
        if ((k & 7) == 0 && pp.part)
          reinterpret_cast<float2*>(pp.part)[(int64_t)row * kFoldSlots + fold_slot<T>(k >> 3)] = float2{tr, tu};
      }
      return;
    }
    // column ln ^ 1 lives in thread threadIdx.x ^ 4, column ln ^ 8 in threadIdx.x ^ 32
    const float partner = EPI == kEpiRope     ? __shfl_xor(v, 4, 64)
                          : EPI == kEpiSwiGLU ? __shfl_xor(v, 32, 64)
                                              : 0.f;
    if (row < n && mine) store_out<TO, EPI>(y, ldy, ra, row, g, ln & 15, v, partner, rp);
    if constexpr (EPI == kEpiPlain && std::is_same<TO, float>::value) {
      if (am.val) {  // uniform
        // a row's 16 columns sit in lanes 4 c + r of this wave (c = ln & 15)
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        if (mine) argmax_merge(bv, bi, v, 16 * g + (ln & 15));
#pragma unroll
        for (int m = 4; m < 64; m <<= 1) {
          const float ov = __shfl_xor(bv, m, 64);
          const int oi = __shfl_xor(bi, m, 64);
          argmax_merge(bv, bi, ov, oi);
        }
        if (row < n && (ln & 15) == 0) {
          am.val[(int64_t)row * gridDim.x + blockIdx.x] = bv;
          am.idx[(int64_t)row * gridDim.x + blockIdx.x] = bi;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// tile: grid (ceil(n/64), ceil(tiles/NB)), 256 threads; wave = 16 rows of x,
// NB weight tiles per workgroup.
template <typename T, typename TO, int EPI, int NB>
__global__ __launch_bounds__(256) void linear_tile_kernel(const T* __restrict__ x, const int32_t* __restrict__ x_rows,
                                                          int64_t ldx, const T* __restrict__ W, TO* __restrict__ y,
                                                          int64_t ldy, int n, int K, int pair_off, int tiles,
                                                          const RopeArgs ra, const float* __restrict__ rscale) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int row0 = (blockIdx.x * 4 + wave) * 16;
  if (row0 >= n) return;  // no barriers in this kernel
  float rsv[4];
  load_row_scales(rsv, rscale, row0 + 4 * grp, n);
  const int P = K / LinTraits<T>::KC;
  __shared__ __align__(16) u32x4 xl[4][kXcUnits];  // each wave's x chunk (coalesced load -> fragments)
  uint32_t xoff[kChunkSteps];
  xc_offsets<T>(xoff, x_rows, ldx, row0, lane, n);
  const __amdgpu_buffer_rsrc_t xrs = buf_rsrc(x);

  const T* wtile[NB];
  bool gok[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    const int g = blockIdx.y * NB + b;
    gok[b] = g < tiles;
    wtile[b] = W + packed_off<T>(gok[b] ? g : 0, 0, P, 0);
  }

  // the RoPE epilogue's per-row operands (position, cache offset) are
  // fetched at launch, the cos / sin pairs after the main loop (at 64 rows
  // 15.4 us against 16.9 with every operand at launch, held through the loop)
  RopeRows rrows;
  gather_rope_rows<EPI>(rrows, ra, row0 + 4 * grp, n);

  // two-stage register pipeline; every load is unconditional (the stage past
  // the last chunk re-reads chunk P-1 and is never used)
  SliceWalk walk(P, 0);
  f32x4 tot[NB], sl[NB], sub[NB];
#pragma unroll
  for (int c = 0; c < NB; ++c) tot[c] = sl[c] = sub[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto add = [&](const f32x4 (&acc)[NB], int p) { contract_add<NB>(sub, sl, tot, acc, walk.end(p)); };
  u32x4 wa[NB][kChunkSteps], wb[NB][kChunkSteps], xa[kChunkSteps], xb[kChunkSteps];
  // chunk partials from coalesced x (through the wave's LDS block)
  auto mma = [&](f32x4 (&acc)[NB], const u32x4 (&xc)[kChunkSteps], const u32x4 (&wr)[NB][kChunkSteps]) {
    u32x4 xf[kChunkSteps];
    xc_store(xl[wave], xc, lane);
    xc_frags(xf, xl[wave], lane);
    chunk_mma<T, NB>(acc, xf, wr);
  };
  load_w<T, NB>(wa, wtile, P, 0, lane);
  load_xc<T>(xa, xrs, xoff, 0);
  for (int p = 0; p < P; p += 2) {
    const int p1 = p + 1 < P ? p + 1 : P - 1;
    load_w<T, NB>(wb, wtile, P, p1, lane);
    load_xc<T>(xb, xrs, xoff, p1);
    f32x4 acc[NB];
    mma(acc, xa, wa);
    add(acc, p);
    if (p + 1 >= P) break;
    const int p2 = p + 2 < P ? p + 2 : P - 1;
    load_w<T, NB>(wa, wtile, P, p2, lane);
    load_xc<T>(xa, xrs, xoff, p2);
    mma(acc, xb, wb);
    add(acc, p + 1);
  }
  RopePre rp[NB][4];
  gather_rope<EPI, NB>(rp, ra, rrows, blockIdx.y * NB, tiles, col);
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (!gok[b]) continue;  // uniform over the workgroup
    const int g = blockIdx.y * NB + b;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int orow = row0 + 4 * grp + r;
      const float v = rscale ? mul_rn(tot[b][r], rsv[r]) : tot[b][r];  // a folded norm pair's row scale
      // column col ^ 1 lives in lane ^ 1, column col ^ 8 in lane ^ 8 (the whole wave takes part)
      const float partner = EPI == kEpiRope     ? __shfl_xor(v, 1, 64)
                            : EPI == kEpiSwiGLU ? __shfl_xor(v, 8, 64)
                                                : 0.f;
      if (orow < n) store_out<TO, EPI>(y, ldy, ra, orow, g, col, v, partner, rp[b][r]);
    }
  }
}

// ---------------------------------------------------------------------------
// XCD-aware work mapping for the many-row kernels. Workgroups are handed to
// the 8 XCDs round-robin by linear id, and each XCD has its own L2. The row
// blocks that share a group of weight tiles are put on one XCD, so the group's
// weights cross the fabric once and the other row blocks read them from that
// XCD's L2 (with the plain 2-D grid they land on R different XCDs and every
// weight byte crosses the fabric R = ceil(n / 64) times). Linear id i:
// XCD i % 8, j = i / 8, row block j % R, tile group (j / R) * 8 + i % 8; the
// grid is R x (tile groups rounded up to 8) and the padding ids return.
constexpr int kXcds = 8;

__host__ __device__ constexpr int xcd_grid(int rb, int groups) {
  return rb * ((groups + kXcds - 1) / kXcds) * kXcds;
}

// Tiles per workgroup of a slice launch (2 or 4; S = K slices in grid y).
// Each workgroup moves 64 rows x 128 K of x (16 KB) and BT x 4 KB of weights
// per chunk, and the XCD-aware grid spreads the workgroups evenly over the 8
// XCDs of 32 CUs, so the busiest CU streams ceil(workgroups / 256) of them:
// the choice minimizes that product (ties: fewer tiles). Eight tiles per
// workgroup (one workgroup per CU by registers) were faster at 192-512 rows
// with fragment loads of x, and slower than four once x is coalesced
// (proj / mlp_proj / adapter at 512 rows: 18.0 / 28.8 / 24.4 -> 14.4 / 25.2 /
// 21.0 us).
constexpr int kCusPerXcd = 32;

static int gemm_tiles_per_workgroup(int rb, int tiles, int S) {
  int best = 2;
  long best_cost = -1;
  for (int bt = 2; bt <= 4; bt *= 2) {
    const long wgs = (long)xcd_grid(rb, (tiles + bt - 1) / bt) * S;
    const long per_cu = ((wgs + kXcds - 1) / kXcds + kCusPerXcd - 1) / kCusPerXcd;
    const long cost = per_cu * (16 + 4 * bt);
    if (best_cost < 0 || cost < best_cost) {
      best_cost = cost;
      best = bt;
    }
  }
  return best;
}

template <int BT>
__device__ __forceinline__ bool xcd_block(int n, int tiles, int& rbk, int& tg) {
  const int R = (n + 63) / 64;
  const int i = blockIdx.x;
  const int j = i / kXcds;
  rbk = j % R;
  tg = (j / R) * kXcds + i % kXcds;
  return tg * BT < tiles;
}

// gemm: grid xcd_grid(ceil(n/64), ceil(tiles/BT)), 256 threads; wave = 16 rows of x,
// workgroup = 64 rows x BT weight tiles. Each chunk's BT weight tiles go
// through LDS once (double-buffered) and all 4 waves read them there, so a
// weight byte crosses L2 once per 64 rows instead of once per 16. Weights and
// x are loaded into registers two chunks ahead of their use, so a chunk's
// memory latency overlaps the MFMAs of the two before it. Same per-chunk
// arithmetic as the wide and tile kernels, so the same bits.
//
// PART (the slice form behind wfd_linear_partials): grid y = slice; the
// workgroup walks only its slice's chunks and stores the fp32 slice partial of
// every (row, column) at part[(slice * n + row) * 16 * tiles + column], with no
// epilogue. Adding the slices in slice order from zero gives the bits of a
// launch that walks all of K.
template <typename T, typename TO, int EPI, int BT, bool PART>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void linear_gemm_kernel(const T* __restrict__ x, const int32_t* __restrict__ x_rows,
                                                          int64_t ldx, const T* __restrict__ W, TO* __restrict__ y,
                                                          int64_t ldy, int n, int K, int pair_off, int tiles,
                                                          const RopeArgs ra, float* __restrict__ part,
                                                          const float* __restrict__ rscale) {
  constexpr int V = LinTraits<T>::V;
  constexpr int FR = BT * kChunkSteps;  // 1 KB fragments per chunk: (tile, step)
  constexpr int FPW = FR / 4;           // fragments each wave stages per chunk
  __shared__ __align__(16) u32x4 wl[2][FR][64];
  __shared__ __align__(16) u32x4 xl[4][kXcUnits];  // each wave's x chunk (coalesced load -> fragments)
  int rbk, tg;
  if (!xcd_block<BT>(n, tiles, rbk, tg)) return;  // padding workgroup (uniform, before any barrier)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int row0 = (rbk * 4 + wave) * 16;
  const int P = K / LinTraits<T>::KC;
  const int Q = slice_chunks(P);
  // chunks [pb, pe): all of K, or the slice of this workgroup
  const int pb = PART ? (int)blockIdx.y * Q : 0;
  const int pe = PART ? min(P, pb + Q) : P;
  // a wave past the last row still stages weights and meets every barrier;
  // its x loads read zeros (no memory traffic), it runs no MFMA and stores
  // nothing
  uint32_t xoff[kChunkSteps];
  if (row0 < n) {
    xc_offsets<T>(xoff, x_rows, ldx, row0, lane, n);
  } else {
#pragma unroll
    for (int s = 0; s < kChunkSteps; ++s) xoff[s] = kBufInvalid;
  }
  const __amdgpu_buffer_rsrc_t xrs = buf_rsrc(x);
  auto load_xs = [&](u32x4 (&xr)[kChunkSteps], int p) { load_xc<T>(xr, xrs, xoff, p); };

  // the fragments this wave stages: f = wave * FPW + i -> (tile f / 4, step f % 4)
  const T* wsrc[FPW];
#pragma unroll
  for (int i = 0; i < FPW; ++i) {
    const int f = wave * FPW + i;
    const int g = tg * BT + f / kChunkSteps;
    wsrc[i] = W + packed_off<T>(g < tiles ? g : tiles - 1, 0, P, lane) + (int64_t)(f % kChunkSteps) * 64 * V;
  }
  const int64_t pstride = (int64_t)kChunkSteps * 64 * V;  // elements from one chunk to the next in a tile
  // every load unconditional: chunks past the last re-read it, never used
  auto cl = [&](int p) { return p < pe ? p : pe - 1; };
  auto fetch_w = [&](u32x4 (&wr)[FPW], int p) {
#pragma unroll
    for (int i = 0; i < FPW; ++i) wr[i] = ld16(wsrc[i] + cl(p) * pstride);
  };
  auto stage_w = [&](const u32x4 (&wr)[FPW], int b) {
#pragma unroll
    for (int i = 0; i < FPW; ++i) wl[b][wave * FPW + i][lane] = wr[i];
  };
  // with 2 tiles the RoPE epilogue's operands are gathered at launch (the
  // tail then waits on no dependent loads: at 128 rows 17.7 us against 18.4
  // with the cos / sin pairs after the loop); with 4 the main loop has no
  // registers to spare for them, so they follow it
  constexpr bool kRopeEarly = BT <= 2;
  float rsv[4];  // folded norm pairs' row scales: early with the RoPE operands, else after the loop
  if constexpr (kRopeEarly) load_row_scales(rsv, PART ? nullptr : rscale, row0 + 4 * grp, n);
  RopeRows rrows;
  RopePre rp[BT][4];
  if constexpr (kRopeEarly) {
    gather_rope_rows<EPI>(rrows, ra, row0 + 4 * grp, n);
    gather_rope<EPI, BT>(rp, ra, rrows, tg * BT, tiles, col);
  }
  SliceWalk walk(P, pb);
  f32x4 tot[BT], sl[BT], sub[BT];
#pragma unroll
  for (int t = 0; t < BT; ++t) tot[t] = sl[t] = sub[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  // chunk p (coalesced x in xr, through the wave's LDS block; weights in LDS
  // stage b): its partial into the contract's running sums
  auto mma = [&](const u32x4 (&xr)[kChunkSteps], int b, int p) {
    if (row0 >= n) return;  // a wave without rows only stages weights (uniform over the wave)
    xc_store(xl[wave], xr, lane);
    auto xfrag = [&](int st) { return xc_frag(xl[wave], st, lane); };
    f32x4 acc[BT];
#pragma unroll
    for (int t = 0; t < BT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // step st's x and weight fragments are read from LDS while step st - 1's MFMAs run
    u32x4 wf[2][BT], xf[2];
    xf[0] = xfrag(0);
#pragma unroll
    for (int t = 0; t < BT; ++t) wf[0][t] = wl[b][t * kChunkSteps][lane];
#pragma unroll
    for (int st = 0; st < kChunkSteps; ++st) {
      if (st + 1 < kChunkSteps) {
        xf[(st + 1) & 1] = xfrag(st + 1);
#pragma unroll
        for (int t = 0; t < BT; ++t) wf[(st + 1) & 1][t] = wl[b][t * kChunkSteps + st + 1][lane];
      }
#pragma unroll
      for (int t = 0; t < BT; ++t) acc[t] = mfma_step<T>(xf[st & 1], wf[st & 1][t], acc[t]);
    }
    contract_add<BT>(sub, sl, tot, acc, walk.end(p));
  };

  // Register rings, statically unrolled by two (no copies, no exit inside
  // the loop): chunk q's weights are fetched two half-iterations before they
  // are staged into LDS stage q & 1, and its x two half-iterations before
  // its MFMAs. Issue order at the top of every pair, oldest first:
  // x0 (chunk p), w1 (p + 1), x1 (p + 1), w0 (p + 2); the prologue builds
  // the same order so the compiler's wait counts are the steady-state ones.
  u32x4 w0[FPW], w1[FPW], x0[kChunkSteps], x1[kChunkSteps];
  fetch_w(w0, pb);
  load_xs(x0, pb);
  fetch_w(w1, pb + 1);
  load_xs(x1, cl(pb + 1));
  stage_w(w0, 0);
  __syncthreads();
  fetch_w(w0, pb + 2);
  for (int p = pb; p + 1 < pe; p += 2) {
    // chunk p: LDS stage 0, x0
    mma(x0, 0, p);
    load_xs(x0, cl(p + 2));
    stage_w(w1, 1);  // chunk p + 1; stage 1 was last read by chunk p - 1, before the previous barrier
    __syncthreads();
    fetch_w(w1, p + 3);
    // chunk p + 1: LDS stage 1, x1
    mma(x1, 1, p + 1);
    load_xs(x1, cl(p + 3));
    stage_w(w0, 0);  // chunk p + 2; stage 0 was last read by chunk p, before the barrier above
    __syncthreads();
    fetch_w(w0, p + 4);
  }
  if ((pe - pb) & 1) mma(x0, 0, pe - 1);  // the last chunk, staged by the last pair (or the prologue)
  if (row0 >= n) return;  // after the last barrier
  if constexpr (PART) {
    const int N = 16 * tiles;
#pragma unroll
    for (int t = 0; t < BT; ++t) {
      const int g = tg * BT + t;
      if (g >= tiles) continue;  // uniform over the workgroup
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int orow = row0 + 4 * grp + r;
        if (orow < n) part[((int64_t)blockIdx.y * n + orow) * N + 16 * g + col] = tot[t][r];  // == the slice sum
      }
    }
    return;
  }
  if constexpr (!kRopeEarly) {
    load_row_scales(rsv, rscale, row0 + 4 * grp, n);
    gather_rope_rows<EPI>(rrows, ra, row0 + 4 * grp, n);
    gather_rope<EPI, BT>(rp, ra, rrows, tg * BT, tiles, col);
  }
#pragma unroll
  for (int t = 0; t < BT; ++t) {
    const int g = tg * BT + t;
    if (g >= tiles) continue;  // uniform over the workgroup
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int orow = row0 + 4 * grp + r;
      const float v = rscale ? mul_rn(tot[t][r], rsv[r]) : tot[t][r];  // a folded norm pair's row scale
      // column col ^ 1 lives in lane ^ 1, column col ^ 8 in lane ^ 8 (the whole wave takes part)
      const float partner = EPI == kEpiRope     ? __shfl_xor(v, 1, 64)
                            : EPI == kEpiSwiGLU ? __shfl_xor(v, 8, 64)
                                                : 0.f;
      if (orow < n) store_out<TO, EPI>(y, ldy, ra, orow, g, col, v, partner, rp[t][r]);
    }
  }
}

// ---------------------------------------------------------------------------
// stream: grid (ceil(n/64), ceil(tiles/BT)), 256 threads; wave = 16 rows of x,
// workgroup = 64 rows x BT weight tiles. Weights and x move global -> LDS
// with the 16-byte direct-to-LDS load (lane l's 16 bytes land at the wave's
// LDS base + 16 l), NS - 1 chunks ahead of the MFMAs, through a ring of NS
// LDS stages: no registers hold data in flight, so the depth of the pipeline
// costs LDS, not VGPRs, and a K-sequential workgroup keeps NS - 1 chunks of
// loads outstanding instead of paying the memory latency once per chunk. The
// weight tiles of a stage are read by all 4 waves; each wave reads only its
// own x rows. Same per-chunk arithmetic as the other kernels, same bits.
//
// Ordering (per wave; vector-memory loads complete in issue order): before
// the barrier of chunk p a wave waits until only the loads of the chunks
// after p remain; the barrier then publishes every wave's chunk p, and
// retires every wave's reads of chunk p - 1, whose stage the loads of chunk
// p + NS - 1 issued right after it overwrite.
// The loads are issued through inline assembly so that the compiler, which
// does not know they write LDS, adds no wait of its own before the LDS reads
// (it would wait for every outstanding load); the waits are the explicit ones
// below. M0 holds the wave's LDS byte address; one wait state separates its
// write from the load that reads it.
__device__ __forceinline__ void load16_lds(const void* src, const u32x4* lds_wave_base) {
  const uint32_t m0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds_wave_base;
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(src) : "memory", "m0");
}

// Wait until at most N of this wave's loads are outstanding and its LDS reads
// have completed, then the workgroup barrier.
template <int N>
__device__ __forceinline__ void wait_vmem_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// The stream kernel's coalesced x sources: a direct-to-LDS load puts lane l's
// 16 bytes at unit 64 s + l of the wave's block, so load s of lane l reads
// row r = 4 s + l / 16, piece (l % 16) ^ r -- the layout xc_frag reads.
// Rows at or past n read the block's first row: they fill fragment rows whose
// results are never stored.
template <typename T>
__device__ __forceinline__ void xc_ptrs(const T* (&src)[kChunkSteps], const T* __restrict__ x,
                                        const int32_t* __restrict__ x_rows, int64_t ldx, int base, int lane, int n) {
  const int m = n - base < 16 ? n - base : 16;  // >= 1: the wave has rows
  int rv[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) rv[j] = x_rows ? x_rows[base + (j < m ? j : 0)] : base + (j < m ? j : 0);
#pragma unroll
  for (int s = 0; s < kChunkSteps; ++s) {
    const int r = 4 * s + (lane >> 4);
    int row = rv[0];
#pragma unroll
    for (int j = 1; j < 16; ++j) row = r == j ? rv[j] : row;
    src[s] = x + (int64_t)row * ldx + ((lane & 15) ^ r) * Chunk<T>::V;
  }
}

template <typename T, typename TO, int EPI, int BT, int NS>
__global__ __launch_bounds__(256) void linear_stream_kernel(const T* __restrict__ x, const int32_t* __restrict__ x_rows,
                                                            int64_t ldx, const T* __restrict__ W, TO* __restrict__ y,
                                                            int64_t ldy, int n, int K, int pair_off, int tiles,
                                                            const RopeArgs ra, const float* __restrict__ rscale) {
  constexpr int V = LinTraits<T>::V;
  constexpr int KC = LinTraits<T>::KC;
  constexpr int FR = BT * kChunkSteps;   // weight fragments (tile, step) per chunk, 1 KB each
  constexpr int FPW = BT;                // of which each wave loads FR / 4
  constexpr int LW = FPW;                // loads per chunk of a wave without rows
  constexpr int LX = FPW + kChunkSteps;  // ... and of a wave with rows
  __shared__ __align__(16) u32x4 wst[NS][FR][64];
  __shared__ __align__(16) u32x4 xst[NS][4][kChunkSteps][64];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int row0 = (blockIdx.x * 4 + wave) * 16;
  const bool rows = row0 < n;  // uniform over the wave
  const int P = K / KC;
  const T* xsrc[kChunkSteps] = {x, x, x, x};
  if (rows) xc_ptrs<T>(xsrc, x, x_rows, ldx, row0, lane, n);
  const T* wsrc[FPW];
#pragma unroll
  for (int i = 0; i < FPW; ++i) {
    const int f = wave * FPW + i;
    const int g = blockIdx.y * BT + f / kChunkSteps;
    wsrc[i] = W + packed_off<T>(g < tiles ? g : tiles - 1, 0, P, lane) + (int64_t)(f % kChunkSteps) * 64 * V;
  }
  const int64_t pstride = (int64_t)kChunkSteps * 64 * V;
  auto issue = [&](int p) {
    const int st = p % NS;
#pragma unroll
    for (int i = 0; i < FPW; ++i) load16_lds(wsrc[i] + p * pstride, &wst[st][wave * FPW + i][0]);
    if (rows) {
#pragma unroll
      for (int s = 0; s < kChunkSteps; ++s) load16_lds(xsrc[s] + (int64_t)p * KC, &xst[st][wave][s][0]);
    }
  };
#pragma unroll
  for (int u = 0; u < NS - 1; ++u)
    if (u < P) issue(u);

  SliceWalk walk(P, 0);
  f32x4 tot[BT], sl[BT], sub[BT];
#pragma unroll
  for (int t = 0; t < BT; ++t) tot[t] = sl[t] = sub[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int p = 0; p < P; ++p) {
    // this wave's chunk p is in LDS once at most the later chunks' loads are outstanding
    if (p + NS - 2 < P) {
      if (rows) wait_vmem_barrier<(NS - 2) * LX>();
      else wait_vmem_barrier<(NS - 2) * LW>();
    } else {
      wait_vmem_barrier<0>();
    }
    if (p + NS - 1 < P) issue(p + NS - 1);
    if (rows) {
      const int st = p % NS;
      f32x4 acc[BT];
#pragma unroll
      for (int t = 0; t < BT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < kChunkSteps; ++s) {
        const u32x4 xf = xc_frag(&xst[st][wave][0][0], s, lane);
#pragma unroll
        for (int t = 0; t < BT; ++t) acc[t] = mfma_step<T>(xf, wst[st][t * kChunkSteps + s][lane], acc[t]);
      }
      contract_add<BT>(sub, sl, tot, acc, walk.end(p));
    }
  }
  if (!rows) return;  // after the last barrier; every load of this wave has completed
  float rsv[4];
  load_row_scales(rsv, rscale, row0 + 4 * grp, n);
  RopeRows rrows;
  gather_rope_rows<EPI>(rrows, ra, row0 + 4 * grp, n);
  RopePre rp[BT][4];
  gather_rope<EPI, BT>(rp, ra, rrows, blockIdx.y * BT, tiles, col);
#pragma unroll
  for (int t = 0; t < BT; ++t) {
    const int g = blockIdx.y * BT + t;
    if (g >= tiles) continue;  // uniform over the workgroup
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int orow = row0 + 4 * grp + r;
      const float v = rscale ? mul_rn(tot[t][r], rsv[r]) : tot[t][r];  // a folded norm pair's row scale
      // column col ^ 1 lives in lane ^ 1, column col ^ 8 in lane ^ 8 (the whole wave takes part)
      const float partner = EPI == kEpiRope     ? __shfl_xor(v, 1, 64)
                            : EPI == kEpiSwiGLU ? __shfl_xor(v, 8, 64)
                                                : 0.f;
      if (orow < n) store_out<TO, EPI>(y, ldy, ra, orow, g, col, v, partner, rp[t][r]);
    }
  }
}

// The few-row regime's launch shape for n rows, `tiles` 16-column tiles and R
// chunks per sub-slice.
struct WidePlan {
  bool wide, half, ww8;
  int groups;  // workgroups of the few-row launch (0 if not few-row)
};
static WidePlan wide_plan(int n, int tiles, int R, bool swiglu) {
  WidePlan w;
  w.wide = n <= kWideMaxRows && R <= kWideMaxChunksPerWave;
  // fewer tiles than half the chip's 256 CUs x 2: split tiles into column halves
  // (not for SwiGLU, whose partner column c ^ 8 lies in the other half)
  w.half = !swiglu && tiles <= kHalfTileMax;
  // more tiles than two 1024-thread workgroups per CU hold: 8-wave workgroups
  // (three per CU by their 48 KB of LDS), so the whole launch is resident in
  // one round (gate|up at 704 tiles: 11.5 -> 10.4 us); each wave then sums
  // two sub-slices, so only for one chunk per sub-slice (K <= 16 chunks)
  w.ww8 = !w.half && tiles > kResidentWide && R == 1;
  w.groups = w.wide ? (w.half ? 2 * tiles : tiles) : 0;
  return w;
}

template <typename T, typename TO, int EPI>
static void launch_linear(const void* x, const int32_t* xr, int64_t ldx, const void* W, void* y, int64_t ldy, int n,
                          int N, int K, int pair_off, const RopeArgs& ra, hipStream_t st,
                          const TileArgmax& am = TileArgmax{nullptr, nullptr}, const wfd_rowscale_t& rs = {},
                          const wfd_prep_t& pp = {}) {
  const int tiles = N / 16;
  const int R = sub_chunks(K / LinTraits<T>::KC);  // chunks per sub-slice: one sub-slice per wave (two with 8 waves)
  const WidePlan wp = wide_plan(n, tiles, R, EPI == kEpiSwiGLU);
  const bool wide = wp.wide, half = wp.half, ww8 = wp.ww8;
#define WFD_WIDE(RMV)                                                                                             \
  if (half)                                                                                                       \
    hipLaunchKernelGGL((linear_wide_kernel<T, TO, EPI, RMV, true, kWideWaves>), dim3(2 * tiles),                 \
                       dim3(64 * kWideWaves), 0, st, (const T*)x, xr, ldx, (const T*)W, (TO*)y, ldy, n, K,       \
                       pair_off, ra, am, rs, pp);                                                                 \
  else                                                                                                            \
    hipLaunchKernelGGL((linear_wide_kernel<T, TO, EPI, RMV, false, kWideWaves>), dim3(tiles), dim3(64 * kWideWaves), \
                       0, st, (const T*)x, xr, ldx, (const T*)W, (TO*)y, ldy, n, K, pair_off, ra, am, rs, pp);
#define WFD_WIDE8(RMV)                                                                                          \
  hipLaunchKernelGGL((linear_wide_kernel<T, TO, EPI, RMV, false, 8>), dim3(tiles), dim3(64 * 8), 0, st,        \
                     (const T*)x, xr, ldx, (const T*)W, (TO*)y, ldy, n, K, pair_off, ra, am, rs, pp);
  if (wide && ww8) {
    WFD_WIDE8(1)
  } else if (wide && R == 1) {
    WFD_WIDE(1)
  } else if (wide && R == 2) {
    WFD_WIDE(2)
  } else if (wide) {
    WFD_WIDE(3)
  } else if constexpr (EPI != kEpiPrep) {  // the prep epilogue has a few-row form only (checked on entry)
#undef WFD_WIDE8
#undef WFD_WIDE
    const float* rsc = rs.scale;  // many rows: the scales precomputed (group sums are few-row only)
    const int rb = (n + 63) / 64;
    if (tiles <= kStreamMaxTiles) {
      // few weight tiles: each workgroup walks all of K, so its chunk chain is
      // the launch's critical path; keep kStreamStages - 1 chunks in flight.
      // One tile per workgroup while that makes at most 256 workgroups, else
      // two (at 192 rows x 128 tiles, 384 one-tile workgroups took ~1.5x as
      // long as 192 two-tile ones).
      if (rb * tiles > 256)
        hipLaunchKernelGGL((linear_stream_kernel<T, TO, EPI, 2, kStreamStages>), dim3(rb, (tiles + 1) / 2), dim3(256),
                           0, st, (const T*)x, xr, ldx, (const T*)W, (TO*)y, ldy, n, K, pair_off, tiles, ra, rsc);
      else
        hipLaunchKernelGGL((linear_stream_kernel<T, TO, EPI, 1, kStreamStages>), dim3(rb, tiles), dim3(256), 0, st,
                           (const T*)x, xr, ldx, (const T*)W, (TO*)y, ldy, n, K, pair_off, tiles, ra, rsc);
      return;
    }
    // few (row block, tile) pairs, or at most 32 rows where four-tile gemm
    // workgroups would not cover the CUs: every wave streams its own weights,
    // no barriers (gate|up at 17-32 rows: 16.1-17.1 -> 14.0-14.9 us; lm_head,
    // with 500 gemm workgroups, stays on the gemm)
    if (rb * tiles <= kGemmMinBlockTiles || (n <= 32 && (tiles + 3) / 4 < 256)) {
      constexpr int NB = 2;
      hipLaunchKernelGGL((linear_tile_kernel<T, TO, EPI, NB>), dim3(rb, (tiles + NB - 1) / NB), dim3(256), 0, st,
                         (const T*)x, xr, ldx, (const T*)W, (TO*)y, ldy, n, K, pair_off, tiles, ra, rsc);
      return;
    }
    // weights through LDS, shared by the 4 waves: 4 tiles per workgroup
    // while that still leaves >= 256 workgroups (128 for the epilogues
    // without the RoPE operand tables), else 2. lm_head at 64 rows: 500
    // four-tile workgroups 34 us, 1000 two-tile ones 42 us; gate|up at 64
    // rows: 176 four-tile ones 16.4 us, 352 two-tile ones 17.8 us (in the
    // bs=32 decode); Wqkv + RoPE at 128 rows keeps 2 (192 four-tile
    // workgroups: 21.1 -> 24.5 us, the epilogue's tables cost registers per
    // tile). Eight tiles per workgroup were slower in the decode for every
    // one-launch shape (Wqkv + RoPE at 192 rows 28 -> 48 us).
    if (rb * ((tiles + 3) / 4) >= (EPI == kEpiRope ? 256 : 128))
      hipLaunchKernelGGL((linear_gemm_kernel<T, TO, EPI, 4, false>), dim3(xcd_grid(rb, (tiles + 3) / 4)), dim3(256), 0,
                         st, (const T*)x, xr, ldx, (const T*)W, (TO*)y, ldy, n, K, pair_off, tiles, ra, nullptr, rsc);
    else
      hipLaunchKernelGGL((linear_gemm_kernel<T, TO, EPI, 2, false>), dim3(xcd_grid(rb, (tiles + 1) / 2)), dim3(256), 0,
                         st, (const T*)x, xr, ldx, (const T*)W, (TO*)y, ldy, n, K, pair_off, tiles, ra, nullptr, rsc);
  }
}

// The slice form: grid (xcd-mapped row blocks x tile groups, slices), 2 or 4
// tiles per workgroup as for the one-launch gemm: each workgroup reads its 64
// rows of x once for 32 or 64 output columns and only its slice of K,
// where the stream kernel reads them for 16 columns and all of K.
template <typename T>
static void launch_linear_partials(const void* x, const int32_t* xr, int64_t ldx, const void* W, float* part, int n,
                                   int N, int K, hipStream_t st) {
  const int tiles = N / 16;
  const int P = K / LinTraits<T>::KC;
  const int S = slice_count(P);
  const int rb = (n + 63) / 64;
  const RopeArgs ra{};
  const int bt = gemm_tiles_per_workgroup(rb, tiles, S);
#define WFD_GEMM_PART(BTV)                                                                                          \
  hipLaunchKernelGGL((linear_gemm_kernel<T, T, kEpiPlain, BTV, true>), dim3(xcd_grid(rb, (tiles + BTV - 1) / BTV), S), \
                     dim3(256), 0, st, (const T*)x, xr, ldx, (const T*)W, (T*)nullptr, 0, n, K, 0, tiles, ra, part,  \
                     nullptr)
  if (bt == 4)
    WFD_GEMM_PART(4);
  else
    WFD_GEMM_PART(2);
#undef WFD_GEMM_PART
}

// The row-scale argument of the consumer entry points: NULL (none), the
// precomputed scales, or group sums (few-row launches only). Returns the
// value to launch with, or sets the error.
static bool rowscale_arg(const wfd_rowscale_t* rs, int n, int N, int K, int dtype, bool swiglu, const char* what,
                         wfd_rowscale_t& out) {
  out = wfd_rowscale_t{};
  if (!rs) return true;
  if (!rs->scale && !rs->part) {
    set_error("%s: a row-scale argument needs scale or part", what);
    return false;
  }
  if (rs->part) {
    const int kc = dtype == kBF16 ? LinTraits<bf16_t>::KC : LinTraits<float>::KC;
    const bool wide = wide_plan(n, N / 16, sub_chunks(K / kc), swiglu).wide;
    const int dmax = dtype == kBF16 ? fold_max_d<bf16_t>() : fold_max_d<float>();
    if (!wide || rs->D <= 0 || rs->D % kc || rs->D > dmax || ((uintptr_t)rs->part & 15)) {
      set_error("%s: group sums (rs->part, 16-byte aligned) need a few-row launch (n=%d <= 16, K=%d) and "
                "0 < D=%d <= %d, a multiple of %d", what, n, K, rs->D, dmax, kc);
      return false;
    }
  }
  out = *rs;
  return true;
}

}  // namespace wfd

extern "C" {

int wfd_linear_slices(int K, int dtype) {
  using namespace wfd;
  const int kc = dtype == kBF16 ? LinTraits<bf16_t>::KC : LinTraits<float>::KC;
  if (K <= 0 || K % kc) return 0;
  return slice_count(K / kc);
}

int wfd_linear_partials(const void* x, const int32_t* x_rows, int64_t ldx, const void* W, float* part, int n, int N,
                        int K, int dtype, hipStream_t stream) {
  using namespace wfd;
  const int kc = dtype == kBF16 ? LinTraits<bf16_t>::KC : LinTraits<float>::KC;
  if (n < 0 || N <= 0 || N % 16 || K <= 0 || K % kc || ldx < K || (dtype != kBF16 && dtype != kF32)) {
    set_error("wfd_linear_partials: bad shape n=%d N=%d K=%d ldx=%lld dtype=%d", n, N, K, (long long)ldx, dtype);
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!x || !W || !part) {
    set_error("wfd_linear_partials: null pointer argument");
    return kBadArg;
  }
  const int64_t es = dtype == kBF16 ? 2 : 4;
  if (!x_rows && (int64_t)n * ldx * es >= (int64_t)kBufInvalid) {
    set_error("wfd_linear_partials: the x operand must span less than 2 GiB");
    return kBadArg;
  }
  if (((uintptr_t)x | (uintptr_t)W | (uintptr_t)part | (uintptr_t)(ldx * es)) & 15) {
    set_error("wfd_linear_partials: x, W, part and the x row pitch must be 16-byte aligned");
    return kBadArg;
  }
  if (dtype == kBF16)
    launch_linear_partials<bf16_t>(x, x_rows, ldx, W, part, n, N, K, stream);
  else
    launch_linear_partials<float>(x, x_rows, ldx, W, part, n, N, K, stream);
  return launch_status("wfd_linear_partials");
}

int wfd_linear_k_multiple(int dtype) {
  using namespace wfd;
  return dtype == kBF16 ? LinTraits<bf16_t>::KC : LinTraits<float>::KC;
}

int wfd_linear_pack(const void* W, void* W_packed, int N, int K, int dtype, int epilogue, int pair_off,
                    hipStream_t stream) {
  using namespace wfd;
  const int kmul = wfd_linear_k_multiple(dtype);
  if (N <= 0 || K <= 0 || N % 16 != 0 || K % kmul != 0) {
    set_error("wfd_linear_pack: N=%d must be a multiple of 16 and K=%d of %d", N, K, kmul);
    return kBadArg;
  }
  if (!W || !W_packed || W == W_packed) {
    set_error("wfd_linear_pack: null or aliased pointer argument");
    return kBadArg;
  }
  if (epilogue == kEpiSwiGLU && (pair_off <= 0 || pair_off % 8 != 0 || N != 2 * pair_off)) {
    set_error("wfd_linear_pack: swiglu needs N == 2*pair_off, pair_off %% 8 == 0 (N=%d pair_off=%d)", N, pair_off);
    return kBadArg;
  }
  if (epilogue != kEpiPlain && epilogue != kEpiSwiGLU) {
    set_error("wfd_linear_pack: unknown epilogue %d", epilogue);
    return kUnsupported;
  }
  const int V = dtype == kBF16 ? Chunk<bf16_t>::V : Chunk<float>::V;
  const int64_t nfrag = (int64_t)N * K / V;
  const dim3 grid((unsigned)((nfrag + 255) / 256)), block(256);
  if (dtype == kBF16 && epilogue == kEpiSwiGLU)
    hipLaunchKernelGGL((linear_pack_kernel<bf16_t, kEpiSwiGLU>), grid, block, 0, stream, (const bf16_t*)W,
                       (bf16_t*)W_packed, K, pair_off, nfrag);
  else if (dtype == kBF16)
    hipLaunchKernelGGL((linear_pack_kernel<bf16_t, kEpiPlain>), grid, block, 0, stream, (const bf16_t*)W,
                       (bf16_t*)W_packed, K, pair_off, nfrag);
  else if (dtype == kF32 && epilogue == kEpiSwiGLU)
    hipLaunchKernelGGL((linear_pack_kernel<float, kEpiSwiGLU>), grid, block, 0, stream, (const float*)W,
                       (float*)W_packed, K, pair_off, nfrag);
  else if (dtype == kF32)
    hipLaunchKernelGGL((linear_pack_kernel<float, kEpiPlain>), grid, block, 0, stream, (const float*)W,
                       (float*)W_packed, K, pair_off, nfrag);
  else {
    set_error("wfd_linear_pack: unsupported dtype %d", dtype);
    return kUnsupported;
  }
  return launch_status("wfd_linear_pack");
}

int wfd_linear(const void* x, const int32_t* x_rows, int64_t ldx, const void* W, void* y, int64_t ldy, int n, int N,
               int K, int dtype, int out_dtype, int epilogue, int pair_off, const wfd_rowscale_t* rs,
               hipStream_t stream) {
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
  const int64_t esz = dtype == kBF16 ? 2 : 4;
  if (!x_rows && (int64_t)n * ldx * esz >= (int64_t)kBufInvalid) {
    set_error("wfd_linear: the x operand must span less than 2 GiB");
    return kBadArg;
  }
  if ((((uintptr_t)x | (uintptr_t)W) & 15) || ((ldx * esz) & 15)) {
    set_error("wfd_linear: x rows and W must be 16-byte aligned (ldx=%lld)", (long long)ldx);
    return kBadArg;
  }
  const int kmul = wfd_linear_k_multiple(dtype);
  if (K % kmul != 0 || N % 16 != 0) {
    set_error("wfd_linear: K=%d must be a multiple of %d and N=%d of 16", K, kmul, N);
    return kUnsupported;
  }
  if (epilogue == kEpiSwiGLU) {
    if (pair_off <= 0 || pair_off % 8 != 0 || N != 2 * pair_off || ldy < pair_off) {
      set_error("wfd_linear: swiglu needs N == 2*pair_off, pair_off %% 8 == 0 (N=%d pair_off=%d)", N, pair_off);
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
  wfd_rowscale_t rsv;
  if (!rowscale_arg(rs, n, N, K, dtype, epilogue == kEpiSwiGLU, "wfd_linear", rsv)) return kBadArg;
  const RopeArgs ra{};
  const TileArgmax am{nullptr, nullptr};
  if (dtype == kBF16 && out_dtype == kBF16) {
    if (epilogue == kEpiSwiGLU)
      launch_linear<bf16_t, bf16_t, kEpiSwiGLU>(x, x_rows, ldx, W, y, ldy, n, N, K, pair_off, ra, stream, am, rsv);
    else
      launch_linear<bf16_t, bf16_t, kEpiPlain>(x, x_rows, ldx, W, y, ldy, n, N, K, 0, ra, stream, am, rsv);
  } else if (dtype == kBF16 && out_dtype == kF32 && epilogue == kEpiPlain) {
    launch_linear<bf16_t, float, kEpiPlain>(x, x_rows, ldx, W, y, ldy, n, N, K, 0, ra, stream, am, rsv);
  } else if (dtype == kF32 && out_dtype == kF32) {
    if (epilogue == kEpiSwiGLU)
      launch_linear<float, float, kEpiSwiGLU>(x, x_rows, ldx, W, y, ldy, n, N, K, pair_off, ra, stream, am, rsv);
    else
      launch_linear<float, float, kEpiPlain>(x, x_rows, ldx, W, y, ldy, n, N, K, 0, ra, stream, am, rsv);
  } else {
    set_error("wfd_linear: unsupported dtype=%d out_dtype=%d epilogue=%d", dtype, out_dtype, epilogue);
    return kUnsupported;
  }
  return launch_status("wfd_linear");
}

int wfd_linear_argmax_groups(int n, int N, int K, int dtype) {
  using namespace wfd;
  if (n <= 0 || N <= 0 || N % 16 != 0 || dtype != kBF16 || K <= 0 || K % wfd_linear_k_multiple(dtype) != 0) return 0;
  return wide_plan(n, N / 16, sub_chunks(K / LinTraits<bf16_t>::KC), false).groups;
}

int wfd_linear_argmax(const void* x, const int32_t* x_rows, int64_t ldx, const void* W, float* y, int64_t ldy, int n,
                      int N, int K, int dtype, float* part_val, int32_t* part_idx, const wfd_rowscale_t* rs,
                      hipStream_t stream) {
  using namespace wfd;
  if (n <= 0 || N <= 0 || K <= 0 || ldx < K) {
    set_error("wfd_linear_argmax: bad shape n=%d N=%d K=%d ldx=%lld", n, N, K, (long long)ldx);
    return kBadArg;
  }
  if (wfd_linear_argmax_groups(n, N, K, dtype) <= 0) {
    set_error("wfd_linear_argmax: n=%d N=%d K=%d dtype=%d is not a few-row bf16 launch (no column groups)", n, N, K,
              dtype);
    return kUnsupported;
  }
  if (!x || !W || !y || !part_val || !part_idx) {
    set_error("wfd_linear_argmax: null pointer argument");
    return kBadArg;
  }
  const int64_t esz = 2;
  if (!x_rows && (int64_t)n * ldx * esz >= (int64_t)kBufInvalid) {
    set_error("wfd_linear_argmax: the x operand must span less than 2 GiB");
    return kBadArg;
  }
  if ((((uintptr_t)x | (uintptr_t)W) & 15) || ((ldx * esz) & 15)) {
    set_error("wfd_linear_argmax: x rows and W must be 16-byte aligned (ldx=%lld)", (long long)ldx);
    return kBadArg;
  }
  if (ldy < N) {
    set_error("wfd_linear_argmax: ldy=%lld < N=%d", (long long)ldy, N);
    return kBadArg;
  }
  wfd_rowscale_t rsv;
  if (!rowscale_arg(rs, n, N, K, dtype, false, "wfd_linear_argmax", rsv)) return kBadArg;
  const RopeArgs ra{};
  launch_linear<bf16_t, float, kEpiPlain>(x, x_rows, ldx, W, y, ldy, n, N, K, 0, ra, stream,
                                          TileArgmax{part_val, part_idx}, rsv);
  return launch_status("wfd_linear_argmax");
}

int wfd_linear_qkv_rope_append(const void* x, const int32_t* x_rows, int64_t ldx, const void* Wqkv, int n, int K,
                               const int32_t* pos, const float* rope_cos, const float* rope_sin, int rope_rows,
                               const int64_t* flat_row, void* q_out, void* k_cache, void* v_cache,
                               int64_t kv_block_rows, int H, int Hkv, int Dh, int dtype, const wfd_rowscale_t* rs,
                               hipStream_t stream) {
  using namespace wfd;
  if (n < 0 || K <= 0 || ldx < K || H <= 0 || Hkv <= 0 || H % Hkv != 0 || Dh <= 0 || Dh % 16 != 0 ||
      rope_rows <= 0 || kv_block_rows < 0) {
    set_error("wfd_linear_qkv_rope_append: bad shape n=%d K=%d H=%d Hkv=%d Dh=%d rope_rows=%d", n, K, H, Hkv, Dh,
              rope_rows);
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!x || !Wqkv || !pos || !rope_cos || !rope_sin || !flat_row || !q_out || !k_cache || !v_cache) {
    set_error("wfd_linear_qkv_rope_append: null pointer argument");
    return kBadArg;
  }
  const int64_t esz = dtype == kBF16 ? 2 : 4;
  if (!x_rows && (int64_t)n * ldx * esz >= (int64_t)kBufInvalid) {
    set_error("wfd_linear_qkv_rope_append: the x operand must span less than 2 GiB");
    return kBadArg;
  }
  if ((((uintptr_t)x | (uintptr_t)Wqkv) & 15) || ((ldx * esz) & 15)) {
    set_error("wfd_linear_qkv_rope_append: x rows and Wqkv must be 16-byte aligned (ldx=%lld)", (long long)ldx);
    return kBadArg;
  }
  const int kmul = wfd_linear_k_multiple(dtype);
  if (K % kmul != 0) {
    set_error("wfd_linear_qkv_rope_append: K=%d must be a multiple of %d", K, kmul);
    return kUnsupported;
  }
  const int N = (H + 2 * Hkv) * Dh;
  wfd_rowscale_t rsv;
  if (!rowscale_arg(rs, n, N, K, dtype, false, "wfd_linear_qkv_rope_append", rsv)) return kBadArg;
  const RopeArgs ra{pos, rope_cos, rope_sin, rope_rows, flat_row, q_out, k_cache, v_cache, kv_block_rows, H, Hkv, Dh};
  const TileArgmax am{nullptr, nullptr};
  if (dtype == kBF16)
    launch_linear<bf16_t, bf16_t, kEpiRope>(x, x_rows, ldx, Wqkv, nullptr, 0, n, N, K, 0, ra, stream, am, rsv);
  else if (dtype == kF32)
    launch_linear<float, float, kEpiRope>(x, x_rows, ldx, Wqkv, nullptr, 0, n, N, K, 0, ra, stream, am, rsv);
  else {
    set_error("wfd_linear_qkv_rope_append: unsupported dtype=%d", dtype);
    return kUnsupported;
  }
  return launch_status("wfd_linear_qkv_rope_append");
}

int wfd_linear_prep(const void* x, const int32_t* x_rows, int64_t ldx, const void* W, int n, int N, int K, int dtype,
                    const wfd_prep_t* pp, hipStream_t stream) {
  using namespace wfd;
  if (n < 0 || N <= 0 || N % 16 || K <= 0 || ldx < K || (dtype != kBF16 && dtype != kF32)) {
    set_error("wfd_linear_prep: bad shape n=%d N=%d K=%d ldx=%lld dtype=%d", n, N, K, (long long)ldx, dtype);
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!x || !W || !pp || !pp->a_out || !pp->wb || !pp->part) {
    set_error("wfd_linear_prep: null pointer argument (x, W, pp, a_out, wb and part are required)");
    return kBadArg;
  }
  const int kc = wfd_linear_k_multiple(dtype);
  const int dmax = dtype == kBF16 ? fold_max_d<bf16_t>() : fold_max_d<float>();
  if (N > dmax || N % kc) {
    set_error("wfd_linear_prep: N=%d must be a multiple of %d, at most %d", N, kc, dmax);
    return kUnsupported;
  }
  if (K % kc || !wide_plan(n, N / 16, sub_chunks(K / kc), false).wide) {
    set_error("wfd_linear_prep: n=%d K=%d is not a few-row launch (n <= 16, K a multiple of %d and at most 48 chunks)",
              n, K, kc);
    return kUnsupported;
  }
  if ((pp->r_in && pp->ld_in < N) || (pp->r_out && pp->ld_out < N) || pp->ld_a < N) {
    set_error("wfd_linear_prep: a row pitch of r_in / r_out / a_out is below N=%d", N);
    return kBadArg;
  }
  const int64_t esz = dtype == kBF16 ? 2 : 4;
  if (!x_rows && (int64_t)n * ldx * esz >= (int64_t)kBufInvalid) {
    set_error("wfd_linear_prep: the x operand must span less than 2 GiB");
    return kBadArg;
  }
  if ((((uintptr_t)x | (uintptr_t)W | (uintptr_t)pp->part) & 15) || ((ldx * esz) & 15)) {
    set_error("wfd_linear_prep: x rows, W and part must be 16-byte aligned");
    return kBadArg;
  }
  const RopeArgs ra{};
  const TileArgmax am{nullptr, nullptr};
  const wfd_rowscale_t none{};
  if (dtype == kBF16)
    launch_linear<bf16_t, bf16_t, kEpiPrep>(x, x_rows, ldx, W, nullptr, 0, n, N, K, 0, ra, stream, am, none, *pp);
  else
    launch_linear<float, float, kEpiPrep>(x, x_rows, ldx, W, nullptr, 0, n, N, K, 0, ra, stream, am, none, *pp);
  return launch_status("wfd_linear_prep");
}

}  // extern "C"
