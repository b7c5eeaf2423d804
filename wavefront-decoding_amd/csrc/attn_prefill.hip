// Causal prefill attention over the slot cache on MFMA (flash-attention
// forward, bf16 in, fp32 softmax and accumulation).
//
// Replaces the prompt pass's dense causal attention: attn_dense(q, k, v,
// causal=True) (src/decoding/fa4_attention.py:189-215) as called by
// _block_dense (src/decoding/huginn_blocks_batch.py:163-170), and the grouped
// bottom-right-causal segments of _core_attn_varlen
// (src/decoding/parcae_blocks.py:435-456): a segment of queries at consecutive
// positions pos0, pos0 + 1, ... of one slot, each attending keys [0, position].
//
// Segment s owns query rows [q_start[s], q_start[s+1]) of q (n, H, Dh); its
// keys are cache rows row_base[s] + [0, pos0[s] + len) (already appended), read
// in place from either cache layout (kv_offset). out row r = softmax over the
// row's causal prefix of (q_r . k) * scale, times V.
//
// Work split: a workgroup owns 128 consecutive query rows of one segment and
// one query head, as NS key streams of 4 waves: stream st takes the 64-key
// tiles t = st, st + NS, ... of the rows' causal range, and its wave w owns
// rows 32w..32w+31, one query per lane column of the 32x32 MFMA tiles.
// Per tile a stream stages K and V row-major in its own LDS buffers (16-byte
// stores, no transpose), with its next tile's global loads (32-bit buffer
// offsets, nothing read past the segment's last key) issued before the
// current tile's math so their latency hides under it. With two streams,
// stream 1 parks each row's running maximum, sum and output in LDS at the end
// and stream 0 merges them into its own (the log-sum-exp merge of two partial
// softmaxes) and stores the row. A segment whose query tiles over all heads
// fit 256 workgroups (at most 256 * 128 / H rows: a 2048-token prompt at 16
// heads) takes two streams: few workgroups, so its time is the longest
// workgroup's chain of tiles, which two streams halve while giving every SIMD
// two waves. Longer segments take one stream (4-wave workgroups, two per CU
// by their LDS, each free to run ahead of the other). The choice depends only
// on the segment's length and H, so a segment's output bits do not depend on
// the other segments of the launch: a launch that mixes both kinds runs the
// kernel once per kind, each skipping the other kind's segments.
// Each wave computes S^T = K Q^T on v_mfma_f32_32x32x16_bf16 (two 32-key
// blocks x Dh/16 steps), then O^T = V^T P^T on the same instruction, its V^T
// operand read straight from the row-major V tile with the LDS transposing
// read (ds_read_b64_tr_b16, two per fragment). Against 16-query blocks on the
// 16x16x32 MFMA this halves the LDS bytes read per flop: every K and V^T
// fragment a wave reads feeds 32 queries.
//
// Key order inside a 32-key block: MFMA row r (lane half hf = lane / 32 holds
// rows 8i + 4hf + j, i, j < 4) reads K row pi(r) = 16(i / 2) + 8hf + 4(i % 2)
// + j, so result register rr of a lane holds key 16(rr / 8) + 8hf + rr % 8 --
// exactly the 8 consecutive keys the B operand of a 16-key P^T step wants in
// that lane. P thus goes from the S^T accumulators to the B operand of
// O^T = V^T P^T by packing to bf16, with no exchange, and the V^T fragment of
// the same lane half is 8 consecutive keys of one d column (two transposing
// LDS reads of 4 keys). A lane's output column is its query, so the online
// softmax's max and sum need one shuffle (the other lane half) and the
// rescale none; the scale folds into the exponent's FMA. Tiles past the
// diagonal are never visited; the diagonal tiles mask keys past each row's
// position (tiles below them skip the mask). Query tiles are dispatched
// longest first.
#include "wfd_common.h"

namespace wfd {

constexpr int kPfWaves = 4;              // query blocks of 32 rows per workgroup (waves per stream)
constexpr int kPfSplitGroups = 256;     // a segment with at most this many (query tile, head) workgroups takes two key streams
constexpr int kPfRows = 32 * kPfWaves;  // query rows per workgroup
constexpr int kPfKeys = 64;             // keys per tile

typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16 mfma32(const u32x4& a, const u32x4& b, f32x16 acc) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc,
                                                 0, 0, 0);
}

// The longest segment (in query rows) that takes two key streams at H query heads.
__host__ __device__ constexpr int pf_split_max_rows(int H) {
  return (kPfSplitGroups / H > 0 ? kPfSplitGroups / H : 1) * kPfRows;
}

template <int DH, int NS>
__global__ __launch_bounds__(64 * kPfWaves * NS) __attribute__((amdgpu_waves_per_eu(2))) void attn_prefill_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ kc, const bf16_t* __restrict__ vc, int64_t block_rows,
    const int64_t* __restrict__ seg_row_base, const int32_t* __restrict__ seg_q_start,
    const int32_t* __restrict__ seg_pos0, bf16_t* __restrict__ out, int H, int Hkv, float scale_log2) {
  static_assert(NS == 1 || NS == 2, "one or two key streams");
  constexpr int NT = 64 * kPfWaves;   // threads per stream
  constexpr int V = 8;                // bf16 per 16-byte fragment
  constexpr int NDS = DH / 16;        // MFMA k-steps over Dh (S^T = K Q^T)
  constexpr int NDB = DH / 32;        // 32-row blocks of O^T (head dim)
  constexpr int NKB = kPfKeys / 32;   // 32-key blocks of S^T
  constexpr int NPS = kPfKeys / 16;   // MFMA k-steps over keys (O^T += V^T P^T)
  constexpr int KP = DH + 8;          // padded LDS row of K (elements)
  // padded LDS row of V: a transposing read takes 4 rows x 64 bytes per 32
  // lanes, which a row of DH + 32 elements (2 DH + 64 bytes) spreads over all
  // 64 banks for DH = 64 and 128
  constexpr int VRP = DH + 32;
  constexpr int CPR = DH / V;         // 16-byte chunks per K / V row
  constexpr int KCH = kPfKeys * CPR / NT;      // K (and V) chunks per thread per tile
  static_assert(KCH >= 1 && kPfKeys * CPR % NT == 0, "tile split");
  // per stream, double-buffered: one barrier per tile pair
  __shared__ __align__(16) bf16_t k_lds[NS][2][kPfKeys * KP];
  __shared__ __align__(16) bf16_t v_lds[NS][2][kPfKeys * VRP];
  constexpr int PW = NDB * 16 + 2;  // floats a lane of stream 1 parks: its output registers, maximum and sum
  static_assert(NS == 1 || sizeof(k_lds) >= sizeof(float) * kPfWaves * PW * 64, "park area");

  // the head is the fastest grid dimension, so the launch hands out the
  // longest query tiles of every head before any shorter one (longest first
  // over the whole launch, not per head: a head's long tiles never start last)
  const int s = blockIdx.z;
  const int h = blockIdx.x;
  const int q0 = seg_q_start[s];
  const int len = seg_q_start[s + 1] - q0;
  if ((len <= pf_split_max_rows(H)) != (NS == 2)) return;  // the other kind's segment (uniform)
  const int tq = (len + kPfRows - 1) / kPfRows - 1 - (int)blockIdx.y;
  if (tq < 0) return;  // uniform for the workgroup
  const int pos0 = seg_pos0[s];
  const int g = h / (H / Hkv);
  const int64_t hb = kv_offset(seg_row_base[s], g, Hkv, DH, block_rows);
  const uint32_t rsb = (uint32_t)((block_rows > 1 ? DH : Hkv * DH) * sizeof(bf16_t));  // key stride, bytes

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int st = NS == 1 ? 0 : wave / kPfWaves;  // key stream
  const int qb = wave % kPfWaves;    // query block
  const int lt = threadIdx.x % NT;   // thread within the stream
  const int lane = threadIdx.x & 63;
  const int col = lane & 31;  // query of this lane
  const int hf = lane >> 5;   // lane half
  const int row0 = tq * kPfRows + qb * 32;
  const int last_row = min((tq + 1) * kPfRows, len) - 1;
  const int kv_hi = pos0 + last_row + 1;  // keys [0, kv_hi) cover every row of the tile
  const int ntiles = (kv_hi + kPfKeys - 1) / kPfKeys;
  // K / V of this head from key 0; the resource ends at key kv_hi - 1, so the
  // staging loads of later keys read zeros (those keys are masked for every row)
  const uint32_t span = (uint32_t)(kv_hi - 1) * rsb + DH * sizeof(bf16_t);
  const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(kc + hb), (short)0, span,
                                                                      0x00020000);
  const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16_t*>(vc + hb), (short)0, span,
                                                                      0x00020000);

  // Q as the MFMA B operand: column col = query row0 + col, dims 16k + 8hf + (0..7)
  u32x4 qf[NDS];
  {
    const int r = min(row0 + col, len - 1);
    const bf16_t* qp = q + ((int64_t)(q0 + r) * H + h) * DH + hf * V;
#pragma unroll
    for (int k = 0; k < NDS; ++k) qf[k] = ld16(qp + k * 16);
  }
  // K row of MFMA row col within a 32-key block (the permutation above)
  const int krow = 16 * ((col >> 3) >> 1) + 8 * ((col >> 2) & 1) + 4 * ((col >> 3) & 1) + (col & 3);

  // staging: thread's K and V chunks (key, 8 dims), both stored row-major
  u32x4 kreg[KCH], vreg[KCH];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = lt + i * NT;
      const int kr_ = c / CPR;
      const uint32_t off = (uint32_t)(k0 + kr_) * rsb + (uint32_t)((c - kr_ * CPR) * V * sizeof(bf16_t));
      kreg[i] = buf_ld16(kr, off);
      vreg[i] = buf_ld16(vr, off);
    }
  };
  auto stage = [&](int b) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = lt + i * NT;
      const int kr_ = c / CPR;
      *reinterpret_cast<u32x4*>(&k_lds[st][b][kr_ * KP + (c - kr_ * CPR) * V]) = kreg[i];
      *reinterpret_cast<u32x4*>(&v_lds[st][b][kr_ * VRP + (c - kr_ * CPR) * V]) = vreg[i];
    }
  };
  // V^T fragment of d-block db, key step k (the A operand of O^T += V^T P^T:
  // lane l holds d = 32 db + l % 32, keys 16 k + 8 (l / 32) + 0..7) from the
  // row-major V tile with two transposing reads. Within each 16-lane group
  // the read hands lane i element i % 4 of the 8-byte chunks that lanes
  // i / 4, 4 + i / 4, 8 + i / 4, 12 + i / 4 address; lane j addressing V[key0 +
  // j / 4][dbase + 4 (j % 4)] thus yields V[key0 + 0..3][dbase + i] in lane i.
  const int tg = lane >> 4;  // 16-lane group: bit 0 picks d + 16, bit 1 keys + 8
  const int ti = lane & 15;
  const int v_lane = ((tg >> 1) * 8 + (ti >> 2)) * VRP + 16 * (tg & 1) + 4 * (ti & 3);
  auto vt_frag = [&](int b, int db, int k) {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
    typedef const __attribute__((address_space(3))) void* lds_ptr;
    const bf16_t* p = &v_lds[st][b][v_lane + 16 * k * VRP + 32 * db];
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_ptr)p);
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(lds_ptr)(p + 4 * VRP));
    const uint2 a = __builtin_bit_cast(uint2, lo), c = __builtin_bit_cast(uint2, hi);
    return u32x4{a.x, a.y, c.x, c.y};
  };

  float mrun = -INFINITY, lrun = 0.f;
  f32x16 o[NDB];
#pragma unroll
  for (int c = 0; c < NDB; ++c)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[c][r] = 0.f;
  const int qpos = pos0 + row0 + col;

  // round it: stream st's tile t = NS it + st lives in its buffer
  // it & 1; the registers hold the stream's next tile while tile t is
  // computed, and are staged into the other buffer after it (that buffer was
  // last read in round it - 1, before the barrier that closed it). Tiles past
  // the last are staged as zeros and not computed.
  const int rounds = (ntiles + NS - 1) / NS;
  fetch(st * kPfKeys);
  stage(0);
  fetch((st + NS) * kPfKeys);
  __syncthreads();
  for (int it = 0; it < rounds; ++it) {
    const int t = it * NS + st;
    const int k0 = t * kPfKeys;
    const int b = it & 1;
    if (t < ntiles) {  // uniform over the stream's waves
    // keys past some row's position only in the diagonal tiles (uniform per wave)
    const bool full = k0 + kPfKeys - 1 <= pos0 + row0;

    // S^T = K Q^T: register rr of block kb holds S[query col][key k0 + 32 kb + 16 (rr / 8) + 8 hf + rr % 8]
    // (the two 32-key blocks' chains interleaved: back-to-back MFMAs are
    // independent; the wave's priority is raised while it issues MFMAs so a
    // wave in its softmax fills the MFMA shadows, not the other way round)
    f32x16 sacc[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int k = 0; k < NDS; ++k)
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const u32x4 afr = *reinterpret_cast<const u32x4*>(&k_lds[st][b][(32 * kb + krow) * KP + 16 * k + hf * V]);
        sacc[kb] = mfma32(afr, qf[k], sacc[kb]);
      }
    __builtin_amdgcn_s_setprio(0);
    // online softmax (log2 domain: p = 2^(s * scale_log2 - m)); stream 0's
    // first tile holds key 0 for every row, so its m is finite from then on;
    // a stream-1 row may see only masked scores (-inf) in its first tiles,
    // whose maximum stays -inf: those take 0 as the reference point, so
    // masked scores give p = 0 without a test
    if (!full) {  // a diagonal tile (uniform over the wave)
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (k0 + 32 * kb + 16 * (r >> 3) + 8 * hf + (r & 7) > qpos) sacc[kb][r] = -INFINITY;
    }
    float mt = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, sacc[kb][r]);
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mnew = fmaxf(mrun, mt * scale_log2);
    const float mref = mnew == -INFINITY ? 0.f : mnew;
    // the hardware 2^x (v_exp_f32): results below 2^-126 flush to zero, which
    // only drops probabilities far below bf16 resolution of the row's sum
    const float corr = __builtin_amdgcn_exp2f(mrun - mref);
    float lt = 0.f;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(fmaf(sacc[kb][r], scale_log2, -mref));
        sacc[kb][r] = p;
        lt += p;
      }
    lt += __shfl_xor(lt, 32, 64);
    lrun = fmaf(lrun, corr, lt);
    mrun = mnew;
    // P^T as the B operand of key step k: keys k0 + 16k + 8hf + (0..7)
    u32x4 pb[NPS];
#pragma unroll
    for (int k = 0; k < NPS; ++k)
#pragma unroll
      for (int e = 0; e < 4; ++e)
        pb[k][e] = f32x2_to_bf16x2_bits(sacc[k >> 1][8 * (k & 1) + 2 * e], sacc[k >> 1][8 * (k & 1) + 2 * e + 1]);
    // O^T = O^T * corr + V^T P^T: register rr of block db holds O[query col][d = 32 db + 8 (rr / 4) + 4 hf + rr % 4];
    // once the running maxima settle most tiles change none of the wave's (corr == 1 exactly)
    if (__builtin_amdgcn_ballot_w64(corr != 1.f)) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[db][r] *= corr;
    }
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int k = 0; k < NPS; ++k)
#pragma unroll
      for (int db = 0; db < NDB; ++db) o[db] = mfma32(vt_frag(b, db, k), pb[k], o[db]);
    __builtin_amdgcn_s_setprio(0);
    }
    if (it + 1 < rounds) {  // uniform over the workgroup
      stage(b ^ 1);
      fetch(k0 + 2 * NS * kPfKeys);  // zeros past the last key
    }
    __syncthreads();
  }

  // stream 1 parks (o, m, l) per lane; its partner wave of stream 0 (same
  // rows, same lane layout) merges them: m = max(m0, m1), each side scaled by
  // 2^(m_side - m). Every LDS read of the loop ended at its last barrier.
  if constexpr (NS == 2) {
  float* park = reinterpret_cast<float*>(&k_lds[0][0][0]) + qb * PW * 64 + lane;
  if (st == 1) {
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) park[(16 * db + r) * 64] = o[db][r];
    park[(16 * NDB) * 64] = mrun;
    park[(16 * NDB + 1) * 64] = lrun;
  }
  __syncthreads();
  if (st != 0) return;  // after the last barrier
  {
    const float mo = park[(16 * NDB) * 64], lo = park[(16 * NDB + 1) * 64];
    const float mm = fmaxf(mrun, mo);  // finite: stream 0 saw key 0 of every row
    const float a = __builtin_amdgcn_exp2f(mrun - mm), c = __builtin_amdgcn_exp2f(mo - mm);
    lrun = fmaf(lrun, a, lo * c);
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[db][r] = fmaf(o[db][r], a, park[(16 * db + r) * 64] * c);
  }
  }

  const int row = row0 + col;
  if (row < len) {
    const float inv = lrun > 0.f ? 1.f / lrun : 0.f;
    bf16_t* op = out + ((int64_t)(q0 + row) * H + h) * DH + 4 * hf;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint2 w;
        w.x = f32x2_to_bf16x2_bits(o[db][4 * i] * inv, o[db][4 * i + 1] * inv);
        w.y = f32x2_to_bf16x2_bits(o[db][4 * i + 2] * inv, o[db][4 * i + 3] * inv);
        *reinterpret_cast<uint2*>(op + 32 * db + 8 * i) = w;
      }
  }
}

}  // namespace wfd

extern "C" {

int wfd_attn_prefill(const void* q, const void* k_cache, const void* v_cache, int64_t kv_block_rows,
                     const int64_t* seg_row_base, const int32_t* seg_q_start, const int32_t* seg_pos0, void* out,
                     int nseg, int max_seg_len, int H, int Hkv, int Dh, int dtype, float scale, hipStream_t stream) {
  using namespace wfd;
  if (nseg < 0 || max_seg_len < 0 || H <= 0 || Hkv <= 0 || H % Hkv != 0 || kv_block_rows < 0) {
    set_error("wfd_attn_prefill: bad shape nseg=%d max_seg_len=%d H=%d Hkv=%d", nseg, max_seg_len, H, Hkv);
    return kBadArg;
  }
  if (nseg == 0 || max_seg_len == 0) return kOk;
  if (!q || !k_cache || !v_cache || !seg_row_base || !seg_q_start || !seg_pos0 || !out) {
    set_error("wfd_attn_prefill: null pointer argument");
    return kBadArg;
  }
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out) & 15) {
    set_error("wfd_attn_prefill: q, the caches and out must be 16-byte aligned");
    return kBadArg;
  }
  if (dtype != kBF16 || (Dh != 64 && Dh != 128)) {
    set_error("wfd_attn_prefill: unsupported dtype=%d Dh=%d (bf16, Dh 64/128)", dtype, Dh);
    return kUnsupported;
  }
  const int qtiles = (max_seg_len + kPfRows - 1) / kPfRows;
  if (qtiles > 65535 || nseg > 65535) {
    set_error("wfd_attn_prefill: max_seg_len=%d / nseg=%d beyond the grid", max_seg_len, nseg);
    return kUnsupported;
  }
  // one-stream segments (longer than pf_split_max_rows(H)) and two-stream
  // ones: the kernel of each kind runs if the launch can hold that kind
  const float sl2 = scale * 1.4426950408889634f;
  const int split_max = pf_split_max_rows(H);
#define WFD_PF(DHV, NSV, QT)                                                                                   \
  hipLaunchKernelGGL((attn_prefill_kernel<DHV, NSV>), dim3(H, QT, nseg), dim3(64 * kPfWaves * NSV), 0, stream,   \
                     (const bf16_t*)q, (const bf16_t*)k_cache, (const bf16_t*)v_cache, kv_block_rows, seg_row_base, \
                     seg_q_start, seg_pos0, (bf16_t*)out, H, Hkv, sl2)
  if (max_seg_len > split_max) {
    if (Dh == 64) WFD_PF(64, 1, qtiles);
    else WFD_PF(128, 1, qtiles);
  }
  if (max_seg_len <= split_max || nseg > 1) {
    const int qt2 = (min(max_seg_len, split_max) + kPfRows - 1) / kPfRows;
    if (Dh == 64) WFD_PF(64, 2, qt2);
    else WFD_PF(128, 2, qt2);
  }
#undef WFD_PF
  return launch_status("wfd_attn_prefill");
}

}  // extern "C"
