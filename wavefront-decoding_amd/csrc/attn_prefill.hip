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
// Work split: a workgroup of 4 waves owns 64 consecutive query rows of one
// segment and one query head; wave w owns rows 16w..16w+15. Per 64-key tile:
// the workgroup stages K (row-major) and V (transposed) in LDS; each wave
// computes S = Q K^T with v_mfma_f32_16x16x32_bf16 (Q fragments held in
// registers for the whole sweep), runs an online softmax per row (the 16
// lanes of a row group exchange max and sum by shuffles), rounds P to bf16
// through its LDS rows into the MFMA A layout, and accumulates O += P V on
// MFMA. Tiles past the diagonal are never visited; the diagonal tile masks
// keys past each row's position. Tiles are dispatched longest first.
#include "wfd_common.h"

namespace wfd {

constexpr int kPfRows = 64;  // query rows per workgroup (4 waves x 16)
constexpr int kPfKeys = 64;  // keys per tile

template <int DH>
__global__ __launch_bounds__(256) void attn_prefill_kernel(const bf16_t* __restrict__ q, const bf16_t* __restrict__ kc,
                                                           const bf16_t* __restrict__ vc, int64_t block_rows,
                                                           const int64_t* __restrict__ seg_row_base,
                                                           const int32_t* __restrict__ seg_q_start,
                                                           const int32_t* __restrict__ seg_pos0,
                                                           bf16_t* __restrict__ out, int H, int Hkv,
                                                           float scale_log2) {
  constexpr int V = 8;                // bf16 per 16-byte fragment
  constexpr int NDS = DH / 32;        // MFMA k-steps over Dh (S = Q K^T)
  constexpr int NCB = DH / 16;        // 16-column blocks of O
  constexpr int NKB = kPfKeys / 16;   // 16-key column blocks of S
  constexpr int NPS = kPfKeys / 32;   // MFMA k-steps over keys (O += P V)
  constexpr int KP = DH + 8;          // padded LDS row of K (elements)
  constexpr int VP = kPfKeys + 8;     // padded LDS row of V^T
  constexpr int PP = kPfKeys + 8;     // padded LDS row of P
  constexpr int CPR = DH / V;         // 16-byte chunks per K/V row
  __shared__ __align__(16) bf16_t k_lds[kPfKeys * KP];
  __shared__ __align__(16) bf16_t vt_lds[DH * VP];
  __shared__ __align__(16) bf16_t p_lds[4][16 * PP];

  const int s = blockIdx.z;
  const int h = blockIdx.y;
  const int q0 = seg_q_start[s];
  const int len = seg_q_start[s + 1] - q0;
  const int tq = (len + kPfRows - 1) / kPfRows - 1 - (int)blockIdx.x;  // longest tiles first
  if (tq < 0) return;  // uniform for the workgroup
  const int pos0 = seg_pos0[s];
  const int g = h / (H / Hkv);
  const int64_t hb = kv_offset(seg_row_base[s], g, Hkv, DH, block_rows);
  const int64_t rs = block_rows > 1 ? (int64_t)DH : (int64_t)Hkv * DH;
  const bf16_t* kb = kc + hb;
  const bf16_t* vb = vc + hb;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int row0 = tq * kPfRows + wave * 16;  // segment row of this wave's first query
  const int last_row = min((tq + 1) * kPfRows, len) - 1;
  const int kv_hi = pos0 + last_row + 1;      // keys [0, kv_hi) cover every row of the tile
  const int ntiles = (kv_hi + kPfKeys - 1) / kPfKeys;

  // Q as the MFMA A operand: row col of this wave, k-group grp
  u32x4 qf[NDS];
  {
    const int r = min(row0 + col, len - 1);
    const bf16_t* qp = q + ((int64_t)(q0 + r) * H + h) * DH + grp * V;
#pragma unroll
    for (int k = 0; k < NDS; ++k) qf[k] = ld16(qp + k * 32);
  }
  float mrun[4], lrun[4];
  f32x4 o[NCB];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    mrun[r] = -INFINITY;
    lrun[r] = 0.f;
  }
#pragma unroll
  for (int c = 0; c < NCB; ++c) o[c] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int t = 0; t < ntiles; ++t) {
    const int k0 = t * kPfKeys;
    // stage the tile: K rows as they are, V transposed (d-major), keys past
    // kv_hi clamped to the last one (masked below)
#pragma unroll
    for (int c = threadIdx.x; c < kPfKeys * CPR; c += 256) {
      const int kr = c / CPR;
      const int d0 = (c - kr * CPR) * V;
      const int key = min(k0 + kr, kv_hi - 1);
      const u32x4 kv = ld16(kb + (int64_t)key * rs + d0);
      const u32x4 vv = ld16(vb + (int64_t)key * rs + d0);
      *reinterpret_cast<u32x4*>(&k_lds[kr * KP + d0]) = kv;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        reinterpret_cast<uint16_t*>(vt_lds)[(d0 + 2 * e) * VP + kr] = (uint16_t)(vv[e] & 0xffffu);
        reinterpret_cast<uint16_t*>(vt_lds)[(d0 + 2 * e + 1) * VP + kr] = (uint16_t)(vv[e] >> 16);
      }
    }
    __syncthreads();

    // S = Q K^T: lane holds S[4*grp + r][16*cb + col]
    f32x4 sacc[NKB];
#pragma unroll
    for (int cb = 0; cb < NKB; ++cb) {
      sacc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < NDS; ++k) {
        const u32x4 bfr = *reinterpret_cast<const u32x4*>(&k_lds[(16 * cb + col) * KP + 32 * k + grp * V]);
        sacc[cb] = mfma_step<bf16_t>(qf[k], bfr, sacc[cb]);
      }
    }
    // online softmax over this tile, one row per (grp, r)
    float corr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int qpos = pos0 + row0 + 4 * grp + r;
      float mt = -INFINITY;
#pragma unroll
      for (int cb = 0; cb < NKB; ++cb) {
        const bool ok = k0 + 16 * cb + col <= qpos;
        const float sv = ok ? sacc[cb][r] * scale_log2 : -INFINITY;
        sacc[cb][r] = sv;
        mt = fmaxf(mt, sv);
      }
#pragma unroll
      for (int m = 8; m >= 1; m >>= 1) mt = fmaxf(mt, __shfl_xor(mt, m, 64));
      const float mnew = fmaxf(mrun[r], mt);
      corr[r] = (mrun[r] == -INFINITY) ? 0.f : exp2f(mrun[r] - mnew);
      float lt = 0.f;
#pragma unroll
      for (int cb = 0; cb < NKB; ++cb) {
        const float p = (sacc[cb][r] == -INFINITY) ? 0.f : exp2f(sacc[cb][r] - mnew);
        sacc[cb][r] = p;
        lt += p;
      }
#pragma unroll
      for (int m = 8; m >= 1; m >>= 1) lt += __shfl_xor(lt, m, 64);
      lrun[r] = fmaf(lrun[r], corr[r], lt);
      mrun[r] = mnew;
    }
    // P (bf16) into this wave's LDS rows, then back as A fragments (row col,
    // keys 32*k + 8*grp .. +7)
    uint16_t* pw = reinterpret_cast<uint16_t*>(p_lds[wave]);
#pragma unroll
    for (int cb = 0; cb < NKB; ++cb)
#pragma unroll
      for (int r = 0; r < 4; ++r) pw[(4 * grp + r) * PP + 16 * cb + col] = f32_to_bf16_bits(sacc[cb][r]);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    u32x4 pa[NPS];
#pragma unroll
    for (int k = 0; k < NPS; ++k) pa[k] = *reinterpret_cast<const u32x4*>(&pw[col * PP + 32 * k + grp * V]);

    // O = O * corr + P V: lane holds O[4*grp + r][16*cb + col]
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) o[cb][r] *= corr[r];
#pragma unroll
      for (int k = 0; k < NPS; ++k) {
        const u32x4 bfr = *reinterpret_cast<const u32x4*>(&vt_lds[(16 * cb + col) * VP + 32 * k + grp * V]);
        o[cb] = mfma_step<bf16_t>(pa[k], bfr, o[cb]);
      }
    }
    __syncthreads();  // K / V^T are restaged by the next tile
  }

#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int row = row0 + 4 * grp + r;
    if (row < len) {
      bf16_t* op = out + ((int64_t)(q0 + row) * H + h) * DH + col;
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb)
        Elem<bf16_t>::store(op + 16 * cb, lrun[r] > 0.f ? o[cb][r] / lrun[r] : 0.f);
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
  if (dtype != kBF16 || (Dh != 64 && Dh != 128)) {
    set_error("wfd_attn_prefill: unsupported dtype=%d Dh=%d (bf16, Dh 64/128)", dtype, Dh);
    return kUnsupported;
  }
  const dim3 grid((max_seg_len + kPfRows - 1) / kPfRows, H, nseg);
  const float sl2 = scale * 1.4426950408889634f;
  if (Dh == 64)
    hipLaunchKernelGGL(attn_prefill_kernel<64>, grid, dim3(256), 0, stream, (const bf16_t*)q, (const bf16_t*)k_cache,
                       (const bf16_t*)v_cache, kv_block_rows, seg_row_base, seg_q_start, seg_pos0, (bf16_t*)out, H,
                       Hkv, sl2);
  else
    hipLaunchKernelGGL(attn_prefill_kernel<128>, grid, dim3(256), 0, stream, (const bf16_t*)q,
                       (const bf16_t*)k_cache, (const bf16_t*)v_cache, kv_block_rows, seg_row_base, seg_q_start,
                       seg_pos0, (bf16_t*)out, H, Hkv, sl2);
  return launch_status("wfd_attn_prefill");
}

}  // extern "C"
