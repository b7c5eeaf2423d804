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
// Work split: a workgroup of 4 waves owns 128 consecutive query rows of one
// segment and one query head; wave w owns rows 32w..32w+31 as two blocks of
// 16, one query per lane column in each. Per 64-key tile the workgroup stages
// K (row-major) and V (transposed, d-major) in LDS, with the next tile's
// global loads (32-bit buffer offsets, nothing read past the segment's last
// key) issued before the current tile's math so their latency hides under
// it. Each wave computes S^T = K Q^T on v_mfma_f32_16x16x32_bf16 -- every K
// fragment read from LDS feeds both query blocks -- so a lane holds 16 of its
// query's 64 scores: the online softmax needs two shuffles per statistic (the
// scale folds into the exponent's FMA), and P stays in registers as the B
// operand of O^T = V^T P^T (the k order inside an MFMA step only has to agree
// between A and B; each V^T fragment again feeds both blocks). The lane's
// output column is its own query, so the softmax rescale needs no exchange.
// Tiles past the diagonal are never visited; the diagonal tiles mask keys
// past each row's position (tiles below them skip the mask). Query tiles are
// dispatched longest first.
#include "wfd_common.h"

namespace wfd {

constexpr int kPfWaves = 8;
constexpr int kPfQB = 1;                        // 16-query blocks per wave
constexpr int kPfRows = 16 * kPfQB * kPfWaves;  // query rows per workgroup
constexpr int kPfKeys = 64;                     // keys per tile

template <int DH>
__global__ __launch_bounds__(64 * kPfWaves) void attn_prefill_kernel(
    const bf16_t* __restrict__ q, const bf16_t* __restrict__ kc, const bf16_t* __restrict__ vc, int64_t block_rows,
    const int64_t* __restrict__ seg_row_base, const int32_t* __restrict__ seg_q_start,
    const int32_t* __restrict__ seg_pos0, bf16_t* __restrict__ out, int H, int Hkv, float scale_log2) {
  constexpr int NT = 64 * kPfWaves;   // threads
  constexpr int V = 8;                // bf16 per 16-byte fragment
  constexpr int NDS = DH / 32;        // MFMA k-steps over Dh (S^T = K Q^T)
  constexpr int NDB = DH / 16;        // 16-row blocks of O^T (head dim)
  constexpr int NKB = kPfKeys / 16;   // 16-key blocks of S^T
  constexpr int NPS = kPfKeys / 32;   // MFMA k-steps over keys (O^T += V^T P^T)
  constexpr int KP = DH + 8;          // padded LDS row of K (elements)
  constexpr int VP = kPfKeys + 8;     // padded LDS row of V^T
  constexpr int CPR = DH / V;         // 16-byte chunks per K row
  constexpr int KCH = kPfKeys * CPR / NT;      // K chunks per thread per tile
  constexpr int VUN = kPfKeys / 2 * CPR;       // V key-pair chunks per tile
  constexpr int VCH = VUN >= NT ? VUN / NT : 1;  // ... per thread (fewer chunks than threads: the first waves)
  static_assert(KCH >= 1 && kPfKeys * CPR % NT == 0 && (VUN % NT == 0 || NT % VUN == 0), "tile split");
  static_assert(VUN >= NT || VUN % 64 == 0, "V staging must be wave-uniform");
  __shared__ __align__(16) bf16_t k_lds[kPfKeys * KP];
  __shared__ __align__(16) bf16_t vt_lds[DH * VP];

  const int s = blockIdx.z;
  const int h = blockIdx.y;
  const int q0 = seg_q_start[s];
  const int len = seg_q_start[s + 1] - q0;
  const int tq = (len + kPfRows - 1) / kPfRows - 1 - (int)blockIdx.x;  // longest tiles first
  if (tq < 0) return;  // uniform for the workgroup
  const int pos0 = seg_pos0[s];
  const int g = h / (H / Hkv);
  const int64_t hb = kv_offset(seg_row_base[s], g, Hkv, DH, block_rows);
  const uint32_t rsb = (uint32_t)((block_rows > 1 ? DH : Hkv * DH) * sizeof(bf16_t));  // key stride, bytes

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int row0 = tq * kPfRows + wave * 16 * kPfQB;
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

  // Q as the MFMA B operand: column col of block qb = query row0 + 16 qb + col, k-group grp
  u32x4 qf[kPfQB][NDS];
#pragma unroll
  for (int qb = 0; qb < kPfQB; ++qb) {
    const int r = min(row0 + 16 * qb + col, len - 1);
    const bf16_t* qp = q + ((int64_t)(q0 + r) * H + h) * DH + grp * V;
#pragma unroll
    for (int k = 0; k < NDS; ++k) qf[qb][k] = ld16(qp + k * 32);
  }

  // staging: thread's K chunks (key, 8 dims) and V key-pair chunks (2 keys, 8 dims)
  u32x4 kreg[KCH], vreg[VCH][2];
  auto fetch = [&](int k0) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = threadIdx.x + i * NT;
      const int kr_ = c / CPR;
      kreg[i] = buf_ld16(kr, (uint32_t)(k0 + kr_) * rsb + (uint32_t)((c - kr_ * CPR) * V * sizeof(bf16_t)));
    }
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int c = threadIdx.x + i * NT;
      if (VUN < NT && c >= VUN) break;  // wave-uniform
      const int kp = c / CPR;
      const uint32_t off = (uint32_t)(k0 + 2 * kp) * rsb + (uint32_t)((c - kp * CPR) * V * sizeof(bf16_t));
      vreg[i][0] = buf_ld16(vr, off);
      vreg[i][1] = buf_ld16(vr, off + rsb);
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int c = threadIdx.x + i * NT;
      const int kr_ = c / CPR;
      *reinterpret_cast<u32x4*>(&k_lds[kr_ * KP + (c - kr_ * CPR) * V]) = kreg[i];
    }
    uint32_t* vt = reinterpret_cast<uint32_t*>(vt_lds);
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int c = threadIdx.x + i * NT;
      if (VUN < NT && c >= VUN) break;  // wave-uniform
      const int kp = c / CPR;
      const int d0 = (c - kp * CPR) * V;
#pragma unroll
      for (int e = 0; e < 4; ++e) {  // dims d0 + 2e, d0 + 2e + 1: (key 2kp, key 2kp+1) pairs
        const uint32_t a = vreg[i][0][e], b = vreg[i][1][e];
        vt[((d0 + 2 * e) * VP + 2 * kp) >> 1] = (a & 0xffffu) | (b << 16);
        vt[((d0 + 2 * e + 1) * VP + 2 * kp) >> 1] = (a >> 16) | (b & 0xffff0000u);
      }
    }
  };

  float mrun[kPfQB], lrun[kPfQB];
  f32x4 o[kPfQB][NDB];
#pragma unroll
  for (int qb = 0; qb < kPfQB; ++qb) {
    mrun[qb] = -INFINITY;
    lrun[qb] = 0.f;
#pragma unroll
    for (int c = 0; c < NDB; ++c) o[qb][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  fetch(0);
  for (int t = 0; t < ntiles; ++t) {
    const int k0 = t * kPfKeys;
    stage();
    __syncthreads();
    fetch(k0 + kPfKeys);  // next tile (zeros past the last key): in flight under this tile's math
    // keys past some row's position only in the diagonal tiles (uniform per wave)
    const bool full = k0 + kPfKeys - 1 <= pos0 + row0;

    // S^T = K Q^T: lane holds S[query 16 qb + col][key k0 + 16 cb + 4 grp + r]
    f32x4 sacc[kPfQB][NKB];
#pragma unroll
    for (int cb = 0; cb < NKB; ++cb) {
#pragma unroll
      for (int qb = 0; qb < kPfQB; ++qb) sacc[qb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < NDS; ++k) {
        const u32x4 afr = *reinterpret_cast<const u32x4*>(&k_lds[(16 * cb + col) * KP + 32 * k + grp * V]);
#pragma unroll
        for (int qb = 0; qb < kPfQB; ++qb) sacc[qb][cb] = mfma_step<bf16_t>(afr, qf[qb][k], sacc[qb][cb]);
      }
    }
    // online softmax per query (log2 domain: p = 2^(s * scale_log2 - m)); the
    // first tile holds key 0 for every row, so m is finite from then on and
    // masked scores (-inf) give p = 0 without a test
    u32x4 pb[kPfQB][NPS];
    float corr[kPfQB];
#pragma unroll
    for (int qb = 0; qb < kPfQB; ++qb) {
      const int qpos = pos0 + row0 + 16 * qb + col;
      float mt = -INFINITY;
#pragma unroll
      for (int cb = 0; cb < NKB; ++cb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (!full && k0 + 16 * cb + 4 * grp + r > qpos) sacc[qb][cb][r] = -INFINITY;
          mt = fmaxf(mt, sacc[qb][cb][r]);
        }
      mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      const float mnew = fmaxf(mrun[qb], mt * scale_log2);
      corr[qb] = exp2f(mrun[qb] - mnew);
      float lt = 0.f;
#pragma unroll
      for (int cb = 0; cb < NKB; ++cb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = exp2f(fmaf(sacc[qb][cb][r], scale_log2, -mnew));
          sacc[qb][cb][r] = p;
          lt += p;
        }
      lt += __shfl_xor(lt, 16, 64);
      lt += __shfl_xor(lt, 32, 64);
      lrun[qb] = fmaf(lrun[qb], corr[qb], lt);
      mrun[qb] = mnew;
      // P^T as the B operand of step k: keys k0 + 32k + 4grp + (0..3) then
      // k0 + 32k + 16 + 4grp + (0..3) -- the order the V^T fragments use below
#pragma unroll
      for (int k = 0; k < NPS; ++k) {
        pb[qb][k][0] = f32x2_to_bf16x2_bits(sacc[qb][2 * k][0], sacc[qb][2 * k][1]);
        pb[qb][k][1] = f32x2_to_bf16x2_bits(sacc[qb][2 * k][2], sacc[qb][2 * k][3]);
        pb[qb][k][2] = f32x2_to_bf16x2_bits(sacc[qb][2 * k + 1][0], sacc[qb][2 * k + 1][1]);
        pb[qb][k][3] = f32x2_to_bf16x2_bits(sacc[qb][2 * k + 1][2], sacc[qb][2 * k + 1][3]);
      }
    }
    // O^T = O^T * corr + V^T P^T: lane holds O[query 16 qb + col][d = 16 db + 4 grp + r]
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int qb = 0; qb < kPfQB; ++qb)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[qb][db][r] *= corr[qb];
#pragma unroll
      for (int k = 0; k < NPS; ++k) {
        const bf16_t* vp = &vt_lds[(16 * db + col) * VP + 32 * k + 4 * grp];
        const uint2 lo = *reinterpret_cast<const uint2*>(vp);
        const uint2 hi = *reinterpret_cast<const uint2*>(vp + 16);
        const u32x4 afr = {lo.x, lo.y, hi.x, hi.y};
#pragma unroll
        for (int qb = 0; qb < kPfQB; ++qb) o[qb][db] = mfma_step<bf16_t>(afr, pb[qb][k], o[qb][db]);
      }
    }
    __syncthreads();  // K / V^T are restaged by the next tile
  }

#pragma unroll
  for (int qb = 0; qb < kPfQB; ++qb) {
    const int row = row0 + 16 * qb + col;
    if (row < len) {
      const float inv = lrun[qb] > 0.f ? 1.f / lrun[qb] : 0.f;
      bf16_t* op = out + ((int64_t)(q0 + row) * H + h) * DH + 4 * grp;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        uint2 w;
        w.x = f32x2_to_bf16x2_bits(o[qb][db][0] * inv, o[qb][db][1] * inv);
        w.y = f32x2_to_bf16x2_bits(o[qb][db][2] * inv, o[qb][db][3] * inv);
        *reinterpret_cast<uint2*>(op + 16 * db) = w;
      }
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
  const dim3 block(64 * kPfWaves);
  const float sl2 = scale * 1.4426950408889634f;
  if (Dh == 64)
    hipLaunchKernelGGL(attn_prefill_kernel<64>, grid, block, 0, stream, (const bf16_t*)q, (const bf16_t*)k_cache,
                       (const bf16_t*)v_cache, kv_block_rows, seg_row_base, seg_q_start, seg_pos0, (bf16_t*)out, H,
                       Hkv, sl2);
  else
    hipLaunchKernelGGL(attn_prefill_kernel<128>, grid, block, 0, stream, (const bf16_t*)q,
                       (const bf16_t*)k_cache, (const bf16_t*)v_cache, kv_block_rows, seg_row_base, seg_q_start,
                       seg_pos0, (bf16_t*)out, H, Hkv, sl2);
  return launch_status("wfd_attn_prefill");
}

}  // extern "C"
