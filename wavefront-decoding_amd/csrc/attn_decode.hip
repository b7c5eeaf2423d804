// Wavefront decode attention over per-depth KV slot caches, read in place.
//
// Replaces the reference's per-token R attention: n gathers of every slot
// prefix + torch.cat into a packed K/V copy + one FA2 varlen call
// (src/decoding/parcae_blocks.py:458-470 -> fa4_attention.py:301-317,348-366;
// batch: huginn_blocks_batch.py:265-285 + fa4_attention.py:320-342; graph:
// graph_blocks.py:40-43,186-194), and the coda per-query cutoff
// (fa4_attention.py:240-291), which is the same operation with
// kv_len = query position + 1.
//
// For query i and head h (kv head g = h / G):
//   o[i,h,:] = softmax_t( q[i,h,:] . K[row_base[i] + t, g, :] * scale ) @ V[row_base[i] + t, g, :],
//   t = 0 .. kv_len[i]-1, fp32 softmax and accumulation.
//
// Layout: row_base[i] is the cache row of position 0 of query i's slot (for
// the batched cache (slot*B + b)*S, src/decoding/batch_kv_cache.py:64-65), so
// key position == row offset. The cache is token-major (rows, Hkv, Dh) or
// head-major blocks (rows / block_rows, Hkv, block_rows, Dh) (kv_offset); with
// blocks, a query's rows lie in one block, so each workgroup streams one
// contiguous run of Dh-element rows per tensor -- on MI355X ~20% more HBM
// bandwidth than the 2 KB-strided rows of the token-major layout.
//
// Work split (a function of kv_len only, never of n or of other queries, so
// results are row-invariant): keys are cut into 1024-key splits; a workgroup
// of 8 waves owns one (split, kv head, query), and its waves take the split's
// key tiles round-robin (TK keys per tile: 64 for Dh 64, 32 for Dh 128, 64
// VGPRs of K and V fragments per lane), each keeping an online softmax. QK^T runs on MFMA (q rows = the G query heads of the kv
// head, padded to 16; K tile as the B operand: whole key rows turned into
// fragments through the wave's LDS for one query row per workgroup, 16-byte
// fragments straight from HBM for grouped rows); P.V runs on the VALU in fp32 with one 16-byte V
// fragment per lane per key, so K and V are each read exactly once. The waves
// merge through LDS in fixed order. A query whose keys fit one split (every
// decode query up to 1024 keys) is finished in its workgroup; longer ones
// leave per-split partials that a second kernel merges in fixed split order.
// A launch of fewer than 256 such workgroups splits each in two by output
// columns (both read all of K, each half of V; see attn_vsplit): the same
// arithmetic per column, so the same bits.
// 1024 rather than 2048 keys per split: with ragged lengths (the batched
// decode) the longest workgroups set the launch's tail, and halving them made
// the B=32 decode 13 % faster; uniform long prefixes lose ~2-3 %.
#include <mutex>

#include "wfd_common.h"

namespace wfd {

constexpr int kAttnSplit = 1024;  // keys per workgroup

__device__ __forceinline__ float attn_finish(float O, float L) { return L > 0.f ? O / L : 0.f; }

// One workgroup = (split, kv head g, group of QG query rows that share a slot).
// MFMA row m = j * G + r carries query row j of the group at query head
// g * G + r (NR = QG * G rows; the rest of the 16 are zero padding). Every
// row's arithmetic -- its scores, its mask (keys < its own kv_len), its
// online softmax statistics, its P.V accumulation order and the merge -- is
// the same whichever group it sits in, so grouping changes no bits: a group
// only reads the shared prefix once instead of once per row.
template <typename T, int DH, int G, int QG, int NW, int TK>
__global__ __launch_bounds__(64 * NW) void attn_split_kernel(const T* __restrict__ q, const T* __restrict__ kc,
                                                             const T* __restrict__ vc,
                                                             const int64_t* __restrict__ row_base,
                                                             const int32_t* __restrict__ kv_len,
                                                             const int32_t* __restrict__ group_first,
                                                             float* __restrict__ part_o, float* __restrict__ part_ml,
                                                             T* __restrict__ out, int H, int Hkv, int max_splits,
                                                             float scale_log2, int64_t block_rows, int vsplit) {
  constexpr int V = Elem<T>::kVec;
  constexpr int KSTEP = 4 * V;
  constexpr int NDS = DH / KSTEP;  // MFMA k-steps per 16-key block
  constexpr int NJ = TK / 16;      // 16-key blocks per tile
  constexpr int LPR = DH / V;      // lanes covering one V row
  constexpr int RG = 64 / LPR;     // V row groups per wave
  constexpr int KPL = TK / RG;     // V rows per lane per tile
  constexpr int NR = QG * G;       // real MFMA rows
  static_assert(DH % KSTEP == 0 && 64 % LPR == 0 && TK % 16 == 0 && TK % RG == 0 && NR <= 16, "unsupported tile");

  // K through LDS (KCO): one query row per workgroup (NR = G <= 4 MFMA rows)
  // in bf16, whose LDS is otherwise at most 20 KB. A K fragment load (16 keys x 64 bytes per
  // instruction) streams at about half the rate of whole key rows per
  // instruction; each wave instead loads its tile's key rows whole (KPI rows
  // per instruction, lane l: key KPI s + l / LPK, 16-byte piece
  // (l % LPK) ^ key), stores them to its LDS block as loaded, and reads the
  // MFMA B fragments back (lane l, step st: key l % 16, piece 4 st + l / 16).
  // The same values reach the same lanes, so the bits are the same.
  constexpr bool KCO = NR <= 4 && sizeof(T) == 2;
  constexpr int LPK = DH / V;    // 16-byte pieces (lanes) per key row
  constexpr int KPI = 64 / LPK;  // key rows per load instruction
  static_assert(!KCO || (64 % LPK == 0 && NDS * 64 == 16 * LPK), "key row layout");
  __shared__ __align__(16) u32x4 k_lds[KCO ? NW : 1][KCO ? NJ * NDS * 64 : 1];
  __shared__ float p_lds[NW][NR][TK];
  __shared__ float o_lds[NW][NR][DH];
  __shared__ float m_lds[NW][NR];
  __shared__ float l_lds[NW][NR];

  const int split = blockIdx.x;
  const int g = blockIdx.y;
  // V split: grid z = vsplit x (rows or groups); part vp owns output columns
  // [vp * DV, vp * DV + DV) and loads only their V fragments (K whole)
  const int nz = gridDim.z / vsplit;
  const int vp = blockIdx.z / nz;
  const int zi = blockIdx.z - vp * nz;
  const int DV = DH / vsplit;
  const int d0 = vp * DV;
  const int q0 = group_first ? group_first[zi] : zi;
  const int qn = group_first ? min(group_first[zi + 1] - q0, QG) : 1;
  if (qn <= 0) return;  // empty group slot (uniform)
  int lenq[QG];
  int maxlen = 0;
#pragma unroll
  for (int j = 0; j < QG; ++j) {
    lenq[j] = j < qn ? kv_len[q0 + j] : 0;
    maxlen = max(maxlen, lenq[j]);
  }
  if (split * kAttnSplit >= maxlen) {  // uniform for the whole workgroup
    // a group whose rows have no keys at all (kv_len <= 0): its first split
    // writes their zero rows (the flash-attention convention for a query that
    // attends nothing)
    if (split == 0)
      for (int idx = threadIdx.x; idx < qn * G * DV; idx += 64 * NW)
        Elem<T>::store(out + ((int64_t)(q0 + idx / (G * DV)) * H + g * G + (idx / DV) % G) * DH + d0 + idx % DV, 0.f);
    return;
  }
  const int kend_max = min(maxlen, (split + 1) * kAttnSplit);
  const int ntiles = (kend_max - split * kAttnSplit + TK - 1) / TK;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int vg = lane / LPR;
  const int dseg = lane % LPR;
  // this lane's V columns belong to the part (the others load nothing and
  // accumulate zeros: the part's columns get exactly the unsplit arithmetic)
  const bool vmine = dseg * V >= d0 && dseg * V < d0 + DV;
  const int64_t hb = kv_offset(row_base[q0], g, Hkv, DH, block_rows);  // position 0, kv head g
  const int64_t rs = block_rows > 1 ? (int64_t)DH : (int64_t)Hkv * DH;  // key stride
  const T* kb = kc + hb;
  const T* vb = vc + hb;

  // this lane's 4 score rows (4*grp + r) and their key bounds in this split
  int kend4[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * grp + r;
    int e = -1;  // padding row: every key masked
#pragma unroll
    for (int j = 0; j < QG; ++j)
      if (m < NR && m / G == j && j < qn) e = min(lenq[j], (split + 1) * kAttnSplit);
    kend4[r] = e;
  }

  u32x4 qf[NDS];
  {
    const int m = col;  // A-operand row of this lane
    const bool real = m < NR && m / G < qn;
    const int j = real ? m / G : 0;
    const int hq = g * G + (real ? m % G : 0);
    const T* qp = q + ((int64_t)(q0 + j) * H + hq) * DH + grp * V;
#pragma unroll
    for (int s = 0; s < NDS; ++s) qf[s] = real ? ld16(qp + s * KSTEP) : zero16();
  }

  // running softmax state of this wave per row: max (log2 domain), sum, output
  float mrun[NR], lrun[NR], o[NR][V];
#pragma unroll
  for (int m = 0; m < NR; ++m) {
    mrun[m] = -INFINITY;
    lrun[m] = 0.f;
#pragma unroll
    for (int e = 0; e < V; ++e) o[m][e] = 0.f;
  }

  for (int t = wave; t < ntiles; t += NW) {  // uniform over the wave
    const int t0 = split * kAttnSplit + t * TK;
    // every load of the tile first: K (MFMA B fragments), V
    u32x4 kf[NJ][NDS];
    if constexpr (KCO) {  // whole key rows, turned into fragments through LDS below
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int s = 0; s < NDS; ++s) {
          const int r = KPI * s + lane / LPK;  // key within the 16-key block
          const int key = min(t0 + 16 * j + r, maxlen - 1);
          kf[j][s] = ld16(kb + (int64_t)key * rs + ((lane % LPK) ^ (r % LPK)) * V);
        }
    } else {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int key = min(t0 + 16 * j + col, maxlen - 1);
        const T* p = kb + (int64_t)key * rs + grp * V;
#pragma unroll
        for (int s = 0; s < NDS; ++s) kf[j][s] = ld16(p + s * KSTEP);
      }
    }
    u32x4 vf[KPL];
#pragma unroll
    for (int k = 0; k < KPL; ++k) {
      const int key = min(t0 + RG * k + vg, maxlen - 1);
      vf[k] = vmine ? ld16(vb + (int64_t)key * rs + dseg * V) : zero16();
    }

    if constexpr (KCO) {
      // the LDS executes one wave's accesses in order: the previous tile's
      // fragment reads come before these stores, the stores before the reads
      asm volatile("" ::: "memory");
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int s = 0; s < NDS; ++s) k_lds[wave][(j * NDS + s) * 64 + lane] = kf[j][s];
      asm volatile("" ::: "memory");
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int s = 0; s < NDS; ++s)
          kf[j][s] = k_lds[wave][j * NDS * 64 + col * LPK + ((4 * s + grp) ^ (col % LPK))];
    }
    // scores: lane (grp, col) holds S[row 4*grp + r][key 16j + col] in acc[j][r]
    f32x4 acc[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NDS; ++s) acc[j] = mfma_step<T>(qf[s], kf[j][s], acc[j]);
    }
    // per row: the 16 lanes of its group reduce max and sum over the tile's
    // keys, then every lane takes the row's statistics from the group's first lane
    float mt4[4], lt4[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float mt = -INFINITY;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const bool valid = (t0 + 16 * j + col) < kend4[r];
        const float sv = valid ? acc[j][r] * scale_log2 : -INFINITY;
        acc[j][r] = sv;
        mt = fmaxf(mt, sv);
      }
#pragma unroll
      for (int sh = 8; sh >= 1; sh >>= 1) mt = fmaxf(mt, __shfl_xor(mt, sh, 64));
      mt4[r] = mt;
    }
    float corr[NR];
    float mnew4[4];
#pragma unroll
    for (int m = 0; m < NR; ++m) {
      const float mt = __uint_as_float(__shfl(__float_as_uint(mt4[m % 4]), 16 * (m / 4), 64));
      const float mnew = fmaxf(mrun[m], mt);
      corr[m] = (mrun[m] == -INFINITY) ? 0.f : exp2f(mrun[m] - mnew);
      mrun[m] = mnew;
      if (m / 4 == grp) mnew4[m % 4] = mnew;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      // lanes of a padding row group keep mnew4 unset: give them -inf (their p are 0)
      const float mn = (4 * grp + r < NR) ? mnew4[r] : -INFINITY;
      float lt = 0.f;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const float p = (acc[j][r] == -INFINITY) ? 0.f : exp2f(acc[j][r] - mn);
        acc[j][r] = p;
        lt += p;
      }
#pragma unroll
      for (int sh = 8; sh >= 1; sh >>= 1) lt += __shfl_xor(lt, sh, 64);
      lt4[r] = lt;
    }
#pragma unroll
    for (int m = 0; m < NR; ++m) {
      const float lt = __uint_as_float(__shfl(__float_as_uint(lt4[m % 4]), 16 * (m / 4), 64));
      lrun[m] = fmaf(lrun[m], corr[m], lt);
    }
    // P to this wave's LDS rows, in the V lanes' key order
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * grp + r;
      if (m < NR) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int kt = 16 * j + col;  // key within the tile
          p_lds[wave][m][(kt % RG) * KPL + kt / RG] = acc[j][r];
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // P.V on the VALU: lane owns V columns [dseg*V, dseg*V+V) of keys RG*k + vg
#pragma unroll
    for (int m = 0; m < NR; ++m)
#pragma unroll
      for (int e = 0; e < V; ++e) o[m][e] *= corr[m];
#pragma unroll
    for (int k = 0; k < KPL; ++k) {
      float v[V];
      Elem<T>::unpack(vf[k], v);
#pragma unroll
      for (int m = 0; m < NR; ++m) {
        const float p = p_lds[wave][m][vg * KPL + k];
#pragma unroll
        for (int e = 0; e < V; ++e) o[m][e] = fmaf(p, v[e], o[m][e]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();  // P rows are rewritten by the next tile
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
#pragma unroll
  for (int sh = LPR; sh < 64; sh <<= 1)
#pragma unroll
    for (int m = 0; m < NR; ++m)
#pragma unroll
      for (int e = 0; e < V; ++e) o[m][e] += __shfl_xor(o[m][e], sh, 64);
  if (vg == 0) {
#pragma unroll
    for (int m = 0; m < NR; ++m)
#pragma unroll
      for (int e = 0; e < V; ++e) o_lds[wave][m][dseg * V + e] = o[m][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int m = 0; m < NR; ++m) {
      m_lds[wave][m] = mrun[m];
      l_lds[wave][m] = lrun[m];
    }
  }
  __syncthreads();

  // Merge the NW waves in fixed order. A row whose keys fit one split is
  // finished here (the split merge over one split, exactly as
  // attn_combine_kernel computes it); otherwise it leaves this split's
  // unnormalised partial. Rows with no keys in this split write nothing.
  for (int idx = threadIdx.x; idx < NR * DV; idx += 64 * NW) {
    const int m = idx / DV;
    const int d = d0 + (idx - m * DV);
    const int j = m / G;
    int len = 0;
#pragma unroll
    for (int jj = 0; jj < QG; ++jj)
      if (jj == j) len = lenq[jj];
    if (j >= qn) continue;
    if (len <= 0) {  // no keys: a zero row, written once
      if (split == 0) Elem<T>::store(out + ((int64_t)(q0 + j) * H + g * G + (m - j * G)) * DH + d, 0.f);
      continue;
    }
    if (split * kAttnSplit >= len) continue;
    int ns = (len + kAttnSplit - 1) / kAttnSplit;
    ns = ns < max_splits ? ns : max_splits;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, m_lds[w][m]);
    float O = 0.f, L = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float mw = m_lds[w][m];
      const float f = (mw == -INFINITY) ? 0.f : exp2f(mw - M);
      O = fmaf(o_lds[w][m][d], f, O);
      L = fmaf(l_lds[w][m], f, L);
    }
    const int i = q0 + j;
    const int h = g * G + (m - j * G);
    if (ns == 1) {
      const float f = (M == -INFINITY) ? 0.f : exp2f(M - M);
      Elem<T>::store(out + ((int64_t)i * H + h) * DH + d, attn_finish(fmaf(O, f, 0.f), fmaf(L, f, 0.f)));
    } else {
      const int64_t pidx = ((int64_t)i * H + h) * max_splits + split;
      part_o[pidx * DH + d] = O;
      if (d == 0) {
        part_ml[pidx * 2] = M;
        part_ml[pidx * 2 + 1] = L;
      }
    }
  }
}

// Merge of a row's split partials, in split order: M = max m_s, then
// L = sum l_s * 2^(m_s - M) and O = sum o_s * 2^(m_s - M), one fma per split.
// The partials are read in batches of kCombineBatch independent loads, so a
// row of many splits waits on memory twice per batch, not twice per split.
constexpr int kCombineBatch = 8;

template <typename T, int DH>
__global__ __launch_bounds__(DH) void attn_combine_kernel(const float* __restrict__ part_o,
                                                          const float* __restrict__ part_ml,
                                                          const int32_t* __restrict__ kv_len, T* __restrict__ out,
                                                          int H, int max_splits) {
  constexpr int B = kCombineBatch;
  const int h = blockIdx.x;
  const int i = blockIdx.y;
  const int d = threadIdx.x;
  const int len = kv_len[i];
  int ns = len > 0 ? (len + kAttnSplit - 1) / kAttnSplit : 0;
  ns = min(ns, max_splits);
  if (ns <= 1) return;  // finished by its split workgroup
  const int64_t base = ((int64_t)i * H + h) * max_splits;
  float M = -INFINITY;
  for (int s0 = 0; s0 < ns; s0 += B) {
    float mv[B];
#pragma unroll
    for (int b = 0; b < B; ++b) mv[b] = s0 + b < ns ? part_ml[(base + s0 + b) * 2] : -INFINITY;
#pragma unroll
    for (int b = 0; b < B; ++b) M = fmaxf(M, mv[b]);
  }
  float O = 0.f, L = 0.f;
  for (int s0 = 0; s0 < ns; s0 += B) {
    float mv[B], lv[B], ov[B];
#pragma unroll
    for (int b = 0; b < B; ++b) {
      const bool ok = s0 + b < ns;
      mv[b] = ok ? part_ml[(base + s0 + b) * 2] : -INFINITY;
      lv[b] = ok ? part_ml[(base + s0 + b) * 2 + 1] : 0.f;
      ov[b] = ok ? part_o[(base + s0 + b) * DH + d] : 0.f;
    }
#pragma unroll
    for (int b = 0; b < B; ++b) {
      if (s0 + b < ns) {
        const float f = (mv[b] == -INFINITY) ? 0.f : exp2f(mv[b] - M);
        L = fmaf(lv[b], f, L);
        O = fmaf(ov[b], f, O);
      }
    }
  }
  Elem<T>::store(out + ((int64_t)i * H + h) * DH + d, attn_finish(O, L));
}

// Per-row tables of a packed varlen call (the FA varlen convention): query
// row r of segment s (rows [cu_q[s], cu_q[s+1]), keys [cu_k[s], cu_k[s+1]) of
// a token-major K / V) reads keys from row cu_k[s]; non-causal it reads the
// whole segment, causal (bottom-right) keys [0, k_len - q_len + r - cu_q[s]].
// Rows at or past cu_q[nseg] get no keys. One thread per row, a binary search
// over cu_q: the tables never leave the device.
__global__ void varlen_rows_kernel(const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k, int nseg,
                                   int total_q, int causal, int64_t* __restrict__ row_base,
                                   int32_t* __restrict__ kv_len) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= total_q) return;
  int lo = 0, hi = nseg;  // find the last s with cu_q[s] <= r
  if (nseg <= 0 || r >= cu_q[nseg] || r < cu_q[0]) {
    row_base[r] = 0;
    kv_len[r] = 0;
    return;
  }
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (cu_q[mid] <= r)
      lo = mid;
    else
      hi = mid;
  }
  const int qs = cu_q[lo], ql = cu_q[lo + 1] - qs;
  const int ks = cu_k[lo], kl = cu_k[lo + 1] - ks;
  row_base[r] = ks;
  kv_len[r] = causal ? max(kl - ql + (r - qs) + 1, 0) : kl;
}

static int max_splits_for(int kv_len_max) { return kv_len_max <= 0 ? 1 : (kv_len_max + kAttnSplit - 1) / kAttnSplit; }

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

static size_t attn_ws_bytes(int n, int H, int Dh, int kv_len_max) {
  const size_t ms = (size_t)max_splits_for(kv_len_max);
  return align256((size_t)n * H * ms * Dh * sizeof(float)) + align256((size_t)n * H * ms * 2 * sizeof(float));
}

// Largest group of query rows one workgroup takes: 8 MFMA rows (NR = QG * G),
// what the per-row output registers and LDS of 8 waves hold.
constexpr int kAttnGroupRows = 8;
constexpr int group_max_rows(int G) { return G >= kAttnGroupRows ? 1 : kAttnGroupRows / G; }

// V split of a launch: a workgroup per (split, kv head, row) streams from one
// CU at ~35-40 GB/s, so a launch of fewer workgroups than the chip has CUs is
// bound by its longest workgroups, not by HBM (one bs=1 layer tick: 8 rows x
// 16 heads = 128). Splitting each in two by output columns cuts the bytes one
// workgroup streams to its whole K plus half its V (K is then read twice).
// Measured on the 2048-d model's layer tick (8 rows, 512-778 keys): 15.2 ->
// 13.7 us; 2 rows 12.3 -> 10.7 us; 4 and 8 parts are slower (21 / 35 us),
// since the repeated K reads reach HBM again whatever the dispatch order.
// Every column keeps the unsplit arithmetic, so the split changes no bits.
constexpr int kAttnFillWorkgroups = 256;
constexpr int kAttnMaxVSplit = 2;

static int attn_vsplit(int ms, int Hkv, int n, int DH) {
  const int64_t base = (int64_t)ms * Hkv * n;
  int vs = 1;
  while (vs < kAttnMaxVSplit && base * vs < kAttnFillWorkgroups && DH % (16 * vs) == 0) vs *= 2;
  return vs;
}

template <typename T, int DH, int G>
static void launch_attn(const void* q, const void* kc, const void* vc, const int64_t* rb, const int32_t* kl,
                        const int32_t* gf, void* out, int n, int H, int Hkv, int ms, float scale, int64_t br,
                        float* po, float* pml, hipStream_t st) {
  const float scale_log2 = scale * 1.4426950408889634f;
  constexpr int TK = DH == 64 ? 64 : 32;  // key tile that fits the registers
  constexpr int NW = 8;  // waves per workgroup: 8 beat 4 and 16 on every measured shape
  constexpr int QG = group_max_rows(G);
  const int vs = attn_vsplit(ms, Hkv, n, DH);
  if (gf)
    hipLaunchKernelGGL((attn_split_kernel<T, DH, G, QG, NW, TK>), dim3(ms, Hkv, n * vs), dim3(64 * NW), 0, st,
                       (const T*)q, (const T*)kc, (const T*)vc, rb, kl, gf, po, pml, (T*)out, H, Hkv, ms, scale_log2,
                       br, vs);
  else
    hipLaunchKernelGGL((attn_split_kernel<T, DH, G, 1, NW, TK>), dim3(ms, Hkv, n * vs), dim3(64 * NW), 0, st,
                       (const T*)q, (const T*)kc, (const T*)vc, rb, kl, gf, po, pml, (T*)out, H, Hkv, ms, scale_log2,
                       br, vs);
  if (ms > 1)  // some query may span several splits
    hipLaunchKernelGGL((attn_combine_kernel<T, DH>), dim3(H, n), dim3(DH), 0, st, po, pml, kl, (T*)out, H, ms);
}

template <typename T>
static int dispatch_attn(int Dh, int G, const void* q, const void* kc, const void* vc, const int64_t* rb,
                         const int32_t* kl, const int32_t* gf, void* out, int n, int H, int Hkv, int ms, float scale,
                         int64_t br, float* po, float* pml, hipStream_t st) {
#define WFD_ATTN_CASE(DHV, GV)                                                              \
  if (Dh == DHV && G == GV) {                                                               \
    launch_attn<T, DHV, GV>(q, kc, vc, rb, kl, gf, out, n, H, Hkv, ms, scale, br, po, pml, st); \
    return kOk;                                                                             \
  }
  WFD_ATTN_CASE(64, 1)
  WFD_ATTN_CASE(64, 2)
  WFD_ATTN_CASE(64, 4)
  WFD_ATTN_CASE(128, 1)
  WFD_ATTN_CASE(128, 2)
  WFD_ATTN_CASE(128, 4)
#undef WFD_ATTN_CASE
  return kUnsupported;
}

// Scratch of wfd_attn_decode_noalloc: the split partials of one launch live
// in this file-scope device array instead of a caller's workspace. Each
// device that runs the library holds its own copy until the process ends.
// Host code never passes the array's name to a kernel (on the host it is only
// a stand-in for the symbol): it resolves the device address once per device
// with hipGetSymbolAddress and passes that.
constexpr size_t kAttnScratchBytes = (size_t)WFD_ATTN_NOALLOC_MAX_BYTES;
__device__ __align__(256) unsigned char scratch[kAttnScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_addr[kMaxDevices] = {};

// Device address of `scratch` on the current device (resolved on the first
// call per device), or nullptr with the error set.
static void* attn_scratch(void) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("wfd_attn_decode_noalloc: no current device (or device index %d beyond %d)", dev, kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_addr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_error("wfd_attn_decode_noalloc: hipGetSymbolAddress failed on device %d: %s", dev, hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_addr[dev] = p;
  }
  return g_scratch_addr[dev];
}

}  // namespace wfd

extern "C" {

int wfd_attn_varlen_rows(const int32_t* cu_q, const int32_t* cu_k, int nseg, int total_q, int causal,
                         int64_t* kv_row_base, int32_t* kv_len, hipStream_t stream) {
  using namespace wfd;
  if (nseg < 0 || total_q < 0) {
    set_error("wfd_attn_varlen_rows: bad shape nseg=%d total_q=%d", nseg, total_q);
    return kBadArg;
  }
  if (total_q == 0) return kOk;
  if (!cu_q || !cu_k || !kv_row_base || !kv_len) {
    set_error("wfd_attn_varlen_rows: null pointer argument");
    return kBadArg;
  }
  hipLaunchKernelGGL(varlen_rows_kernel, dim3((total_q + 255) / 256), dim3(256), 0, stream, cu_q, cu_k, nseg, total_q,
                     causal ? 1 : 0, kv_row_base, kv_len);
  return launch_status("wfd_attn_varlen_rows");
}

size_t wfd_attn_workspace_bytes(int n, int H, int Dh, int kv_len_max) {
  if (n < 0 || H <= 0 || Dh <= 0) return 0;
  return wfd::attn_ws_bytes(n, H, Dh, kv_len_max);
}

int wfd_attn_split_keys(void) { return wfd::kAttnSplit; }

int wfd_attn_group_max_rows(int H, int Hkv) {
  if (H <= 0 || Hkv <= 0 || H % Hkv != 0) return 0;
  return wfd::group_max_rows(H / Hkv);
}

int wfd_attn_decode(const void* q, const void* k_cache, const void* v_cache, int64_t kv_block_rows,
                    const int64_t* kv_row_base, const int32_t* kv_len, const int32_t* group_first, void* out, int n,
                    int H, int Hkv, int Dh, int dtype, float scale, int kv_len_max, void* workspace, size_t ws_bytes,
                    hipStream_t stream) {
  using namespace wfd;
  if (n < 0 || H <= 0 || Hkv <= 0 || H % Hkv != 0 || kv_len_max < 1 || kv_block_rows < 0 ||
      (kv_block_rows > 1 && kv_len_max > kv_block_rows)) {
    set_error("wfd_attn_decode: bad shape n=%d H=%d Hkv=%d kv_len_max=%d kv_block_rows=%lld", n, H, Hkv, kv_len_max,
              (long long)kv_block_rows);
    return kBadArg;
  }
  if (n == 0) return kOk;
  if (!q || !k_cache || !v_cache || !kv_row_base || !kv_len || !out || !workspace) {
    set_error("wfd_attn_decode: null pointer argument");
    return kBadArg;
  }
  if (((uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out | (uintptr_t)workspace) & 15) {
    set_error("wfd_attn_decode: q, the caches, out and workspace must be 16-byte aligned");
    return kBadArg;
  }
  const int G = H / Hkv;
  const int ms = max_splits_for(kv_len_max);
  const size_t need = attn_ws_bytes(n, H, Dh, kv_len_max);
  if (ws_bytes < need) {
    set_error("wfd_attn_decode: workspace %zu bytes < required %zu", ws_bytes, need);
    return kWorkspace;
  }
  float* po = (float*)workspace;
  float* pml = (float*)((char*)workspace + align256((size_t)n * H * ms * Dh * sizeof(float)));
  int rc;
  if (dtype == kBF16)
    rc = dispatch_attn<bf16_t>(Dh, G, q, k_cache, v_cache, kv_row_base, kv_len, group_first, out, n, H, Hkv, ms,
                               scale, kv_block_rows, po, pml, stream);
  else if (dtype == kF32)
    rc = dispatch_attn<float>(Dh, G, q, k_cache, v_cache, kv_row_base, kv_len, group_first, out, n, H, Hkv, ms,
                              scale, kv_block_rows, po, pml, stream);
  else
    rc = kUnsupported;
  if (rc != kOk) {
    set_error("wfd_attn_decode: unsupported dtype=%d Dh=%d G=%d (supported: Dh 64/128, G 1/2/4)", dtype, Dh, G);
    return rc;
  }
  return launch_status("wfd_attn_decode");
}



int wfd_attn_decode_noalloc(const void* q, const void* k_cache, const void* v_cache, int64_t kv_block_rows,
                            const int64_t* kv_row_base, const int32_t* kv_len, const int32_t* group_first, void* out,
                            int n, int H, int Hkv, int Dh, int dtype, float scale, int kv_len_max,
                            hipStream_t stream) {
  using namespace wfd;
  if (n > 0 && H > 0 && Dh > 0 && kv_len_max >= 1) {
    const size_t need = attn_ws_bytes(n, H, Dh, kv_len_max);
    if (need > kAttnScratchBytes) {
      set_error("wfd_attn_decode_noalloc: this launch needs %zu bytes of split partials, more than the %zu-byte "
                "static scratch (n=%d H=%d Dh=%d kv_len_max=%d); use wfd_attn_decode with a workspace",
                need, kAttnScratchBytes, n, H, Dh, kv_len_max);
      return kWorkspace;
    }
  }
  if (n == 0) return wfd_attn_decode(q, k_cache, v_cache, kv_block_rows, kv_row_base, kv_len, group_first, out, n,
                                     H, Hkv, Dh, dtype, scale, kv_len_max, nullptr, 0, stream);
  void* ws = nullptr;
  if (n > 0 && H > 0 && Dh > 0) {  // shape errors are reported by the shared path below
    ws = attn_scratch();
    if (!ws) return kLaunch;
  }
  return wfd_attn_decode(q, k_cache, v_cache, kv_block_rows, kv_row_base, kv_len, group_first, out, n, H, Hkv, Dh,
                         dtype, scale, kv_len_max, ws, kAttnScratchBytes, stream);
}

}  // extern "C"
