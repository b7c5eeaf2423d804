/*
 * wfd.h -- C ABI of the MI355X wavefront-decode library (libwfd.so).
 *
 * Every compute entry point is stream-ordered on the caller's hipStream_t,
 * allocates nothing, never synchronizes and throws nothing: it returns 0 on
 * success or a negative status (WFD_BAD_ARG, WFD_UNSUPPORTED, WFD_LAUNCH,
 * WFD_WORKSPACE) and leaves a message for wfd_last_error(). All tensors are
 * plain device pointers to contiguous row-major storage; `dtype` is
 * WFD_F32 (0) or WFD_BF16 (1). Lengths, positions and row tables are device
 * data, so a launch sequence can be captured once in a hipGraph and replayed
 * as the wave advances. Row tables (x_rows, flat_row, kv_row_base, ...) are
 * trusted: the caller guarantees they index inside the buffers it passes.
 *
 * KV slot caches: a cache row is one token position of one (slot, sequence);
 * `kv_block_rows` picks the layout of the K and V buffers:
 *   0 or 1: token-major (rows, Hkv, Dh) -- the reference's slot buffer layout;
 *   B >= 2: head-major blocks (rows / B, Hkv, B, Dh): element (row, h, d) at
 *           ((row / B * Hkv + h) * B + row % B) * Dh + d.
 * With B = the slot length S, each (slot, sequence) is one block and a
 * query's keys of one head are one contiguous run, which attention streams
 * ~20% faster than token-major rows.
 *
 * Each entry point names the reference interface (file:line under the
 * reference checkout) whose work it replaces.
 */
#ifndef WFD_H_
#define WFD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* wfd_stream_t; /* == hipStream_t */

enum { WFD_F32 = 0, WFD_BF16 = 1 };
enum { WFD_OK = 0, WFD_BAD_ARG = -1, WFD_UNSUPPORTED = -2, WFD_LAUNCH = -3, WFD_WORKSPACE = -4 };
enum { WFD_EPI_PLAIN = 0, WFD_EPI_SWIGLU = 1 };

/* Message for the last failing call on this thread. */
const char* wfd_last_error(void);
/* Bumped whenever an entry point's signature changes or one is added (5: wfd_argmax's
   accept flags, wfd_attn_varlen_rows; 6: wfd_linear_argmax, wfd_argmax_groups;
   7: folded norm pairs -- wfd_linear_prep, wfd_norm_prep, the row-scale argument of
   wfd_linear, wfd_linear_qkv_rope_append and wfd_linear_argmax). */
int wfd_abi_version(void);

/*
 * Folded RMSNorm pairs (decode). A block's residual stream is kept as r (one
 * dtype row per token) and the per-row scale s of the norm that last
 * normalized it: the residual the block adds is x = round((r * s) * w) (w
 * that norm's weight; without a norm, x = r). A linear that reads a pair of
 * norms -- first a (weight wa; may be absent), then b (weight wb) -- of
 * r does not read the normalized row: it reads A = round((r * wa) * wb) and
 * multiplies its fp32 output by scale = s_a * s_b, where
 *   s_a = 1 / sqrt(sum(r^2) / D + eps)             (1 when a is absent),
 *   s_b = 1 / sqrt(s_a^2 * sum((r * wa)^2) / D + eps),
 * which is norm_b(norm_a(r)) applied after the product instead of before it.
 * The linear that produces r (proj, the MLP down projection, the adapter)
 * computes r = round(y + x), A and the sums in its epilogue, so no launch
 * sits between the two linears. The sums are reduced in one fixed order
 * wherever they are formed: per 8-column group g (columns 8g..8g+7) the tree
 * ((c0+c1)+(c2+c3))+((c4+c5)+(c6+c7)) of the squares; the groups are dealt
 * to the 64 lanes of a wave as wfd_linear's chunk layout deals a row's
 * elements (lane c + 16 j takes, for s = 0..3, the group of elements
 * 128 c + 32 s + 8 j for bf16, or 64 c + 16 s + 8 (j / 2) for fp32 from the
 * even j), each lane adds its groups in s order from +0, and the 64 lane sums
 * meet in a butterfly (xor 32, 16, ..., 1). Every product and sum is rounded
 * on its own (no fused multiply-add). So a row's bits never depend on n or on
 * which kernels formed them. Rows up to 2048 (bf16) / 1024 (fp32) wide.
 */
typedef struct wfd_prep {
  const void* r_in;   /* residual stream to add (NULL: none) ... */
  int64_t ld_in;
  const float* s_in;  /* ... its per-row scale (NULL: 1) ... */
  const void* w_in;   /* ... and norm weight (NULL: none): x = round((r_in * s_in) * w_in) */
  void* r_out;        /* r = round(y + x), or y without r_in (NULL: not kept) */
  int64_t ld_out;
  void* a_out;        /* the next linear's operand A = round((r * wa) * wb) */
  int64_t ld_a;
  const void* wa;     /* the next pair's weights (wa NULL: norm a absent) */
  const void* wb;
  float* part;        /* wfd_linear_prep: the two sums of each 8-column group, 256 float pairs per row
                         (16-byte aligned), group g of row m at pair m * 256 + 4 (c + 16 j) + s for the
                         lane (c, j) and step s that take it (above) */
} wfd_prep_t;

typedef struct wfd_rowscale {
  const float* scale; /* the per-row scale s_a * s_b (from wfd_norm_prep), or NULL and ... */
  const float* part;  /* ... the group sums a wfd_linear_prep left (few-row launches only; 16-byte aligned) */
  int D;              /* row width of r (a multiple of 128 bf16 / 64 fp32 values) */
  int two;            /* 1: norm a present; 0: absent (s_a = 1) */
  float eps;
  float* s_out;       /* with part: s_a per row (NULL: not kept) */
} wfd_rowscale_t;

/*
 * Wavefront decode attention (per-query slot prefix, read in place).
 * Replaces: fa4_attention.attn_varlen / _attn_varlen_torch
 *   (src/decoding/fa4_attention.py:301-317,348-366) as called by
 *   ParcaeBlocks._core_attn_varlen (src/decoding/parcae_blocks.py:458-470),
 *   attn_varlen_q1_padded (fa4_attention.py:320-342) as called by
 *   HuginnBlocksBatch._union_attn (src/decoding/huginn_blocks_batch.py:282-285),
 *   the graph path _fa_varlen (src/decoding/graph_blocks.py:40-43,186-194),
 *   and attn_cutoff_multi (fa4_attention.py:240-291) -- a per-query cutoff is
 *   kv_len = position + 1.
 * q: (n, H, Dh); k_cache/v_cache: KV caches in the kv_block_rows layout;
 * out: (n, H, Dh). Query i attends rows kv_row_base[i] .. kv_row_base[i] +
 * kv_len[i] - 1 (with blocks, rows of one block). kv_len_max >= every
 * kv_len[i] sizes the grid (and must not exceed a block); workspace >=
 * wfd_attn_workspace_bytes(n, H, Dh, kv_len_max). A query with kv_len <= 0
 * gets a zero output row. Dh in {64, 128};
 * H / Hkv in {1, 2, 4}. q, the caches, out and workspace are 16-byte aligned.
 * group_first (optional, device int32, n + 1 entries): group g = query rows
 * [group_first[g], group_first[g+1]) -- rows that share one slot (the same
 * kv_row_base), at most wfd_attn_group_max_rows(H, Hkv) of them; a workgroup
 * then reads the shared prefix once for the whole group (draft-then-verify
 * sources, a coda's verify + draft). Entries past the last group repeat
 * group_first[ngroups] (empty groups). Every row's output bits are the same
 * with or without grouping. NULL: one row per group.
 * (wide-wavefront grouping replaces the grouped causal calls of
 * _core_attn_varlen, src/decoding/parcae_blocks.py:391-456, and the coda
 * grouping of huginn_blocks_batch.py:331-343.)
 */
size_t wfd_attn_workspace_bytes(int n, int H, int Dh, int kv_len_max);
int wfd_attn_split_keys(void);
int wfd_attn_group_max_rows(int H, int Hkv);
int wfd_attn_decode(const void* q, const void* k_cache, const void* v_cache, int64_t kv_block_rows,
                    const int64_t* kv_row_base, const int32_t* kv_len, const int32_t* group_first, void* out, int n,
                    int H, int Hkv, int Dh, int dtype, float scale, int kv_len_max, void* workspace, size_t ws_bytes,
                    wfd_stream_t stream);

/*
 * wfd_attn_decode without a workspace argument: the split partials go to a
 * static scratch array inside the library (WFD_ATTN_NOALLOC_MAX_BYTES per
 * device, held by every device the library runs on until the process ends),
 * so the call allocates nothing, for callers that cannot allocate (code
 * under hipGraph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It has no counterpart in the reference. Same arguments, same
 * kernels and the same output bits as wfd_attn_decode; a launch whose
 * partials need more than the maximum (wfd_attn_workspace_bytes(n, H, Dh,
 * kv_len_max) > WFD_ATTN_NOALLOC_MAX_BYTES) is rejected with WFD_WORKSPACE.
 * Every call on a device shares that device's scratch: calls that overlap on
 * one device (concurrent streams) race. Nothing in it needs clearing: a
 * launch writes every partial it reads.
 */
#define WFD_ATTN_NOALLOC_MAX_BYTES (32u << 20)
int wfd_attn_decode_noalloc(const void* q, const void* k_cache, const void* v_cache, int64_t kv_block_rows,
                            const int64_t* kv_row_base, const int32_t* kv_len, const int32_t* group_first, void* out,
                            int n, int H, int Hkv, int Dh, int dtype, float scale, int kv_len_max,
                            wfd_stream_t stream);

/*
 * Row tables of a packed varlen attention call, built on the device: query
 * row r of segment s (rows [cu_q[s], cu_q[s+1]) of q; keys [cu_k[s],
 * cu_k[s+1]) of a token-major K / V) gets kv_row_base[r] = cu_k[s] and
 * kv_len[r] = k_len (causal == 0) or max(k_len - q_len + (r - cu_q[s]) + 1, 0)
 * (causal != 0: bottom-right per segment, the FA varlen convention; a row
 * with no keys yields a zero output row from wfd_attn_decode). Rows at or
 * past cu_q[nseg] get kv_len 0. cu_q, cu_k: int32 (nseg + 1), device data;
 * the outputs then feed wfd_attn_decode with kv_block_rows = 0, so the whole
 * call never reads a length back to the host.
 * Replaces: the cu_seqlens handling of fa4_attention.attn_varlen /
 *   _attn_varlen_torch (src/decoding/fa4_attention.py:301-317,348-366).
 */
int wfd_attn_varlen_rows(const int32_t* cu_q, const int32_t* cu_k, int nseg, int total_q, int causal,
                         int64_t* kv_row_base, int32_t* kv_len, wfd_stream_t stream);

/*
 * Causal prefill attention on MFMA (bf16; Dh 64 or 128; any H / Hkv).
 * Segment s owns query rows [seg_q_start[s], seg_q_start[s+1]) of q (n, H, Dh)
 * at positions seg_pos0[s], seg_pos0[s] + 1, ... of one slot whose cache rows
 * start at seg_row_base[s]; query row j attends that slot's keys [0, its
 * position] (bottom-right causal), which must already be appended. out: (n, H,
 * Dh). max_seg_len >= every segment length sizes the grid. Tables are device
 * data. q, the caches and out are 16-byte aligned. A segment of at most
 * (256 / H) * 128 rows is computed with two key streams per workgroup, a
 * longer one with one; the choice depends only on the segment's length and H,
 * so a segment's output bits do not depend on the other segments of the call.
 * Replaces: attn_dense(q, k, v, causal=True) (src/decoding/fa4_attention.py:189-215)
 *   from _block_dense (src/decoding/huginn_blocks_batch.py:163-170), and the
 *   grouped causal segments of _core_attn_varlen (src/decoding/parcae_blocks.py:435-456).
 */
int wfd_attn_prefill(const void* q, const void* k_cache, const void* v_cache, int64_t kv_block_rows,
                     const int64_t* seg_row_base, const int32_t* seg_q_start, const int32_t* seg_pos0, void* out,
                     int nseg, int max_seg_len, int H, int Hkv, int Dh, int dtype, float scale,
                     wfd_stream_t stream);

/*
 * Slot-cache append: cache row flat_row[i] of k_cache / v_cache (layout
 * kv_block_rows) = k[i] / v[i], each (Hkv, Dh).
 * Replaces: StaticKVCache.write_range / write_scatter
 *   (src/decoding/kv_cache.py:97-114), BatchStaticKVCache.write_tokens
 *   (src/decoding/batch_kv_cache.py:61-73), and the graph index_copy_ writes
 *   (src/decoding/graph_blocks.py:172-176,306-310).
 */
int wfd_kv_append(const void* k, const void* v, void* k_cache, void* v_cache, int64_t kv_block_rows,
                  const int64_t* flat_row, int n, int Hkv, int Dh, int dtype, wfd_stream_t stream);

/*
 * SwiGLU of n rows laid out [gate (F) | up (F)] with row stride ldg:
 * out[i][j] = silu(gu[i][j]) * gu[i][F + j] (silu(v) = v / (1 + e^-v)) in
 * fp32, rounded once to `dtype`, row stride ldo. F, ldg and ldo are
 * multiples of 8 (bf16) / 4 (fp32) elements and both pointers 16-byte
 * aligned. The linear layer's SwiGLU epilogue for a gate|up product made
 * elsewhere (the prompt pass's library GEMM).
 * Replaces: the gated MLP's silu(gate) * up inside block.mlp in the prompt
 *   pass (src/decoding/huginn_blocks_batch.py:159-161,163-170).
 */
int wfd_swiglu(const void* gu, int64_t ldg, void* out, int64_t ldo, int n, int F, int dtype, wfd_stream_t stream);

/*
 * Fused QKV epilogue: split qkv rows (n, (H + 2*Hkv) * Dh) into q|k|v, rotate
 * q and k by RoPE at pos[i] (interleaved pairs (2j, 2j+1), angle
 * pos * base^(-2j/Dh), tables (rope_rows, Dh/2) fp32), write q to q_out
 * (n, H, Dh) and append k, v at cache row flat_row[i] (layout kv_block_rows).
 * Replaces: HuginnBlocks._qkv + the cache write
 *   (src/decoding/huginn_blocks.py:77-87,96-97; huginn_blocks_batch.py:147-157,
 *   308-310; graph_blocks.py:296-310).
 */
int wfd_qkv_rope_append(const void* qkv, int64_t ldq, const int32_t* pos, const float* rope_cos,
                        const float* rope_sin, int rope_rows, const int64_t* flat_row, void* q_out, void* k_cache,
                        void* v_cache, int64_t kv_block_rows, int n, int H, int Hkv, int Dh, int dtype,
                        wfd_stream_t stream);

/* Granularity of K for wfd_linear: 128 (bf16) / 64 (fp32) elements. */
int wfd_linear_k_multiple(int dtype);

/*
 * Packs a row-major weight W (N, K) -- nn.Linear layout, for SwiGLU the gate
 * rows [0, pair_off) then the up rows [pair_off, N) -- into the layout
 * wfd_linear and wfd_linear_qkv_rope_append read: MFMA fragment order, tile
 * by tile (16 output columns; a SwiGLU tile pairs 8 gate rows with their 8 up
 * rows), so each weight load of the kernels reads 1 KB of contiguous memory.
 * Same size as W; W_packed must not overlap W. Pack once, at load time.
 * Replaces: nothing in the reference (its weights are read in place by
 *   cuBLAS); the packed copy is the device-resident weight of this library.
 */
int wfd_linear_pack(const void* W, void* W_packed, int N, int K, int dtype, int epilogue, int pair_off,
                    wfd_stream_t stream);

/*
 * Row-invariant linear: y[m, :] = x[x_rows ? x_rows[m] : m, :K] @ W^T with W
 * (N, K) given packed by wfd_linear_pack (same epilogue and pair_off).
 * Epilogue WFD_EPI_SWIGLU: N = 2*pair_off, y[m, j] = silu(g_j) * u_j with
 * g_j = row j, u_j = row pair_off + j of the product. out_dtype may be
 * WFD_F32 for bf16 inputs (logits). K must be a multiple of
 * wfd_linear_k_multiple(dtype), N of 16. K is summed in fixed 128 (bf16) /
 * 64 (fp32) element chunks: the P chunks form wfd_linear_slices(K) slices of
 * Q = ceil(P / 4) chunks, each slice up to 4 sub-slices of ceil(Q / 4)
 * chunks; chunk partials are added in chunk order within a sub-slice,
 * sub-slice sums in order within a slice and slice sums in slice order, each
 * sum from zero in fp32, so y[m] does not depend on n, on where row m sits,
 * or on whether the slices ran in one workgroup or in several
 * (wfd_linear_partials). Every x row read (x_rows[m] * ldx)
 * must lie within the first 2 GiB of x. x, W and the x row pitch (ldx
 * elements) must be 16-byte aligned.
 * Replaces: the nn.Linear calls of the block forwards -- Wqkv, proj, the gated
 *   MLP, adapter, lm_head (src/decoding/huginn_blocks.py:79,100-102,216,291;
 *   huginn_blocks_batch.py:149,160-161,299,345).
 */
int wfd_linear(const void* x, const int32_t* x_rows, int64_t ldx, const void* W, void* y, int64_t ldy, int n, int N,
               int K, int dtype, int out_dtype, int epilogue, int pair_off, const wfd_rowscale_t* rs,
               wfd_stream_t stream);
/* rs (NULL: none): x holds the A rows of a folded norm pair (see wfd_prep_t) and
 * each output row is multiplied by its scale before the epilogue (SwiGLU after
 * the scale). rs->part (group sums) is accepted for n <= 16 only. */

/*
 * A d_model-output linear (plain epilogue, n <= 16) whose epilogue prepares
 * the residual stream and the next linear's operand: with y the linear's fp32
 * output, r = round(y + x) (see wfd_prep_t; x from r_in / s_in / w_in),
 * A = round((r * wa) * wb), and the group sums of r^2 and (r * wa)^2 for the
 * consumer's row scale. W packed (plain). n <= 16 and N a multiple of 16.
 * Replaces: proj / the MLP down projection / the adapter with the residual
 *   add and the residual norms after them (src/decoding/huginn_blocks.py:95,
 *   100-102,216; huginn_blocks_batch.py:159-161,299), whose full-row sums
 *   move into the consuming linear.
 */
int wfd_linear_prep(const void* x, const int32_t* x_rows, int64_t ldx, const void* W, int n, int N, int K, int dtype,
                    const wfd_prep_t* pp, wfd_stream_t stream);

/*
 * The row form of a folded norm pair, one wave per row: the row y is
 * a[i * lda] (part NULL) or the in-order slice sum of wfd_linear_partials'
 * part (rounded to dtype, wfd_linear's output bit for bit); r and A as
 * wfd_linear_prep computes them (r into pp->r_out if given), scale_out[i] =
 * s_a * s_b and s_out[i] = s_a (same sums, same order) when pp->a_out is
 * given; and with h_out, h_out[h_rows ? h_rows[i] : i] = round((r * s_a) * wa),
 * the output of norm a itself -- the normalized residual a many-row pass
 * keeps instead of (r, s_a), or, without pp->a_out, the block's last norm.
 * two = 1 exactly when pp->wa is given (norm a absent: s_a = 1, h = r).
 * D a multiple of 128 (bf16) / 64 (fp32), at most 2048 (bf16) / 1024 (fp32).
 * Replaces: the residual norms after proj, the MLP down projection and the
 *   adapter (src/decoding/huginn_blocks.py:95,101-102,216;
 *   huginn_blocks_batch.py:159-161,299), for many-row unions and for the
 *   last norm of a pass.
 */
int wfd_norm_prep(const void* a, int64_t lda, const float* part, int64_t slice_stride, int nslices,
                  const wfd_prep_t* pp, int two, float eps, float* scale_out, float* s_out, void* h_out,
                  const int32_t* h_rows, int64_t ldh, int n, int D, int dtype, wfd_stream_t stream);

/* Number of K slices of wfd_linear's arithmetic contract for this K (1..4);
 * 0 if K is not a positive multiple of wfd_linear_k_multiple(dtype). */
int wfd_linear_slices(int K, int dtype);

/*
 * Split-K form of wfd_linear (plain epilogue): one workgroup per (64 rows,
 * 32 or 64 columns, K slice), so a many-row projection with few output
 * columns fills the chip and reads each x row once per 32-64 columns. Writes
 * the fp32 slice sums part[(q * n + m) * N + j] for q < wfd_linear_slices(K);
 * adding them in slice order from zero and rounding to dtype gives wfd_linear's
 * y[m, j] bit for bit (wfd_add_rmsnorm_split does exactly that). Shapes,
 * x_rows and alignment as for wfd_linear; part 16-byte aligned.
 * Replaces: the same nn.Linear calls as wfd_linear where the output feeds a
 *   residual norm -- proj, the MLP down projection and the adapter
 *   (src/decoding/huginn_blocks.py:100-102,216; huginn_blocks_batch.py:159-161,299).
 */
int wfd_linear_partials(const void* x, const int32_t* x_rows, int64_t ldx, const void* W, float* part, int n, int N,
                        int K, int dtype, wfd_stream_t stream);

/*
 * The fused q|k|v projection with wfd_qkv_rope_append as its epilogue:
 * qkv = x[x_rows ? x_rows[i] : i] @ Wqkv^T, Wqkv ((H + 2*Hkv) * Dh, K) packed
 * by wfd_linear_pack (plain epilogue), under wfd_linear's arithmetic
 * contract; each qkv value is rounded to `dtype`, then
 * rotated, written and appended exactly as wfd_qkv_rope_append does, so the
 * result equals wfd_linear followed by wfd_qkv_rope_append bit for bit. The
 * qkv rows themselves are never stored. Dh % 16 == 0, K as for wfd_linear.
 * Replaces: the Wqkv projection + HuginnBlocks._qkv + the cache write
 *   (src/decoding/huginn_blocks.py:77-87,96-97; huginn_blocks_batch.py:147-157,
 *   308-310; graph_blocks.py:296-310).
 */
int wfd_linear_qkv_rope_append(const void* x, const int32_t* x_rows, int64_t ldx, const void* Wqkv, int n, int K,
                               const int32_t* pos, const float* rope_cos, const float* rope_sin, int rope_rows,
                               const int64_t* flat_row, void* q_out, void* k_cache, void* v_cache,
                               int64_t kv_block_rows, int H, int Hkv, int Dh, int dtype, const wfd_rowscale_t* rs,
                               wfd_stream_t stream);
/* rs as for wfd_linear: the row scale multiplies the qkv values before they are
 * rounded and rotated. */

/*
 * x_out[out_rows ? out_rows[i] : i] = rmsnorm(a[a_rows ? a_rows[i] : i] + res[i]) * w1
 * and, if w2, h_out[i] = rmsnorm(x_out row) * w2. res may be NULL (plain
 * RMSNorm). With w2, x_out may be NULL (not kept). D <= 4096 and a multiple of
 * 128 (bf16) / 64 (fp32); every row 16-byte aligned. One wave per row; the
 * sum of squares is reduced in wfd_linear's chunk order (chunks of 128 / 64
 * elements), so a row's bits never depend on n.
 * Replaces: the SandwichBlock residual norms `norm_2(att + x)`, `norm_3`,
 *   `norm_4(mlp + x)`, `norm_1` and `ln_f`
 *   (src/decoding/huginn_blocks.py:95,101-102,268,290;
 *   huginn_blocks_batch.py:159-161,329,344).
 */
int wfd_add_rmsnorm(const void* a, const int32_t* a_rows, int64_t lda, const void* res, int64_t ldr, const void* w1,
                    const void* w2, void* x_out, const int32_t* out_rows, int64_t ldo, void* h_out, int64_t ldh, int n,
                    int D, float eps, int dtype, wfd_stream_t stream);

/*
 * wfd_add_rmsnorm whose `a` rows come from wfd_linear_partials: row i of `a`
 * is sum_{q < nslices} part[q * slice_stride + i * D + :], added in slice order
 * from zero and rounded to dtype -- wfd_linear's output row, bit for bit. If
 * a_out is given, that row is also stored there (a_out[i * lda_out]); the
 * rest is wfd_add_rmsnorm's math on the same values (a_rows is implicitly
 * the identity). slice_stride >= n * D.
 * Replaces: the residual norms after proj, the MLP down projection and the
 *   adapter (src/decoding/huginn_blocks.py:95,101-102,216;
 *   huginn_blocks_batch.py:160-161,299) with their linear's K reduction.
 */
int wfd_add_rmsnorm_split(const float* part, int64_t slice_stride, int nslices, void* a_out, int64_t lda_out,
                          const void* res, int64_t ldr, const void* w1, const void* w2, void* x_out,
                          const int32_t* out_rows, int64_t ldo, void* h_out, int64_t ldh, int n, int D, float eps,
                          int dtype, wfd_stream_t stream);

/*
 * out[i] = table[id_i] * scale, id_i = ids[i]; a negative ids[i] with a ring
 * is a token handle: id_i = ring[-ids[i] - 1] (the device token ring that
 * wfd_argmax fills), so a sampled token feeds the next prelude without a
 * host round trip. Ids are clamped into [0, vocab).
 * Replaces: wte(ids) * emb_scale (src/decoding/huginn_blocks.py:184-186;
 *   huginn_blocks_batch.py:215-217).
 */
int wfd_embed(const int64_t* ids, const int64_t* ring, int64_t ring_len, const void* table, float scale, void* out,
              int64_t ldo, int n, int vocab, int D, int dtype, wfd_stream_t stream);

/*
 * The opening of a prelude pass in one launch: x_out[i] = wfd_embed's row i
 * (table[id_i] * scale, ids / ring handles as there) if x_out is given,
 * h_out[i] = rmsnorm(that row) * w1 (wfd_add_rmsnorm's math), and, with
 * cp_src, the side copy cp_dst[cp_dst_rows[i], :cp_width] =
 * cp_src[cp_src_rows[i], :cp_width] (the token's initial loop state into its
 * wave-state row). Same bits as wfd_embed + wfd_add_rmsnorm + wfd_copy_rows.
 * D and the row pitches as for wfd_add_rmsnorm; cp_width a multiple of 16 bytes.
 * Replaces: wte(ids) * emb_scale, the first prelude block's norm_1 and the s0
 *   table lookup (src/decoding/huginn_blocks.py:95,184-186,190;
 *   huginn_blocks_batch.py:215-217; parcae_blocks.py:137-146).
 */
int wfd_embed_rmsnorm(const int64_t* ids, const int64_t* ring, int64_t ring_len, const void* table, float scale,
                      int vocab, const void* w1, void* x_out, int64_t ldx, void* h_out, int64_t ldh,
                      const void* cp_src, const int32_t* cp_src_rows, int64_t cp_lds, void* cp_dst,
                      const int32_t* cp_dst_rows, int64_t cp_ldd, int cp_width, int n, int D, float eps, int dtype,
                      wfd_stream_t stream);

/*
 * dst[dst_rows ? dst_rows[i] : i, :width] = src[src_rows ? src_rows[i] : i, :width].
 * Replaces: the per-token torch.stack of hidden/static rows and the s0 table
 *   lookup (src/decoding/huginn_blocks.py:190,205-209; parcae_blocks.py:137-146).
 */
int wfd_copy_rows(const void* src, const int32_t* src_rows, int64_t lds, void* dst, const int32_t* dst_rows,
                  int64_t ldd, int n, int width, int dtype, wfd_stream_t stream);

/*
 * out[i] = argmax_j logits[i, j] (first index on ties), logits fp32, 16-byte
 * aligned; with a ring, also ring[ring_rows[i]] = out[i] (rows outside
 * [0, ring_len) are skipped). With expect / accept (both or neither):
 * accept[i] = 1 if out[i] equals the expected token -- expect[i] >= 0 a plain
 * id, -ring_len <= expect[i] < 0 a ring handle -(slot + 1) whose id an
 * earlier pass wrote -- else 0 (also for any other expect[i]: no comparison).
 * `accept` may be device memory or the device address of mapped, coherent
 * pinned host memory, which the host can then poll for the flags (each flag
 * is one 4-byte store of row i's workgroup) instead of copying them back.
 * Replaces: greedy_sample's argmax and its .item() (src/decoding/acceptance.py:40-44),
 *   greedy_accept's draft == argmax comparison (acceptance.py:47-58), and
 *   coda_argmax_union's argmax + .tolist() (src/decoding/huginn_blocks_batch.py:345-346):
 *   with the ring and the accept flags, ids stay on the device and a greedy
 *   verify reads back one flag per row.
 */
int wfd_argmax(const float* logits, int64_t ld, int64_t* out, int64_t* ring, const int32_t* ring_rows,
               int64_t ring_len, const int64_t* expect, int32_t* accept, int n, int vocab, wfd_stream_t stream);

/*
 * Column groups of wfd_linear_argmax for this shape: the few-row launch's
 * workgroups (a 16-column tile, or half a tile when there are few tiles), or
 * 0 where wfd_linear would not take the few-row kernel (n above 16, a K too
 * long for it) or dtype is not WFD_BF16.
 */
int wfd_linear_argmax_groups(int n, int N, int K, int dtype);

/*
 * wfd_linear with bf16 x / W and fp32 y (plain epilogue; the same kernel, so
 * y has the same bits) that also leaves, for each row m and column group
 * s < G = wfd_linear_argmax_groups(n, N, K, dtype), the first largest value of
 * y[m] over the group's columns and its column index: part_val[m * G + s],
 * part_idx[m * G + s]. wfd_argmax_groups over them gives wfd_argmax(y)'s ids
 * while reading G entries per row instead of N. WFD_UNSUPPORTED where G is 0.
 * Replaces: the lm_head call of the coda (src/decoding/huginn_blocks.py:291;
 *   huginn_blocks_batch.py:345) together with the logits read of
 *   greedy_sample's argmax (src/decoding/acceptance.py:40-44).
 */
int wfd_linear_argmax(const void* x, const int32_t* x_rows, int64_t ldx, const void* W, float* y, int64_t ldy, int n,
                      int N, int K, int dtype, float* part_val, int32_t* part_idx, const wfd_rowscale_t* rs,
                      wfd_stream_t stream);
/* rs as for wfd_linear: the logits are scaled before the group bests are taken. */

/*
 * wfd_argmax from the column-group bests wfd_linear_argmax left (groups per
 * row): out[i] = the first index of row i's largest value, with the same ring
 * and expect / accept semantics as wfd_argmax.
 * Replaces: greedy_sample's argmax and greedy_accept's comparison
 *   (src/decoding/acceptance.py:40-58; huginn_blocks_batch.py:345-346), as wfd_argmax.
 */
int wfd_argmax_groups(const float* part_val, const int32_t* part_idx, int groups, int64_t* out, int64_t* ring,
                      const int32_t* ring_rows, int64_t ring_len, const int64_t* expect, int32_t* accept, int n,
                      wfd_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* WFD_H_ */
