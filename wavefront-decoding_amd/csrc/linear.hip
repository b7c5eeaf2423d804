// Row-invariant skinny linear layer: y[m, :] = x[m, :] @ W^T on MFMA.
//
// Replaces the nn.Linear calls of the block forwards (Wqkv, proj, the gated
// MLP, the adapter, lm_head; src/decoding/huginn_blocks.py:79,100-102,216,291
// and huginn_blocks_batch.py:149,160-161,299,345). At decode M = n is 1..~512
// rows while W is 4-128 MB, so the layer is a weight stream: each weight byte
// is read from HBM once per launch.
//
// Work split: a workgroup owns NT tiles of 16 output features and all rows;
// its 8 waves split K into 8 fixed contiguous ranges. A wave keeps a chunk of
// its weight fragment in registers and sweeps every 16-row M-tile of x over
// it (x comes from L2), accumulating one MFMA per k-step in k order. The 8
// wave partials are summed through LDS in wave order. The k partition and the
// summation order depend only on K, so y[m] is bit-identical whatever n is and
// wherever row m sits -- the property sequential and wavefront decode need to
// agree token for token.
//
// Epilogues: plain store (bf16 or fp32 out) and SwiGLU, where tile 0 is the
// gate feature block and tile 1 the matching up block `pair_off` rows below
// it: out = silu(gate) * up.
#include "wfd_common.h"

namespace wfd {

constexpr int kLinWaves = 8;
enum Epilogue : int { kEpiPlain = 0, kEpiSwiGLU = 1 };

template <typename T, typename TO, int NT, int EPI, int MT, int CH>
__global__ __launch_bounds__(64 * kLinWaves) void linear_kernel(const T* __restrict__ x,
                                                                const int32_t* __restrict__ x_rows, int64_t ldx,
                                                                const T* __restrict__ W, TO* __restrict__ y,
                                                                int64_t ldy, int n, int K, int pair_off) {
  constexpr int V = Elem<T>::kVec;
  constexpr int KSTEP = 4 * V;
  __shared__ float red[kLinWaves][NT][64][4];

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int spw = K / (KSTEP * kLinWaves);  // k-steps per wave
  const int s0 = wave * spw;

  int c0[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (EPI == kEpiSwiGLU)
      c0[t] = (t == 0 ? 0 : pair_off) + blockIdx.x * 16;
    else
      c0[t] = (blockIdx.x * NT + t) * 16;
  }
  const T* wrow[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) wrow[t] = W + (int64_t)(c0[t] + col) * K + grp * V;

  for (int rb = 0; rb < n; rb += MT * 16) {
    f32x4 acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[mt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    int xr[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int row = rb + mt * 16 + col;
      xr[mt] = row < n ? (x_rows ? x_rows[row] : row) : -1;
    }

    for (int ch = 0; ch < spw; ch += CH) {
      u32x4 wf[NT][CH];
#pragma unroll
      for (int s = 0; s < CH; ++s)
#pragma unroll
        for (int t = 0; t < NT; ++t)
          wf[t][s] = (ch + s < spw) ? ld16(wrow[t] + (int64_t)(s0 + ch + s) * KSTEP) : zero16();
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (rb + mt * 16 >= n) break;  // uniform across the workgroup
        u32x4 xf[CH];
        const T* xp = x + (int64_t)(xr[mt] < 0 ? 0 : xr[mt]) * ldx + grp * V;
#pragma unroll
        for (int s = 0; s < CH; ++s)
          xf[s] = (xr[mt] >= 0 && ch + s < spw) ? ld16(xp + (int64_t)(s0 + ch + s) * KSTEP) : zero16();
#pragma unroll
        for (int s = 0; s < CH; ++s) {
          if (ch + s < spw) {
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[mt][t] = mfma_step<T>(xf[s], wf[t][s], acc[mt][t]);
          }
        }
      }
    }

    // Reduce the 8 wave partials of each M-tile in wave order, then store.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (rb + mt * 16 >= n) break;
      __syncthreads();
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][t][lane][r] = acc[mt][t][r];
      __syncthreads();
      const int tid = threadIdx.x;
      const int nthreads_out = (EPI == kEpiSwiGLU) ? 256 : 256 * NT;
      if (tid < nthreads_out) {
        const int t = (EPI == kEpiSwiGLU) ? 0 : tid >> 8;
        const int ln = (tid & 255) >> 2;
        const int r = tid & 3;
        const int m = 4 * (ln >> 4) + r;
        const int cc = ln & 15;
        const int row = rb + mt * 16 + m;
        if (row < n) {
          float v0 = 0.f;
#pragma unroll
          for (int w = 0; w < kLinWaves; ++w) v0 += red[w][t][ln][r];
          float res;
          if (EPI == kEpiSwiGLU) {
            float v1 = 0.f;
#pragma unroll
            for (int w = 0; w < kLinWaves; ++w) v1 += red[w][NT - 1][ln][r];
            res = (v0 / (1.0f + expf(-v0))) * v1;
          } else {
            res = v0;
          }
          const int outc = (EPI == kEpiSwiGLU) ? (blockIdx.x * 16 + cc) : (c0[t] + cc);
          Elem<TO>::store(y + (int64_t)row * ldy + outc, res);
        }
      }
    }
  }
}

template <typename T, typename TO, int NT, int EPI>
static void launch_linear_mt(const void* x, const int32_t* xr, int64_t ldx, const void* W, void* y, int64_t ldy,
                             int n, int N, int K, int pair_off, hipStream_t st) {
  const int groups = (EPI == kEpiSwiGLU) ? pair_off / 16 : N / (16 * NT);
  const dim3 grid(groups), block(64 * kLinWaves);
  // MT only changes how many M-tiles share one weight chunk; per-row
  // arithmetic (k order, wave order) is identical in every variant.
  if (n <= 16)
    hipLaunchKernelGGL((linear_kernel<T, TO, NT, EPI, 1, 8>), grid, block, 0, st, (const T*)x, xr, ldx, (const T*)W,
                       (TO*)y, ldy, n, K, pair_off);
  else if (n <= 32)
    hipLaunchKernelGGL((linear_kernel<T, TO, NT, EPI, 2, 8>), grid, block, 0, st, (const T*)x, xr, ldx, (const T*)W,
                       (TO*)y, ldy, n, K, pair_off);
  else if (n <= 64)
    hipLaunchKernelGGL((linear_kernel<T, TO, NT, EPI, 4, 8>), grid, block, 0, st, (const T*)x, xr, ldx, (const T*)W,
                       (TO*)y, ldy, n, K, pair_off);
  else
    hipLaunchKernelGGL((linear_kernel<T, TO, NT, EPI, 8, 8>), grid, block, 0, st, (const T*)x, xr, ldx, (const T*)W,
                       (TO*)y, ldy, n, K, pair_off);
}

}  // namespace wfd

extern "C" {

// Minimum K granularity: K must be a multiple of this for the given dtype.
int wfd_linear_k_multiple(int dtype) {
  using namespace wfd;
  return (dtype == kBF16 ? 32 : 16) * kLinWaves;
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
  const bool nt2 = (epilogue == kEpiPlain) && (N % 32 == 0);
  if (dtype == kBF16 && out_dtype == kBF16) {
    if (epilogue == kEpiSwiGLU)
      launch_linear_mt<bf16_t, bf16_t, 2, kEpiSwiGLU>(x, x_rows, ldx, W, y, ldy, n, N, K, pair_off, stream);
    else if (nt2)
      launch_linear_mt<bf16_t, bf16_t, 2, kEpiPlain>(x, x_rows, ldx, W, y, ldy, n, N, K, 0, stream);
    else
      launch_linear_mt<bf16_t, bf16_t, 1, kEpiPlain>(x, x_rows, ldx, W, y, ldy, n, N, K, 0, stream);
  } else if (dtype == kBF16 && out_dtype == kF32 && epilogue == kEpiPlain) {
    if (nt2)
      launch_linear_mt<bf16_t, float, 2, kEpiPlain>(x, x_rows, ldx, W, y, ldy, n, N, K, 0, stream);
    else
      launch_linear_mt<bf16_t, float, 1, kEpiPlain>(x, x_rows, ldx, W, y, ldy, n, N, K, 0, stream);
  } else if (dtype == kF32 && out_dtype == kF32) {
    if (epilogue == kEpiSwiGLU)
      launch_linear_mt<float, float, 2, kEpiSwiGLU>(x, x_rows, ldx, W, y, ldy, n, N, K, pair_off, stream);
    else if (nt2)
      launch_linear_mt<float, float, 2, kEpiPlain>(x, x_rows, ldx, W, y, ldy, n, N, K, 0, stream);
    else
      launch_linear_mt<float, float, 1, kEpiPlain>(x, x_rows, ldx, W, y, ldy, n, N, K, 0, stream);
  } else {
    set_error("wfd_linear: unsupported dtype=%d out_dtype=%d epilogue=%d", dtype, out_dtype, epilogue);
    return kUnsupported;
  }
  return launch_status("wfd_linear");
}

}  // extern "C"
