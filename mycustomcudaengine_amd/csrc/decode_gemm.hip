// Decode-sized GEMM for gfx950: out[M, N] (op)= X[M, K] . W[N, K]^T with
// M <= 16 (one token per sequence), fp16 in, fp32 accumulation, fused
// epilogues.  This is the projection work of the engine's decode step
// (engine/models/llama.py:94-174 runs it through torch.matmul); at these
// shapes it is a weight-streaming problem: every W byte is read once and
// the MFMA work is negligible.
//
// Layout of one launch:
//   * a workgroup owns 16 output columns (16 rows of W) -- two 16-row tiles
//     for the SwiGLU epilogue (gate rows j and up rows n + j) -- and has one
//     wave per 512-wide slice of K per tile;
//   * a wave issues all 16 of its W loads (16 rows x 64 bytes per instruction,
//     consecutive instructions covering consecutive 64-byte halves of the same
//     128-byte lines) and its X loads (L2-resident) up front, then runs 16
//     v_mfma_f32_16x16x32_f16: A = W tile (lane l: row l % 16, k 8 (l / 16)
//     .. +7), B = X^T (lane l: token l % 16, same k); tokens >= M are zeros;
//   * the K-slice partials (4 floats per lane: rows 4 (l / 16) .. +3, token
//     l % 16) are summed through LDS and the first wave applies the epilogue.
// Epilogues: STORE  out[m, n] = acc
//            ADD    out[m, n] = out[m, n] + acc   (residual stream in place)
//            SWIGLU out[m, j] = silu(acc_gate[m, j]) * acc_up[m, j], W being
//                   [2 n, K] with the gate rows first (the fused gate/up
//                   weight), so one launch replaces GEMM + SwiGLU.
#include "mce_common.h"

namespace mce {

constexpr int DG_SLICE = 512;       // K per wave
constexpr int DG_CHUNKS = DG_SLICE / 32;
constexpr int DG_MAX_WAVES = 16;    // per workgroup (1024 threads)

struct DecodeGemmArgs {
  const uint16_t *x, *w;
  uint16_t *out;
  int M, N, K;
  int64_t x_stride, out_stride;
};

template <int EPI, int T>  // T tiles per workgroup (2 for SWIGLU)
__global__ __launch_bounds__(DG_MAX_WAVES * 64) void decode_gemm_kernel(DecodeGemmArgs a) {
  const int nw = a.K / DG_SLICE;  // waves per tile
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile = wave / nw, slice = wave - tile * nw;
  const int col0 = blockIdx.x * 16;                   // first output column
  const int wrow0 = col0 + tile * a.N;                // first W row of this tile
  const int r = lane & 15, q = lane >> 4;
  const int k0 = slice * DG_SLICE + 8 * q;

  // all loads of the wave first: 16 W fragments (HBM) and 16 X fragments
  const uint16_t *wp = a.w + (int64_t)(wrow0 + r) * a.K + k0;
  const bool tok_ok = r < a.M;
  const uint16_t *xp = a.x + (int64_t)(tok_ok ? r : 0) * a.x_stride + k0;
  u32x4 wf[DG_CHUNKS], xf[DG_CHUNKS];
#pragma unroll
  for (int c = 0; c < DG_CHUNKS; ++c)
    wf[c] = *reinterpret_cast<const u32x4 *>(wp + 32 * c);
#pragma unroll
  for (int c = 0; c < DG_CHUNKS; ++c)
    xf[c] = tok_ok ? *reinterpret_cast<const u32x4 *>(xp + 32 * c) : u32x4{0, 0, 0, 0};
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < DG_CHUNKS; ++c)
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, wf[c]),
                                                 __builtin_bit_cast(half8, xf[c]), acc, 0, 0, 0);

  // sum the K slices: red[wave][component][lane]
  __shared__ float red[DG_MAX_WAVES][4][64];
#pragma unroll
  for (int i = 0; i < 4; ++i) red[wave][i][lane] = acc[i];
  lds_barrier();
  if (wave != 0) return;
  float v[T][4];
#pragma unroll
  for (int t = 0; t < T; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float s = 0.f;
      for (int sl = 0; sl < nw; ++sl) s += red[t * nw + sl][i][lane];
      v[t][i] = s;
    }
  if (!tok_ok) return;
  // lane holds columns col0 + 4 q .. +3 of token r
  uint16_t *op = a.out + (int64_t)r * a.out_stride + col0 + 4 * q;
  float o[4];
  if constexpr (EPI == 1) {
    const u32x2 old = *reinterpret_cast<const u32x2 *>(op);
    o[0] = F16T::lo(old[0]) + v[0][0];
    o[1] = F16T::hi(old[0]) + v[0][1];
    o[2] = F16T::lo(old[1]) + v[0][2];
    o[3] = F16T::hi(old[1]) + v[0][3];
  } else if constexpr (EPI == 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float g = v[0][i];
      o[i] = g / (1.0f + __expf(-g)) * v[T - 1][i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = v[0][i];
  }
  u32x2 pr;
  pr[0] = pack2<F16T>(o[0], o[1]);
  pr[1] = pack2<F16T>(o[2], o[3]);
  *reinterpret_cast<u32x2 *>(op) = pr;
}

}  // namespace mce

using namespace mce;

extern "C" int mce_decode_gemm(int dtype, const void *x, const void *w, void *out, int m, int n,
                               int k, int64_t x_stride, int64_t out_stride, int epilogue,
                               void *stream) {
  clear_error();
  MCE_REQUIRE(dtype == MCE_F16 || dtype == MCE_BF16, "mce_decode_gemm: unknown dtype %d", dtype);
  if (dtype != MCE_F16)
    return set_error(MCE_ERR_UNSUPPORTED, "mce_decode_gemm: only fp16 is implemented");
  MCE_REQUIRE(epilogue >= MCE_EPI_STORE && epilogue <= MCE_EPI_SWIGLU,
              "mce_decode_gemm: unknown epilogue %d", epilogue);
  MCE_REQUIRE(m >= 0 && n >= 0 && k >= 0, "mce_decode_gemm: bad shape");
  if (m == 0 || n == 0) return MCE_OK;
  if (m > 16 || n % 16 != 0 || k % DG_SLICE != 0 || k == 0 ||
      k / DG_SLICE * (epilogue == MCE_EPI_SWIGLU ? 2 : 1) > DG_MAX_WAVES)
    return set_error(MCE_ERR_UNSUPPORTED,
                     "mce_decode_gemm: needs m <= 16, n %% 16 == 0, k a multiple of %d with "
                     "k / %d (x2 for SwiGLU) <= %d waves (got m=%d n=%d k=%d)",
                     DG_SLICE, DG_SLICE, DG_MAX_WAVES, m, n, k);
  MCE_REQUIRE(x && w && out, "mce_decode_gemm: null pointer");
  MCE_REQUIRE(x_stride >= k && x_stride % 8 == 0 && out_stride >= n && out_stride % 4 == 0,
              "mce_decode_gemm: bad row strides");
  MCE_REQUIRE(aligned16(x) && aligned16(w) && (reinterpret_cast<uintptr_t>(out) & 7) == 0,
              "mce_decode_gemm: x and w must be 16-byte aligned, out 8-byte aligned");
  MCE_REQUIRE((int64_t)n * k * (epilogue == MCE_EPI_SWIGLU ? 2 : 1) < ((int64_t)1 << 31),
              "mce_decode_gemm: weight too large");
  DecodeGemmArgs a{};
  a.x = (const uint16_t *)x;
  a.w = (const uint16_t *)w;
  a.out = (uint16_t *)out;
  a.M = m;
  a.N = n;
  a.K = k;
  a.x_stride = x_stride;
  a.out_stride = out_stride;
  hipStream_t st = (hipStream_t)stream;
  const int nw = k / DG_SLICE;
  const dim3 grid(n / 16);
  if (epilogue == MCE_EPI_STORE)
    decode_gemm_kernel<0, 1><<<grid, nw * 64, 0, st>>>(a);
  else if (epilogue == MCE_EPI_ADD)
    decode_gemm_kernel<1, 1><<<grid, nw * 64, 0, st>>>(a);
  else
    decode_gemm_kernel<2, 2><<<grid, 2 * nw * 64, 0, st>>>(a);
  return check_launch("mce_decode_gemm");
}
