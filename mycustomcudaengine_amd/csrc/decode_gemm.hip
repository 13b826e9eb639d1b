// Decode-sized GEMM for gfx950: out[M, N] (op)= xn[M, K] . W[N, K]^T with
// M <= 16 (one token per sequence), fp16 in, fp32 accumulation; xn is x or
// RMSNorm(x) (fused in front), and the epilogue stores, adds into the
// residual stream or applies SwiGLU.  This is the projection work of the
// engine's decode step (engine/models/llama.py:94-174 runs it through
// torch.matmul with separate RMSNorm and SwiGLU kernels); at these shapes it
// is a weight-streaming problem: every W byte is read once and the MFMA work
// is negligible.
//
// Layout of one launch (grid = N / 16 workgroups of 8 waves):
//   * a workgroup owns 16 output columns (16 rows of W; gate rows j and up
//     rows n + j for SwiGLU); wave w takes the K slice [w K / 8, (w + 1) K / 8)
//     as C = K / 256 chunks of 32;
//   * x (normalised when fused) is staged once per workgroup in LDS as the
//     MFMA B operand: 16-byte groups of 8 consecutive k, [k / 8][token slot],
//     the slot XOR-swizzled by the group index so that the staging writes (a
//     wave per token, consecutive groups) and the fragment reads (the tokens
//     of one group) both hit 16 different 16-byte bank groups;
//   * W fragments (A operand: lane l holds row l % 16, k 8 (l / 16) .. +7) go
//     from HBM straight into registers: the x loads are issued first (loads
//     return in order, so staging x waits for x only), then the W fragments
//     -- all of them, or half when registers are short (SwiGLU's two tiles),
//     the rest issued once x is staged.  Register use stays low enough for
//     every workgroup of a launch to be resident, so the whole weight is in
//     flight at once.  Launches of many rounds of workgroups (lm_head) load
//     instead in chunk pairs (64 k), each load instruction reading 8 rows x
//     128 contiguous bytes with 8 consecutive lanes per row, which streams
//     ~13% faster than 16 rows x 64 bytes; each pair then goes through a 2 KB
//     wave-private LDS buffer (XOR-swizzled: conflict-free writes of 8 rows
//     and reads of 16) to become the A fragments.  In a single round of
//     workgroups the LDS step costs more than the grouping saves;
//   * one v_mfma_f32_16x16x32_f16 per chunk and tile (tokens >= M are zeros);
//     the 8 K-slice partials (lane l: rows 4 (l / 16) .. +3, token l % 16)
//     are summed in LDS and wave 0 applies the epilogue:
//       STORE  out[m, n] = acc
//       ADD    out[m, n] = out[m, n] + acc          (residual stream, in place)
//       SWIGLU out[m, j] = silu(acc_gate) * acc_up  (W = [2 n, K], gate rows first)
// The fused RMSNorm computes each token's scale exactly as mce_rmsnorm does
// (same per-lane chunk order, reduction and rounding), so xn is bit-identical
// to that op's output.
#include "mce_common.h"

namespace mce {

constexpr int DG_WAVES = 8;

struct DecodeGemmArgs {
  const uint16_t *x, *w, *norm_w;
  uint16_t *out;
  int M, N;
  int64_t x_stride, out_stride;
  float eps;
};

// 16-byte group index of k group kg, token slot t in the staged x
template <int MP>
__device__ __forceinline__ int xs_group(int kg, int t) {
  if constexpr (MP == 16)
    return kg * 16 + (t ^ (kg & 15));
  else
    return kg * 8 + (t ^ ((kg >> 1) & 7));
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.0f + __expf(-g)) * u;
}

// EPI: 0 store, 1 add, 2 SwiGLU; TT tiles per workgroup (SwiGLU: the gate
// and up tiles); MP token slots (8 or 16); NORM: fuse RMSNorm; C chunks of 32
// k per wave; R output columns per tile (16, 12, 10 or 8: lanes of rows >= R
// re-read row R - 1 and their results are dropped), so that the grid can be
// sized to a whole number of workgroups per CU.
// ROWS128: W loads of 8 rows x 128 bytes, fragments rebuilt through LDS.
template <int EPI, int TT, int MP, bool NORM, int C, int WPE, int R, bool ROWS128>
__global__ __launch_bounds__(DG_WAVES * 64) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void decode_gemm_kernel(DecodeGemmArgs a) {
  static_assert(R % 2 == 0 && R >= 8 && R <= 16, "tile rows");
  constexpr int K = C * 256;
  constexpr int VPT = K / 512;      // 16-byte groups of one token row per lane
  constexpr int NTOK = MP / 8;      // token rows staged per wave
  // W chunks fetched before x is staged: all of them when the registers of
  // the W fragments, the x rows and the norm weights fit the occupancy
  // target together, else half (the rest once x is in LDS)
  constexpr int REGS = 4 * (TT * C + NTOK * VPT + (NORM ? VPT : 0)) + 24;
  constexpr int C1 = REGS <= 512 / WPE ? C : (C + 1) / 2;
  __shared__ __attribute__((aligned(16))) uint16_t xs[K / 8 * MP * 8];
  // ROWS128, per wave: 16 rows x 64 k of W (a chunk pair), row pitch 128
  // bytes, the 16-byte k group g of row p stored at group g ^ ((p >> 1) & 7)
  __shared__ __attribute__((aligned(16))) uint32_t wx[ROWS128 ? DG_WAVES : 1][16 * 32];
  static_assert(K / 8 * MP * 8 * 2 >= DG_WAVES * TT * 4 * 64 * 4, "reduction fits");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // first output column of the workgroup (SwiGLU: of its gate / up tile pair)
  const int col0 = blockIdx.x * (EPI == 2 ? R : R * TT);
  const int r = lane & 15, q = lane >> 4;

  // 1. this wave's token rows of x (and the norm weights)
  u32x4 xv[NTOK][VPT];
  u32x4 nw[NORM ? VPT : 1];
#pragma unroll
  for (int j = 0; j < NTOK; ++j) {
    const int m = wave + 8 * j;
    if (m < a.M) {
      const uint16_t *xr = a.x + (int64_t)m * a.x_stride;
#pragma unroll
      for (int i = 0; i < VPT; ++i)
        xv[j][i] = *reinterpret_cast<const u32x4 *>(xr + (lane + 64 * i) * 8);
    }
  }
  if constexpr (NORM) {
#pragma unroll
    for (int i = 0; i < VPT; ++i)
      nw[i] = *reinterpret_cast<const u32x4 *>(a.norm_w + (lane + 64 * i) * 8);
  }

  // 2. first half of the W loads.  ROWS128: load c of a tile reads rows
  // 8 (c & 1) .. +7 of its 16, lane l taking row 8 (c & 1) + l / 8 at k group
  // l % 8 of chunk pair c / 2; otherwise load c is chunk c's fragment.
  static_assert(!ROWS128 || (C % 2 == 0 && C1 % 2 == 0), "chunk pairs");
  const uint16_t *wp[TT][2];
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = ROWS128 ? (lane >> 3) + 8 * h : r;
      wp[t][h] = a.w + (int64_t)(col0 + t * (EPI == 2 ? a.N : R) + (row < R ? row : R - 1)) * K +
                 wave * (K / 8) + 8 * (ROWS128 ? lane & 7 : q);
    }
  auto w_addr = [&](int t, int c) {
    return ROWS128 ? wp[t][c & 1] + 64 * (c >> 1) : wp[t][0] + 32 * c;
  };
  u32x4 wf[TT][C];
#pragma unroll
  for (int c = 0; c < C1; ++c)
#pragma unroll
    for (int t = 0; t < TT; ++t) wf[t][c] = *reinterpret_cast<const u32x4 *>(w_addr(t, c));
  // keep these loads ahead of the staging below (the scheduler would
  // otherwise sink most of them past it to save registers)
  __builtin_amdgcn_sched_barrier(0);

  // 3. stage x (normalised) into LDS; slots of tokens >= M hold zeros
#pragma unroll
  for (int j = 0; j < NTOK; ++j) {
    const int m = wave + 8 * j;
    if (m < a.M) {
      float inv = 1.0f;
      if constexpr (NORM) {
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < VPT; ++i) ss = sumsq8<F16T>(xv[j][i], ss);
        inv = rms_inv(wave_sum(ss), K, a.eps);
      }
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        const u32x4 val = NORM ? rms_scale8<F16T>(xv[j][i], nw[NORM ? i : 0], inv) : xv[j][i];
        *reinterpret_cast<u32x4 *>(&xs[xs_group<MP>(lane + 64 * i, m) * 8]) = val;
      }
    } else {
#pragma unroll
      for (int i = 0; i < VPT; ++i)
        *reinterpret_cast<u32x4 *>(&xs[xs_group<MP>(lane + 64 * i, m) * 8]) = u32x4{0, 0, 0, 0};
    }
  }

  // 4. second half of the W fragments, then the MFMAs
#pragma unroll
  for (int c = C1; c < C; ++c)
#pragma unroll
    for (int t = 0; t < TT; ++t) wf[t][c] = *reinterpret_cast<const u32x4 *>(w_addr(t, c));
  lds_barrier();
  floatx4 acc[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
  uint32_t *const wxw = wx[ROWS128 ? wave : 0];
  // this lane's write slot (row l / 8 + 8 h, k group l % 8) and read slot
  // (row l % 16, k group 4 hh + l / 16) in the swizzled pair buffer
  auto wslot = [&](int h) {
    const int p = (lane >> 3) + 8 * h;
    return p * 32 + 4 * ((lane & 7) ^ ((p >> 1) & 7));
  };
  auto rslot = [&](int hh) { return r * 32 + 4 * ((4 * hh + q) ^ ((r >> 1) & 7)); };
#pragma unroll
  for (int c = 0; c < C; c += 2) {
    u32x4 xf[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const int kg = (wave * C + c + hh) * 4 + q;
      xf[hh] = *reinterpret_cast<const u32x4 *>(&xs[xs_group<MP>(kg, r & (MP - 1)) * 8]);
      if constexpr (MP == 8) xf[hh] = r < 8 ? xf[hh] : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
      if constexpr (!ROWS128) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, wf[t][c + hh]),
                                                          __builtin_bit_cast(half8, xf[hh]), acc[t],
                                                          0, 0, 0);
        continue;
      }
      // the wave's own LDS operations complete in order: only the compiler
      // has to keep the writes before the reads (and the next pair's writes
      // after them)
      *reinterpret_cast<u32x4 *>(wxw + wslot(0)) = wf[t][c];
      *reinterpret_cast<u32x4 *>(wxw + wslot(1)) = wf[t][c + 1];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
      u32x4 f[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) f[hh] = *reinterpret_cast<const u32x4 *>(wxw + rslot(hh));
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, f[hh]),
                                                        __builtin_bit_cast(half8, xf[hh]), acc[t],
                                                        0, 0, 0);
    }
  }

  // 5. sum the K slices: red[wave][tile][component][lane]
  lds_barrier();  // every wave is done reading xs
  float *const red = reinterpret_cast<float *>(xs);
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((wave * TT + t) * 4 + i) * 64 + lane] = acc[t][i];
  lds_barrier();
  if (wave != 0 || r >= a.M) return;
  float v[TT][4];
#pragma unroll
  for (int t = 0; t < TT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float s = 0.f;
#pragma unroll
      for (int sl = 0; sl < DG_WAVES; ++sl) s += red[((sl * TT + t) * 4 + i) * 64 + lane];
      v[t][i] = s;
    }
  // lane holds rows 4 q .. +3 of each tile for token r: output columns
  // col0 (+ t R) + 4 q .. +3, written as column pairs (rows < R only)
  if (4 * q >= R) return;
  constexpr int NOUT = EPI == 2 ? 1 : TT;
#pragma unroll
  for (int t = 0; t < NOUT; ++t) {
    uint32_t *op = reinterpret_cast<uint32_t *>(a.out + (int64_t)r * a.out_stride + col0 + t * R +
                                                4 * q);
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = EPI == 2 ? silu_mul(v[0][i], v[TT - 1][i]) : v[t][i];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (4 * q + 2 * h >= R) break;
      float lo = o[2 * h], hi = o[2 * h + 1];
      if constexpr (EPI == 1) {
        const uint32_t old = op[h];
        lo += F16T::lo(old);
        hi += F16T::hi(old);
      }
      op[h] = pack2<F16T>(lo, hi);
    }
  }
}

template <int EPI, int TT, int MP, bool NORM, int C, int R>
void launch_dg(const DecodeGemmArgs &a, hipStream_t st) {
  // registers of the W fragments decide how many waves fit per SIMD; every
  // workgroup of a launch should be resident at once
  constexpr int WPE = TT * C <= 24 && MP == 8 ? 4 : 2;
  const int grid = a.N / (EPI == 2 ? R : R * TT);
  // many rounds of workgroups (lm_head: 8016 over 256 CUs): 128-byte row loads
  if constexpr (EPI == 0 && TT == 1 && R == 16) {
    if (grid >= 8 * cu_count()) {
      decode_gemm_kernel<EPI, TT, MP, NORM, C, WPE, R, true><<<grid, DG_WAVES * 64, 0, st>>>(a);
      return;
    }
  }
  decode_gemm_kernel<EPI, TT, MP, NORM, C, WPE, R, false><<<grid, DG_WAVES * 64, 0, st>>>(a);
}

template <int EPI, int TT, int MP, bool NORM, int R>
int dispatch_k(const DecodeGemmArgs &a, int k, hipStream_t st) {
  switch (k) {
    case 2048: launch_dg<EPI, TT, MP, NORM, 8, R>(a, st); return MCE_OK;
    case 3072: launch_dg<EPI, TT, MP, NORM, 12, R>(a, st); return MCE_OK;
    case 4096: launch_dg<EPI, TT, MP, NORM, 16, R>(a, st); return MCE_OK;
    case 8192:
      if constexpr (TT == 1 && !NORM && MP == 8) {  // 128 KB of staged x
        launch_dg<EPI, TT, MP, NORM, 32, R>(a, st);
        return MCE_OK;
      }
      break;
  }
  return MCE_ERR_UNSUPPORTED;
}

// Output columns per workgroup: R columns per tile times TT tiles (SwiGLU: R
// gate / up column pairs).  The widest tile is kept unless a narrower one
// cuts the columns of the busiest CU (whole rounds of workgroups over the
// CUs times the columns per workgroup) by more than 10%: 3072 columns run as
// 256 workgroups of 12, 5120 as 256 of 2 x 10, instead of 192 / 320 of 16.
struct DgTile {
  int r, tt;
};

DgTile pick_tile(int n, bool swiglu, int k) {
  static const DgTile plain[] = {{16, 1}, {12, 1}, {10, 2}, {8, 1}};
  static const DgTile glu[] = {{16, 2}, {8, 2}};
  const int64_t cus = cu_count();
  DgTile best = swiglu ? glu[0] : plain[0];
  int64_t best_cost = -1;
  const DgTile *cand = swiglu ? glu : plain;
  const int n_cand = swiglu ? 2 : 4;
  for (int i = 0; i < n_cand; ++i) {
    const DgTile &t = cand[i];
    if (t.tt == 2 && !swiglu && k == 8192) continue;  // one tile only at k = 8192
    const int cols = swiglu ? t.r : t.r * t.tt;
    if (n % cols != 0) continue;
    const int64_t cost = ((n / cols) + cus - 1) / cus * cols;
    if (best_cost < 0 || 10 * cost < 9 * best_cost) {
      best = t;
      best_cost = cost;
    }
  }
  return best;
}

template <int EPI, int MP, bool NORM>
int dispatch_tile(const DecodeGemmArgs &a, int k, const DgTile &t, hipStream_t st) {
  if constexpr (EPI == 2) {
    return t.r == 8 ? dispatch_k<EPI, 2, MP, NORM, 8>(a, k, st) : dispatch_k<EPI, 2, MP, NORM, 16>(a, k, st);
  } else {
    switch (t.r) {
      case 12: return dispatch_k<EPI, 1, MP, NORM, 12>(a, k, st);
      case 10: return dispatch_k<EPI, 2, MP, NORM, 10>(a, k, st);
      case 8: return dispatch_k<EPI, 1, MP, NORM, 8>(a, k, st);
      default: return dispatch_k<EPI, 1, MP, NORM, 16>(a, k, st);
    }
  }
}

template <bool NORM>
int dispatch(const DecodeGemmArgs &a, int k, int epilogue, hipStream_t st) {
  const bool small = a.M <= 8;
  const DgTile t = pick_tile(a.N, epilogue == MCE_EPI_SWIGLU, k);
  if (epilogue == MCE_EPI_STORE)
    return small ? dispatch_tile<0, 8, NORM>(a, k, t, st) : dispatch_tile<0, 16, NORM>(a, k, t, st);
  if (epilogue == MCE_EPI_ADD)
    return small ? dispatch_tile<1, 8, NORM>(a, k, t, st) : dispatch_tile<1, 16, NORM>(a, k, t, st);
  return small ? dispatch_tile<2, 8, NORM>(a, k, t, st) : dispatch_tile<2, 16, NORM>(a, k, t, st);
}

int decode_gemm_impl(const char *name, int dtype, const void *x, const void *norm_w, float eps,
                     const void *w, void *out, int m, int n, int k, int64_t x_stride,
                     int64_t out_stride, int epilogue, void *stream) {
  clear_error();
  MCE_REQUIRE(dtype == MCE_F16 || dtype == MCE_BF16, "%s: unknown dtype %d", name, dtype);
  if (dtype != MCE_F16) return set_error(MCE_ERR_UNSUPPORTED, "%s: only fp16 is implemented", name);
  MCE_REQUIRE(epilogue >= MCE_EPI_STORE && epilogue <= MCE_EPI_SWIGLU, "%s: unknown epilogue %d",
              name, epilogue);
  MCE_REQUIRE(m >= 0 && n >= 0 && k >= 0, "%s: bad shape", name);
  if (m == 0 || n == 0) return MCE_OK;
  const bool norm = norm_w != nullptr;
  const bool k_ok = k == 2048 || k == 3072 || k == 4096 ||
                    (k == 8192 && !norm && epilogue != MCE_EPI_SWIGLU && m <= 8);
  if (m > 16 || n % 16 != 0 || !k_ok)
    return set_error(MCE_ERR_UNSUPPORTED,
                     "%s: needs m <= 16, n %% 16 == 0 and k in {2048, 3072, 4096} (8192 for m <= 8 "
                     "without the fused RMSNorm or SwiGLU) (got m=%d n=%d k=%d)",
                     name, m, n, k);
  MCE_REQUIRE(x && w && out, "%s: null pointer", name);
  MCE_REQUIRE(x_stride >= k && x_stride % 8 == 0 && out_stride >= n && out_stride % 4 == 0,
              "%s: bad row strides", name);
  MCE_REQUIRE(aligned16(x) && aligned16(w) && (!norm || aligned16(norm_w)) &&
                  (reinterpret_cast<uintptr_t>(out) & 7) == 0,
              "%s: x, w and the norm weight must be 16-byte aligned, out 8-byte aligned", name);
  {
    // every workgroup reads all of x while others already write their
    // columns of out: the two must not overlap
    const uintptr_t x0 = reinterpret_cast<uintptr_t>(x), o0 = reinterpret_cast<uintptr_t>(out);
    const uintptr_t x1 = x0 + (uintptr_t)(((int64_t)(m - 1) * x_stride + k) * 2);
    const uintptr_t o1 = o0 + (uintptr_t)(((int64_t)(m - 1) * out_stride + n) * 2);
    MCE_REQUIRE(x1 <= o0 || o1 <= x0, "%s: out must not overlap x", name);
  }
  MCE_REQUIRE((int64_t)n * k * (epilogue == MCE_EPI_SWIGLU ? 2 : 1) < ((int64_t)1 << 31),
              "%s: weight too large", name);
  DecodeGemmArgs a{};
  a.x = (const uint16_t *)x;
  a.w = (const uint16_t *)w;
  a.norm_w = (const uint16_t *)norm_w;
  a.out = (uint16_t *)out;
  a.M = m;
  a.N = n;
  a.x_stride = x_stride;
  a.out_stride = out_stride;
  a.eps = eps;
  hipStream_t st = (hipStream_t)stream;
  const int rc = norm ? dispatch<true>(a, k, epilogue, st) : dispatch<false>(a, k, epilogue, st);
  if (rc != MCE_OK) return set_error(rc, "%s: no kernel for k=%d", name, k);
  return check_launch(name);
}

}  // namespace mce

using namespace mce;

extern "C" int mce_decode_gemm(int dtype, const void *x, const void *w, void *out, int m, int n,
                               int k, int64_t x_stride, int64_t out_stride, int epilogue,
                               void *stream) {
  return decode_gemm_impl("mce_decode_gemm", dtype, x, nullptr, 0.f, w, out, m, n, k, x_stride,
                          out_stride, epilogue, stream);
}

extern "C" int mce_rmsnorm_decode_gemm(int dtype, const void *x, const void *norm_weight,
                                       float eps, const void *w, void *out, int m, int n, int k,
                                       int64_t x_stride, int64_t out_stride, int epilogue,
                                       void *stream) {
  clear_error();
  MCE_REQUIRE(norm_weight != nullptr, "mce_rmsnorm_decode_gemm: null norm weight");
  MCE_REQUIRE(eps >= 0.f, "mce_rmsnorm_decode_gemm: eps must be >= 0");
  return decode_gemm_impl("mce_rmsnorm_decode_gemm", dtype, x, norm_weight, eps, w, out, m, n, k,
                          x_stride, out_stride, epilogue, stream);
}
