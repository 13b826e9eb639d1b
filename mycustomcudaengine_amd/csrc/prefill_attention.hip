// Causal flash prefill attention for gfx950 (reference semantics:
// csrc/kernels/prefill_attention.cu:15-269, host wrapper :271-309).
//
// Rows: the G = Hq / Hkv query heads that share a kv head are packed into the
// M dimension.  For batch b and kv head g, row r = position * G + (query head
// - g G), so one workgroup's rows cover consecutive positions of all G heads
// and every K/V tile staged in LDS serves all of them (the reference stages
// K/V once per query head).
//
// Work items: a workgroup takes BM = 32 * NW consecutive rows of one (b, g).
// Causal cost grows with the row index, so workgroups are numbered heaviest
// item first.
//
// Each wave owns 32 rows and uses v_mfma_f32_32x32x16_f16 throughout:
//   S^T[64 keys x 32 rows] = K . Q^T   (A = K from LDS, B = Q^T in registers)
//     -> lane l holds the scores of row (l % 32) for 32 of the 64 keys, so the
//        row softmax is in-lane plus one exchange with lane l ^ 32.
//   O^T[128 dims x 32 rows] += V^T . P^T (A = V^T from LDS, B = P^T straight
//     from the S^T registers, converted to f16): lane l again holds row
//     (l % 32), so the online-softmax rescale is a per-lane multiply.
// The k-index permutation used for P^T (keys 8(v/4) + 4(l/32) + v%4 of the
// S^T output layout) is mirrored by the V^T reads, two 8-byte LDS reads of 4
// consecutive keys each.  V is transposed into LDS ([dim][key]) on the way in;
// K is stored row-major with a 16-byte row pad (conflict-free 16-byte reads).
// The next tile's K/V are loaded into registers while the current tile is
// computed.
//
// Softmax: p = exp2(s c - m c) with c = scale log2(e) as one FMA on the raw
// score; only tiles that reach a wave's diagonal (or the sequence end) are
// masked; the running max is only raised (and O, l rescaled) when a row's
// max grows by more than 2^8 in p units, so most tiles skip the rescale
// (p then stays below 256, well inside fp16).
#include "mce_common.h"

namespace mce {

constexpr int PF_HD = 128;
constexpr int PF_BN = 64;
constexpr int KS_PITCH = PF_HD + 8;  // halfs per K row in LDS (272 B)
constexpr int VT_PITCH = PF_BN + 4;  // halfs per V^T row in LDS (136 B)
constexpr float RESCALE_TAU = 8.0f;  // log2 headroom before raising the max

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

struct PrefillArgs {
  const uint16_t *q, *k, *v;
  uint16_t *out;
  int B, S, Hq, Hkv, G;
  int n_items;
  float scale_log2;
};

template <int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_causal_kernel(PrefillArgs a) {
  constexpr int BM = 32 * NW;
  constexpr int NT = NW * 64;
  constexpr int K_PIECES = PF_BN * PF_HD / 8;      // 16-byte pieces per K tile
  constexpr int V_GROUPS = PF_BN / 4 * PF_HD / 8;  // 4-key x 8-dim groups per V tile
  constexpr int KP = (K_PIECES + NT - 1) / NT;
  constexpr int VG = (V_GROUPS + NT - 1) / NT;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[PF_BN * KS_PITCH];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[PF_HD * VT_PITCH];

  // workgroup -> (item, batch, kv head); kv head fastest so that the
  // workgroups of one kv head share an XCD (and its L2) when Hkv B == 8.
  const int id = blockIdx.x;
  const int g = id % a.Hkv;
  const int b = (id / a.Hkv) % a.B;
  const int item_rank = id / (a.Hkv * a.B);
  const int G = a.G, S = a.S;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hf = lane >> 5, r32 = lane & 31;

  const int64_t q_row_stride = (int64_t)a.Hq * PF_HD;
  const int kv_row = a.Hkv * PF_HD;  // elements between consecutive keys
  const uint16_t *kbase = a.k + ((int64_t)b * S * a.Hkv + g) * PF_HD;
  const uint16_t *vbase = a.v + ((int64_t)b * S * a.Hkv + g) * PF_HD;
  const float c = a.scale_log2;

  // Per-thread staging assignments (fixed for the whole kernel).
  //  K: piece pc -> key pc / 16, 16-byte column pc % 16 (16 lanes per key row).
  //  V: group gc -> keys 4 (gc % 16) .. +3, dims 8 (gc / 16) .. +7, so the 16
  //     lanes of a group write one 128-byte run of a V^T row (no bank
  //     conflicts) after transposing 4 keys x 8 dims in registers.
  //  (NT is a multiple of 16, so piece it of this thread sits NT / 16 keys
  //  below piece it - 1: one base offset plus a uniform step.)
  static_assert(NT % 16 == 0, "staging assumes whole 16-lane groups");
  const int k_off0 = (tid >> 4) * kv_row + (tid & 15) * 8;
  const int k_step = (NT / 16) * kv_row;
  int v_off[VG];
#pragma unroll
  for (int gi = 0; gi < VG; ++gi) {
    const int gc = tid + gi * NT;
    v_off[gi] = 4 * (gc & 15) * kv_row + (gc >> 4) * 8;
  }

  u32x4 kreg[KP], vreg[VG * 4];
  auto load_tile = [&](int n0) {
    const uint16_t *kt = kbase + (int64_t)n0 * kv_row;
    const uint16_t *vt = vbase + (int64_t)n0 * kv_row;
#pragma unroll
    for (int it = 0; it < KP; ++it) {
      const int pc = tid + it * NT;
      const int key = n0 + (pc >> 4);
      kreg[it] = (pc < K_PIECES && key < S)
                     ? *reinterpret_cast<const u32x4 *>(kt + k_off0 + it * k_step)
                     : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int gi = 0; gi < VG; ++gi) {
      const int gc = tid + gi * NT;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int key = n0 + 4 * (gc & 15) + kk;
        vreg[gi * 4 + kk] = (gc < V_GROUPS && key < S)
                                ? *reinterpret_cast<const u32x4 *>(vt + v_off[gi] + kk * kv_row)
                                : u32x4{0, 0, 0, 0};
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int it = 0; it < KP; ++it) {
      const int pc = tid + it * NT;
      if (pc < K_PIECES)
        *reinterpret_cast<u32x4 *>(&Ks[(pc >> 4) * KS_PITCH + (pc & 15) * 8]) = kreg[it];
    }
#pragma unroll
    for (int gi = 0; gi < VG; ++gi) {
      const int gc = tid + gi * NT;
      if (gc < V_GROUPS) {
        const int key0 = 4 * (gc & 15), piece = gc >> 4;
        const u32x4 *x = &vreg[gi * 4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // dims 8 piece + 2e (low halves) and + 2e + 1 (high halves)
          u32x2 lo, hi;
          lo[0] = __builtin_amdgcn_perm(x[1][e], x[0][e], 0x05040100u);
          lo[1] = __builtin_amdgcn_perm(x[3][e], x[2][e], 0x05040100u);
          hi[0] = __builtin_amdgcn_perm(x[1][e], x[0][e], 0x07060302u);
          hi[1] = __builtin_amdgcn_perm(x[3][e], x[2][e], 0x07060302u);
          const int d = piece * 8 + 2 * e;
          *reinterpret_cast<u32x2 *>(&Vt[d * VT_PITCH + key0]) = lo;
          *reinterpret_cast<u32x2 *>(&Vt[(d + 1) * VT_PITCH + key0]) = hi;
        }
      }
    }
  };

  const int rows_total = S * G;
  {
    const int item = a.n_items - 1 - item_rank;  // heaviest items first
    const int r_item = item * BM;
    const int r_wave = r_item + 32 * w;
    const int row = r_wave + r32;                 // this lane's row
    const int pos = row / G, h = g * G + (row - pos * G);
    const bool row_ok = row < rows_total;
    const int wave_min_pos = r_wave / G;
    const int wave_max_pos = min(S - 1, (r_wave + 31) / G);
    const int item_max_pos = min(S - 1, (r_item + BM - 1) / G);
    const int n_ktiles = item_max_pos / PF_BN + 1;
    // tiles [0, n_full) need no mask for this wave: every key <= its first
    // position and < S
    const int n_full = min((wave_min_pos + 1) / PF_BN, S / PF_BN);
    const int lim = min(pos, S - 1) - 4 * hf;  // masked tiles: key offset limit + n0

    // Q^T as MFMA B operand: lane supplies Q[pos, h][16 i + 8 hf + j].
    half8 qreg[8];
    {
      const uint16_t *qp = a.q + ((int64_t)b * S + (row_ok ? pos : 0)) * q_row_stride +
                           (int64_t)(row_ok ? h : 0) * PF_HD + 8 * hf;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        qreg[i] = row_ok ? __builtin_bit_cast(
                               half8, *reinterpret_cast<const u32x4 *>(qp + 16 * i))
                         : half8{0, 0, 0, 0, 0, 0, 0, 0};
    }

    float m_i = -INFINITY, l_i = 0.f;
    floatx16 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;

    // One key tile: scores, (masked) online softmax, P V.
    auto tile = [&](int n0, bool masked) {
      floatx16 st[2];
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
        for (int e = 0; e < 16; ++e) st[kh][e] = 0.f;
        const uint16_t *kp = &Ks[(kh * 32 + r32) * KS_PITCH + 8 * hf];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          half8 ka = __builtin_bit_cast(half8, *reinterpret_cast<const u32x4 *>(kp + 16 * i));
          st[kh] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka, qreg[i], st[kh], 0, 0, 0);
        }
      }
      if (masked) {
        const int l2 = lim - n0;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (kh * 32 + 8 * (e >> 2) + (e & 3) > l2) st[kh][e] = -INFINITY;
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, st[kh][e]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      // raise the running max only when p would exceed 2^TAU
      const bool grow = (mx - m_i) * c > RESCALE_TAU;  // true on the first tile
      if (__ballot(grow)) {
        const float m_new = grow ? mx : m_i;
        const float alpha = fast_exp2((m_i - m_new) * c);
        l_i *= alpha;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;
        m_i = m_new;
      }
      const float neg_mc = m_i == -INFINITY ? 0.f : -m_i * c;
      float psum = 0.f;
      half8 pk[2][2];
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2) {
          const float p0 = fast_exp2(__builtin_fmaf(st[kh][2 * e2], c, neg_mc));
          const float p1 = fast_exp2(__builtin_fmaf(st[kh][2 * e2 + 1], c, neg_mc));
          psum += p0 + p1;
          const h2 pp = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(p0, p1));
          pk[kh][e2 >> 2][2 * (e2 & 3)] = pp[0];
          pk[kh][e2 >> 2][2 * (e2 & 3) + 1] = pp[1];
        }
      l_i += psum;
      // O^T += V^T P^T
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const uint16_t *vp = &Vt[(dt * 32 + r32) * VT_PITCH + 4 * hf];
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) {
            const int kb = kh * 32 + 16 * kk;
            u32x2 x0 = *reinterpret_cast<const u32x2 *>(vp + kb);
            u32x2 x1 = *reinterpret_cast<const u32x2 *>(vp + kb + 8);
            u32x4 xa = {x0[0], x0[1], x1[0], x1[1]};
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                __builtin_bit_cast(half8, xa), pk[kh][kk], o[dt], 0, 0, 0);
          }
      }
    };

    // Barriers match by count, so the two loops may split at a different tile
    // in each wave: every iteration of either loop stages exactly one tile.
    load_tile(0);
    int kt = 0;
    for (; kt < n_full; ++kt) {  // tiles entirely below this wave's rows
      __syncthreads();
      store_tile();
      __syncthreads();
      if (kt + 1 < n_ktiles) load_tile((kt + 1) * PF_BN);
      tile(kt * PF_BN, false);
    }
    for (; kt < n_ktiles; ++kt) {  // diagonal / end-of-sequence tiles
      __syncthreads();
      store_tile();
      __syncthreads();
      if (kt + 1 < n_ktiles) load_tile((kt + 1) * PF_BN);
      if (kt * PF_BN <= wave_max_pos) tile(kt * PF_BN, true);
    }

    // ---- normalise and store: lane holds dims dt*32 + 8(e/4) + 4hf + e%4 ----
    const float l_tot = l_i + __shfl_xor(l_i, 32, 64);
    if (row_ok) {
      const float inv = 1.0f / l_tot;
      uint16_t *op = a.out + ((int64_t)b * S + pos) * q_row_stride + (int64_t)h * PF_HD + 4 * hf;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int e4 = 0; e4 < 4; ++e4) {
          u32x2 pr;
          pr[0] = pack2<F16T>(o[dt][4 * e4] * inv, o[dt][4 * e4 + 1] * inv);
          pr[1] = pack2<F16T>(o[dt][4 * e4 + 2] * inv, o[dt][4 * e4 + 3] * inv);
          *reinterpret_cast<u32x2 *>(op + dt * 32 + 8 * e4) = pr;
        }
    }
  }
}

}  // namespace mce

using namespace mce;

extern "C" int mce_prefill_attention(int dtype, const void *query,
                                     const void *key, const void *value,
                                     void *output, int batch, int seq_len,
                                     int num_heads, int num_kv_heads,
                                     int head_dim, float scale, void *stream) {
  clear_error();
  MCE_REQUIRE(dtype == MCE_F16 || dtype == MCE_BF16,
              "mce_prefill_attention: unknown dtype %d", dtype);
  if (dtype != MCE_F16)
    return set_error(MCE_ERR_UNSUPPORTED,
                     "mce_prefill_attention: only fp16 is implemented");
  MCE_REQUIRE(head_dim == PF_HD,
              "mce_prefill_attention: head_dim must be 128 (got %d)", head_dim);
  MCE_REQUIRE(batch >= 0 && seq_len >= 0 && num_heads >= 1 && num_kv_heads >= 1,
              "mce_prefill_attention: bad shape");
  MCE_REQUIRE(num_heads % num_kv_heads == 0,
              "mce_prefill_attention: num_heads %d not a multiple of num_kv_heads %d",
              num_heads, num_kv_heads);
  if (batch == 0 || seq_len == 0) return MCE_OK;
  MCE_REQUIRE(query && key && value && output, "mce_prefill_attention: null pointer");
  MCE_REQUIRE(aligned16(query) && aligned16(key) && aligned16(value) &&
                  aligned16(output),
              "mce_prefill_attention: tensors must be 16-byte aligned");
  const int G = num_heads / num_kv_heads;
  MCE_REQUIRE((int64_t)seq_len * G < ((int64_t)1 << 30), "mce_prefill_attention: sequence too long");
  // Items of 128 rows, one per workgroup, heaviest first: when there are more
  // items than workgroup slots, the dispatcher hands the lighter ones to the
  // CUs that free up first (longest-processing-time-first scheduling).
  constexpr int nw = 4;
  PrefillArgs a{};
  a.q = (const uint16_t *)query;
  a.k = (const uint16_t *)key;
  a.v = (const uint16_t *)value;
  a.out = (uint16_t *)output;
  a.B = batch;
  a.S = seq_len;
  a.Hq = num_heads;
  a.Hkv = num_kv_heads;
  a.G = G;
  a.n_items = (int)(((int64_t)seq_len * G + 32 * nw - 1) / (32 * nw));
  a.scale_log2 = scale * 1.4426950408889634f;
  const int64_t grid = (int64_t)a.n_items * batch * num_kv_heads;
  MCE_REQUIRE(grid < ((int64_t)1 << 31), "mce_prefill_attention: problem too large");
  hipStream_t st = (hipStream_t)stream;
  prefill_causal_kernel<nw><<<(unsigned)grid, nw * 64, 0, st>>>(a);
  return check_launch("mce_prefill_attention");
}
