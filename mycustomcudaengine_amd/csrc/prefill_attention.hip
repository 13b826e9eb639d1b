// Causal flash prefill attention for gfx950 (reference semantics:
// csrc/kernels/prefill_attention.cu:15-269, host wrapper :271-309).
//
// One workgroup = BM = 32 * NW query rows of one (batch, head); it walks the
// causal key range in BN = 64-key tiles staged through LDS.
//
// Each wave owns 32 query rows and uses v_mfma_f32_32x32x16_f16 throughout:
//   S^T[64 keys x 32 rows] = K . Q^T   (A = K from LDS, B = Q^T in registers)
//     -> lane l holds the scores of query row (l % 32) for 32 of the 64 keys,
//        so the row softmax is in-lane plus one exchange with lane l ^ 32.
//   O^T[128 dims x 32 rows] += V^T . P^T (A = V^T from LDS, B = P^T straight
//     from the S^T registers, converted to f16): lane l again holds row
//     (l % 32), so the online-softmax rescale is a per-lane multiply.
// The k-index permutation used for P^T (keys 8(v/4) + 4(l/32) + v%4 of the
// S^T output layout) is mirrored by the V^T reads, two 8-byte LDS reads of 4
// consecutive keys each.  V is transposed into LDS ([dim][key]) on the way in;
// K is stored row-major with a 16-byte row pad (conflict-free 16-byte reads).
// The next tile's K/V are loaded into registers while the current tile is
// computed.  Workgroups are numbered heaviest (last query tile) first.
#include "mce_common.h"

namespace mce {

constexpr int PF_HD = 128;
constexpr int PF_BN = 64;
constexpr int KS_PITCH = PF_HD + 8;  // halfs per K row in LDS (272 B)
constexpr int VT_PITCH = PF_BN + 4;  // halfs per V^T row in LDS (136 B)

template <int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2))) void prefill_causal_kernel(
    const uint16_t *__restrict__ q, const uint16_t *__restrict__ k,
    const uint16_t *__restrict__ v, uint16_t *__restrict__ out, int B, int S,
    int Hq, int Hkv, float scale_log2, int n_qtiles) {
  constexpr int BM = 32 * NW;
  constexpr int NT = NW * 64;
  constexpr int KV_PIECES = PF_BN * PF_HD / 8 / NT;  // 16-byte pieces / thread
  __shared__ __attribute__((aligned(16))) uint16_t Ks[PF_BN * KS_PITCH];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[PF_HD * VT_PITCH];

  const int per_tile = B * Hq;
  const int qt = n_qtiles - 1 - (int)(blockIdx.x / per_tile);
  const int rem = blockIdx.x % per_tile;
  const int h = rem % Hq, b = rem / Hq;
  const int g = h / (Hq / Hkv);
  const int m0 = qt * BM;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hf = lane >> 5, r32 = lane & 31;
  const int row = m0 + 32 * w + r32;  // this lane's query row
  const int wave_row_max = m0 + 32 * w + 31;

  const int64_t q_row_stride = (int64_t)Hq * PF_HD;
  const int64_t kv_row_stride = (int64_t)Hkv * PF_HD;
  const uint16_t *kbase = k + ((int64_t)b * S * Hkv + g) * PF_HD;
  const uint16_t *vbase = v + ((int64_t)b * S * Hkv + g) * PF_HD;

  // Q^T as MFMA B operand: lane supplies Q[row][16 i + 8 hf + j].
  half8 qreg[8];
  {
    const bool ok = row < S;
    const uint16_t *qp = q + ((int64_t)b * S + (ok ? row : 0)) * q_row_stride +
                         (int64_t)h * PF_HD + 8 * hf;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      qreg[i] = ok ? __builtin_bit_cast(
                         half8, *reinterpret_cast<const u32x4 *>(qp + 16 * i))
                   : half8{0, 0, 0, 0, 0, 0, 0, 0};
  }

  const int last_key = min(S - 1, m0 + BM - 1);
  const int n_ktiles = last_key / PF_BN + 1;

  // Global -> register staging.  K: thread takes key (tid/16 + 16 it), piece
  // tid%16.  V: thread takes keys 4 (tid/16) .. +3 (+64/NT*... for NW<4),
  // dims 8 (tid%16) .. +7, so it can write 4-key runs of V^T.
  u32x4 kreg[KV_PIECES], vreg[KV_PIECES];
  const int piece = tid & 15;
  auto load_tile = [&](int n0) {
#pragma unroll
    for (int it = 0; it < KV_PIECES; ++it) {
      const int key = n0 + (tid >> 4) + it * (NT / 16);
      kreg[it] = key < S ? *reinterpret_cast<const u32x4 *>(
                               kbase + (int64_t)key * kv_row_stride + piece * 8)
                         : u32x4{0, 0, 0, 0};
    }
    constexpr int VGROUPS = KV_PIECES / 4;  // 4-key groups per thread
#pragma unroll
    for (int gi = 0; gi < VGROUPS; ++gi)
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int key = n0 + 4 * ((tid >> 4) + gi * (NT / 16)) + kk;
        vreg[gi * 4 + kk] =
            key < S ? *reinterpret_cast<const u32x4 *>(
                          vbase + (int64_t)key * kv_row_stride + piece * 8)
                    : u32x4{0, 0, 0, 0};
      }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int it = 0; it < KV_PIECES; ++it) {
      const int key = (tid >> 4) + it * (NT / 16);
      *reinterpret_cast<u32x4 *>(&Ks[key * KS_PITCH + piece * 8]) = kreg[it];
    }
    constexpr int VGROUPS = KV_PIECES / 4;
#pragma unroll
    for (int gi = 0; gi < VGROUPS; ++gi) {
      const int key0 = 4 * ((tid >> 4) + gi * (NT / 16));
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
  };

  float m_i = -INFINITY, l_i = 0.f;
  floatx16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;

  load_tile(0);
  for (int kt = 0; kt < n_ktiles; ++kt) {
    const int n0 = kt * PF_BN;
    __syncthreads();
    store_tile();
    __syncthreads();
    if (kt + 1 < n_ktiles) load_tile(n0 + PF_BN);
    if (n0 > wave_row_max) continue;  // every key of this tile is masked

    // ---- S^T = K Q^T ----
    floatx16 st[2];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
      for (int e = 0; e < 16; ++e) st[kh][e] = 0.f;
      const uint16_t *kp = &Ks[(kh * 32 + r32) * KS_PITCH + 8 * hf];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        half8 a = __builtin_bit_cast(half8,
                                     *reinterpret_cast<const u32x4 *>(kp + 16 * i));
        st[kh] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qreg[i], st[kh], 0, 0, 0);
      }
    }
    // ---- mask + online softmax (base 2) ----
    float mx = -INFINITY;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int key = n0 + kh * 32 + 8 * (e >> 2) + 4 * hf + (e & 3);
        const float sv = st[kh][e] * scale_log2;
        st[kh][e] = (key <= row && key < S) ? sv : -INFINITY;
        mx = fmaxf(mx, st[kh][e]);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_i, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m_i - m_use);
    float psum = 0.f;
    half8 pk[2][2];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const float p = fast_exp2(st[kh][e] - m_use);
        psum += p;
        pk[kh][e >> 3][e & 7] = (_Float16)p;
      }
    l_i = l_i * alpha + psum;
    m_i = m_new;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;

    // ---- O^T += V^T P^T ----
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
  }

  // ---- normalise and store: lane holds dims dt*32 + 8(e/4) + 4hf + e%4 ----
  const float l_tot = l_i + __shfl_xor(l_i, 32, 64);
  if (row < S) {
    const float inv = 1.0f / l_tot;
    uint16_t *op = out + ((int64_t)b * S + row) * q_row_stride +
                   (int64_t)h * PF_HD + 4 * hf;
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
  constexpr int NW = 4;
  const int BM = 32 * NW;
  const int n_qtiles = (seq_len + BM - 1) / BM;
  const int64_t grid = (int64_t)n_qtiles * batch * num_heads;
  MCE_REQUIRE(grid < ((int64_t)1 << 31), "mce_prefill_attention: problem too large");
  const float scale_log2 = scale * 1.4426950408889634f;
  prefill_causal_kernel<NW><<<(unsigned)grid, NW * 64, 0, (hipStream_t)stream>>>(
      (const uint16_t *)query, (const uint16_t *)key, (const uint16_t *)value,
      (uint16_t *)output, batch, seq_len, num_heads, num_kv_heads, scale_log2,
      n_qtiles);
  return check_launch("mce_prefill_attention");
}
