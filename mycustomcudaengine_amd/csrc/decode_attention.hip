// Paged decode attention for gfx950 (reference semantics:
// csrc/kernels/flash_attn_paged.cu:25-142, host wrapper :144-168).
//
// Work decomposition (split-K / flash-decoding):
//   one workgroup = (kv head g, chunk c of CHUNK tokens, sequence b).
//   All G = num_heads / num_kv_heads query heads of kv head g are handled by
//   the same workgroup, so every K/V byte is read from HBM exactly once (the
//   reference launches one warp per query head and reads each KV row G times).
//   Chunks of one sequence run in parallel; each writes its partial softmax
//   state (max m, sum l, unnormalised acc[128]) to the workspace, and a small
//   merge kernel combines them by log-sum-exp.  A sequence that fits in one
//   chunk is normalised and written directly.
//
// Inside a workgroup NW waves take 32-token tiles round-robin.  Per tile:
//   * K^T tile -> MFMA B operand straight from global memory: lane l loads
//     token (l % 16) of each 16-token half, 4 x 16 bytes, so one instruction
//     covers 64 contiguous bytes of 16 token rows.
//     S = Q K^T with v_mfma_f32_16x16x32_f16, A = Q (rows = query heads,
//     zero-padded to 16).  S row h lands in lane group h / 4, register h % 4.
//   * online softmax in base 2 (scale * log2 e folded in), per wave.
//   * p goes through a 2 KB LDS slice; V rows are read as 16-byte pieces
//     (16 lanes cover one 256-byte token row, 4 rows per instruction) and
//     accumulated on the VALU in fp32.
// At the end the NW waves' states are merged in LDS.
#include "mce_common.h"

namespace mce {

constexpr int HD = 128;        // head_dim
constexpr int TILE = 32;       // tokens per wave iteration
constexpr int DEC_NW = 4;      // waves per workgroup

template <int G>
struct DecodeCfg {
  static constexpr int NG4 = (G + 3) / 4;  // lane groups holding S rows
};

template <int G, int CHUNK>
__global__ __launch_bounds__(DEC_NW * 64) void paged_decode_kernel(
    const uint16_t *__restrict__ query, const uint16_t *__restrict__ kcache,
    const uint16_t *__restrict__ vcache, const int32_t *__restrict__ btab,
    const int32_t *__restrict__ ctx_lens, uint16_t *__restrict__ out,
    float *__restrict__ ws_acc, float *__restrict__ ws_ml, int Hq, int Hkv,
    int maxb, int bs_log2, int64_t num_blocks, float scale_log2,
    int max_chunks) {
  constexpr int NG4 = DecodeCfg<G>::NG4;
  const int g = blockIdx.x, c = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int bs = 1 << bs_log2;

  int ctx = ctx_lens[b];
  const int cap = maxb << bs_log2;
  ctx = ctx > cap ? cap : ctx;
  const int head0 = g * G;

  if (ctx <= 0) {  // defined output for empty sequences: zeros
    if (c == 0)
      for (int i = tid; i < G * HD; i += DEC_NW * 64)
        out[((int64_t)b * Hq + head0) * HD + i] = 0;
    return;
  }
  const int t_begin = c * CHUNK;
  if (t_begin >= ctx) return;
  const int t_end = min(t_begin + CHUNK, ctx);
  const int nchunks = (ctx + CHUNK - 1) / CHUNK;

  __shared__ floatx4 p_lds[DEC_NW][TILE][NG4];
  __shared__ float red_acc[DEC_NW][G][HD];
  __shared__ float red_m[DEC_NW][G], red_l[DEC_NW][G];

  // Q as MFMA A operand: row = query head lr, k-piece (4i + lg) = dims
  // [8(4i+lg), 8(4i+lg)+8).  The same piece mapping is used for K below.
  half8 qa[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (lr < G) {
      const uint16_t *qp =
          query + ((int64_t)b * Hq + head0 + lr) * HD + (4 * i + lg) * 8;
      qa[i] = __builtin_bit_cast(half8, *reinterpret_cast<const u32x4 *>(qp));
    } else {
      qa[i] = half8{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }

  float m_run[G], l_part[4], acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m_run[h] = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) l_part[j] = 0.f;

  const int32_t *bt = btab + (int64_t)b * maxb;
  const int64_t head_stride = HD;              // elements between heads
  const int64_t slot_stride = (int64_t)Hkv * HD;  // elements between slots
  const int64_t nb_max = num_blocks - 1;

  auto slot_base = [&](int t) -> int64_t {  // element offset of token t, head g
    int64_t phys = bt[t >> bs_log2];
    phys = phys < 0 ? 0 : (phys > nb_max ? nb_max : phys);
    return ((phys << bs_log2) + (t & (bs - 1))) * slot_stride + g * head_stride;
  };

  for (int tile_t0 = t_begin + w * TILE; tile_t0 < t_end;
       tile_t0 += DEC_NW * TILE) {
    // ---- issue K loads (MFMA B operand layout) ----
    half8 kb[2][4];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      int t = tile_t0 + 16 * u + lr;
      t = t < ctx ? t : ctx - 1;
      const uint16_t *kp = kcache + slot_base(t) + lg * 8;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        kb[u][i] = __builtin_bit_cast(
            half8, *reinterpret_cast<const u32x4 *>(kp + i * 32));
    }
    // ---- issue V loads: lane group lg owns tokens tile_t0 + 8 lg + s ----
    u32x4 vv[8];
    const int tv = tile_t0 + 8 * lg;
    if (tv < ctx) {
      const uint16_t *vp = vcache + slot_base(tv) + lr * 8;
#pragma unroll
      for (int s = 0; s < 8; ++s)
        vv[s] = *reinterpret_cast<const u32x4 *>(vp + s * slot_stride);
#pragma unroll
      for (int s = 0; s < 8; ++s)
        if (tv + s >= ctx) vv[s] = u32x4{0, 0, 0, 0};
    } else {
#pragma unroll
      for (int s = 0; s < 8; ++s) vv[s] = u32x4{0, 0, 0, 0};
    }

    // ---- S = Q K^T on MFMA ----
    floatx4 sacc[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      sacc[u] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sacc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[i], kb[u][i],
                                                         sacc[u], 0, 0, 0);
    }

    // ---- online softmax (base 2) ----
    float s[2][4];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const bool valid = tile_t0 + 16 * u + lr < ctx;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        s[u][j] = valid ? sacc[u][j] * scale_log2 : -INFINITY;
    }
    float mx[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) mx[j] = row16_max(fmaxf(s[0][j], s[1][j]));

    float alpha[G], m_lane[4];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float tmax = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mx[h & 3]),
                                           16 * (h >> 2)));
      const float mn = fmaxf(m_run[h], tmax);
      alpha[h] = fast_exp2(m_run[h] - mn);
      m_run[h] = mn;
    }
    // m of the head held in register j of this lane (head 4 lg + j).
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float mj = 0.f;
#pragma unroll
      for (int h = 0; h < G; ++h)
        if ((h & 3) == j) mj = (lg == (h >> 2)) ? m_run[h] : mj;
      m_lane[j] = mj;
    }
    float p[2][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      p[0][j] = fast_exp2(s[0][j] - m_lane[j]);
      p[1][j] = fast_exp2(s[1][j] - m_lane[j]);
      float a = 1.f;
#pragma unroll
      for (int h = 0; h < G; ++h)
        if ((h & 3) == j) a = (lg == (h >> 2)) ? alpha[h] : a;
      l_part[j] = l_part[j] * a + p[0][j] + p[1][j];
    }
    if (lg < NG4) {
      p_lds[w][lr][lg] = floatx4{p[0][0], p[0][1], p[0][2], p[0][3]};
      p_lds[w][16 + lr][lg] = floatx4{p[1][0], p[1][1], p[1][2], p[1][3]};
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- acc = acc * alpha + P V ----
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] *= alpha[h];
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) {
      floatx4 pv[NG4];
#pragma unroll
      for (int q4 = 0; q4 < NG4; ++q4) pv[q4] = p_lds[w][8 * lg + s8][q4];
      float vf[8];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        vf[2 * k] = F16T::lo(vv[s8][k]);
        vf[2 * k + 1] = F16T::hi(vv[s8][k]);
      }
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float ph = pv[h >> 2][h & 3];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] += ph * vf[e];
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- per-wave reduction ----
  float l_tot[G];
#pragma unroll
  for (int j = 0; j < 4; ++j) l_part[j] = row16_sum(l_part[j]);
#pragma unroll
  for (int h = 0; h < G; ++h)
    l_tot[h] = __builtin_bit_cast(
        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, l_part[h & 3]),
                                         16 * (h >> 2)));
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = acc[h][e];
      v += __shfl_xor(v, 16, 64);
      v += __shfl_xor(v, 32, 64);
      acc[h][e] = v;
    }
  if (lg == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      *reinterpret_cast<floatx4 *>(&red_acc[w][h][lr * 8]) =
          floatx4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
      *reinterpret_cast<floatx4 *>(&red_acc[w][h][lr * 8 + 4]) =
          floatx4{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      red_m[w][h] = m_run[h];
      red_l[w][h] = l_tot[h];
    }
  }
  __syncthreads();

  // ---- cross-wave merge; write final row or split-K partial ----
  for (int idx = tid; idx < G * HD; idx += DEC_NW * 64) {
    const int h = idx / HD, d = idx - h * HD;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < DEC_NW; ++ww) M = fmaxf(M, red_m[ww][h]);
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int ww = 0; ww < DEC_NW; ++ww) {
      const float sc = fast_exp2(red_m[ww][h] - M);
      L += red_l[ww][h] * sc;
      A += red_acc[ww][h][d] * sc;
    }
    const int64_t row = (int64_t)b * Hq + head0 + h;
    if (nchunks == 1) {
      out[row * HD + d] = F16T::from_float(A / L);
    } else {
      const int64_t pr = row * max_chunks + c;
      ws_acc[pr * HD + d] = A;
      if (d == 0) {
        ws_ml[pr * 2] = M;
        ws_ml[pr * 2 + 1] = L;
      }
    }
  }
}

// Log-sum-exp merge of split-K partials: one 128-lane workgroup per
// (query head, sequence).
template <int CHUNK>
__global__ __launch_bounds__(HD) void paged_decode_merge_kernel(
    const float *__restrict__ ws_acc, const float *__restrict__ ws_ml,
    const int32_t *__restrict__ ctx_lens, uint16_t *__restrict__ out, int Hq,
    int maxb, int bs_log2, int max_chunks) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  int ctx = ctx_lens[b];
  const int cap = maxb << bs_log2;
  ctx = ctx > cap ? cap : ctx;
  const int n = (ctx + CHUNK - 1) / CHUNK;
  if (ctx <= 0 || n <= 1) return;
  const int64_t row = (int64_t)b * Hq + h;
  const float *ml = ws_ml + row * max_chunks * 2;
  const float *ac = ws_acc + row * max_chunks * HD;
  float M = -INFINITY;
  for (int i = 0; i < n; ++i) M = fmaxf(M, ml[2 * i]);
  float L = 0.f, A = 0.f;
  for (int i = 0; i < n; ++i) {
    const float sc = fast_exp2(ml[2 * i] - M);
    L += ml[2 * i + 1] * sc;
    A += ac[(int64_t)i * HD + d] * sc;
  }
  out[row * HD + d] = F16T::from_float(A / L);
}

constexpr int DEC_CHUNK = 256;

static int max_chunks_for(int max_blocks_per_seq, int block_size) {
  const int64_t cap = (int64_t)max_blocks_per_seq * block_size;
  return (int)((cap + DEC_CHUNK - 1) / DEC_CHUNK);
}

template <int G>
static void launch_decode(const uint16_t *q, const uint16_t *kc,
                          const uint16_t *vc, const int32_t *bt,
                          const int32_t *cl, uint16_t *out, float *wacc,
                          float *wml, int B, int Hq, int Hkv, int maxb,
                          int bs_log2, int64_t nblocks, float scale_log2,
                          int max_chunks, hipStream_t st) {
  dim3 grid(Hkv, max_chunks, B);
  paged_decode_kernel<G, DEC_CHUNK><<<grid, DEC_NW * 64, 0, st>>>(
      q, kc, vc, bt, cl, out, wacc, wml, Hq, Hkv, maxb, bs_log2, nblocks,
      scale_log2, max_chunks);
  if (max_chunks > 1)
    paged_decode_merge_kernel<DEC_CHUNK><<<dim3(Hq, B), HD, 0, st>>>(
        wacc, wml, cl, out, Hq, maxb, bs_log2, max_chunks);
}

}  // namespace mce

using namespace mce;

extern "C" size_t mce_paged_attention_decode_workspace_size(
    int batch, int num_heads, int max_blocks_per_seq, int block_size) {
  if (batch <= 0 || num_heads <= 0 || max_blocks_per_seq <= 0 ||
      block_size <= 0)
    return 0;
  const int mc = max_chunks_for(max_blocks_per_seq, block_size);
  if (mc <= 1) return 0;
  // acc [B, Hq, mc, 128] fp32, then (m, l) [B, Hq, mc, 2] fp32
  return (size_t)batch * num_heads * mc * (HD + 2) * sizeof(float);
}

extern "C" int mce_paged_attention_decode(
    int dtype, const void *query, const void *key_cache,
    const void *value_cache, const int32_t *block_tables,
    const int32_t *context_lens, void *output, int batch, int num_heads,
    int num_kv_heads, int head_dim, int max_blocks_per_seq, int block_size,
    int64_t num_blocks, float scale, void *workspace, size_t workspace_bytes,
    void *stream) {
  clear_error();
  MCE_REQUIRE(dtype == MCE_F16 || dtype == MCE_BF16,
              "mce_paged_attention_decode: unknown dtype %d", dtype);
  if (dtype != MCE_F16)
    return set_error(MCE_ERR_UNSUPPORTED,
                     "mce_paged_attention_decode: only fp16 is implemented");
  MCE_REQUIRE(head_dim == HD, "mce_paged_attention_decode: head_dim must be 128 (got %d)", head_dim);
  MCE_REQUIRE(batch >= 0 && num_heads >= 1 && num_kv_heads >= 1,
              "mce_paged_attention_decode: bad head counts");
  MCE_REQUIRE(num_heads % num_kv_heads == 0,
              "mce_paged_attention_decode: num_heads %d not a multiple of num_kv_heads %d",
              num_heads, num_kv_heads);
  const int G = num_heads / num_kv_heads;
  if (G > 8)
    return set_error(MCE_ERR_UNSUPPORTED,
                     "mce_paged_attention_decode: GQA group %d > 8 unsupported", G);
  MCE_REQUIRE(is_pow2(block_size) && block_size >= 8 && block_size <= 256,
              "mce_paged_attention_decode: block_size must be a power of two in [8, 256] (got %d)",
              block_size);
  MCE_REQUIRE(max_blocks_per_seq >= 1, "mce_paged_attention_decode: max_blocks_per_seq must be >= 1");
  MCE_REQUIRE(num_blocks >= 1, "mce_paged_attention_decode: empty KV pool");
  if (batch == 0) return MCE_OK;
  MCE_REQUIRE(query && key_cache && value_cache && block_tables &&
                  context_lens && output,
              "mce_paged_attention_decode: null pointer");
  MCE_REQUIRE(aligned16(query) && aligned16(key_cache) &&
                  aligned16(value_cache),
              "mce_paged_attention_decode: query and caches must be 16-byte aligned");
  const int max_chunks = max_chunks_for(max_blocks_per_seq, block_size);
  MCE_REQUIRE(max_chunks <= 65535, "mce_paged_attention_decode: context too long");
  MCE_REQUIRE(batch <= 65535, "mce_paged_attention_decode: batch too large");
  const size_t need = mce_paged_attention_decode_workspace_size(
      batch, num_heads, max_blocks_per_seq, block_size);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need))
    return set_error(MCE_ERR_WORKSPACE,
                     "mce_paged_attention_decode: workspace of %zu bytes required, %zu given",
                     need, workspace_bytes);
  float *wacc = (float *)workspace;
  float *wml = wacc ? wacc + (size_t)batch * num_heads * max_chunks * HD : nullptr;
  const float scale_log2 = scale * 1.4426950408889634f;
  const int bs_log2 = ilog2(block_size);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t *q = (const uint16_t *)query;
  const uint16_t *kc = (const uint16_t *)key_cache;
  const uint16_t *vc = (const uint16_t *)value_cache;
  uint16_t *out = (uint16_t *)output;
#define MCE_DEC_CASE(GG)                                                      \
  case GG:                                                                    \
    launch_decode<GG>(q, kc, vc, block_tables, context_lens, out, wacc, wml,  \
                      batch, num_heads, num_kv_heads, max_blocks_per_seq,     \
                      bs_log2, num_blocks, scale_log2, max_chunks, st);       \
    break;
  switch (G) {
    MCE_DEC_CASE(1)
    MCE_DEC_CASE(2)
    MCE_DEC_CASE(3)
    MCE_DEC_CASE(4)
    MCE_DEC_CASE(5)
    MCE_DEC_CASE(6)
    MCE_DEC_CASE(7)
    MCE_DEC_CASE(8)
  }
#undef MCE_DEC_CASE
  return check_launch("mce_paged_attention_decode");
}
