// Paged decode attention for gfx950 (reference semantics:
// csrc/kernels/flash_attn_paged.cu:25-142, host wrapper :144-168).
//
// Work decomposition (split-K / flash-decoding):
//   one workgroup = (kv head g, chunk c of `chunk` tokens, sequence b).
//   All G = num_heads / num_kv_heads query heads of kv head g are handled by
//   the same workgroup, so every K/V byte is read from HBM exactly once (the
//   reference launches one warp per query head and reads each KV row G times).
//   A sequence that fits in one chunk is normalised and written directly.
//   Otherwise every chunk writes its partial softmax state (max m, sum l,
//   unnormalised acc[128], per query head) to the workspace, and a second
//   kernel merges the partials of each (sequence, query head) by log-sum-exp.
//   (Merging in the last-arriving workgroup instead would need agent-scope
//   release/acquire fences, which on gfx950 write back the whole L2 per
//   workgroup; the kernel boundary gives the same visibility for free.)
//
// Inside a workgroup DEC_NW waves take 32-token tiles round-robin, with the
// next tile's K/V loads in flight while the current tile is computed:
//   * the chunk's physical block ids are staged once in LDS;
//   * K^T tile -> MFMA B operand straight from global memory: lane l loads
//     token (l % 16) of each 16-token half, 4 x 16 bytes, so one instruction
//     covers 64 contiguous bytes of 16 token rows.
//     S = Q K^T with v_mfma_f32_16x16x32_f16, A = Q (rows = query heads,
//     zero-padded to 16).  S row h lands in lane group h / 4, register h % 4.
//   * online softmax in base 2 (scale * log2 e folded in), per wave.
//   * p goes through a small LDS slice as fp16 ([head][token]); V rows are
//     read as 16-byte pieces (16 lanes cover one 256-byte token row, 4 rows
//     per instruction) and accumulated with v_dot2_f32_f16 over token pairs.
#include "mce_common.h"

namespace mce {

constexpr int HD = 128;         // head_dim
constexpr int TILE = 32;        // tokens per wave iteration
constexpr int DEC_NW = 4;       // waves per workgroup
constexpr int MAX_CHUNK = 1024;
constexpr int MIN_BS = 8;
constexpr int MAX_CHUNK_BLOCKS = MAX_CHUNK / MIN_BS + 1;

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

struct DecodeWs {
  float *ml;   // [B, Hq, max_chunks, 2]  (m, l) per chunk
  float *acc;  // [B, Hq, max_chunks, HD] unnormalised partial output
};

template <int G>
__global__ __launch_bounds__(DEC_NW * 64) __attribute__((amdgpu_waves_per_eu(2)))
void paged_decode_kernel(
    const uint16_t *__restrict__ query, const uint16_t *__restrict__ kcache,
    const uint16_t *__restrict__ vcache, const int32_t *__restrict__ btab,
    const int32_t *__restrict__ ctx_lens, uint16_t *__restrict__ out,
    DecodeWs ws, int Hq, int Hkv, int maxb, int bs_log2, int64_t num_blocks,
    float scale_log2, int chunk, int max_chunks) {
  const int g = blockIdx.x, c = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int bs = 1 << bs_log2;
  const int head0 = g * G;

  int ctx = ctx_lens[b];
  const int cap = maxb << bs_log2;
  ctx = ctx > cap ? cap : ctx;
  if (ctx <= 0) {  // defined output for empty sequences: zeros
    if (c == 0)
      for (int i = tid; i < G * HD; i += DEC_NW * 64)
        out[((int64_t)b * Hq + head0) * HD + i] = 0;
    return;
  }
  const int t_begin = c * chunk;
  if (t_begin >= ctx) return;
  const int t_end = min(t_begin + chunk, ctx);
  const int nchunks = (ctx + chunk - 1) / chunk;

  __shared__ int blk_lds[MAX_CHUNK_BLOCKS];
  // p of one tile as packed fp16 token pairs: [wave][head][pair / 4][pair % 4]
  __shared__ u32x4 p_lds[DEC_NW][G][TILE / 8];
  __shared__ float red_acc[DEC_NW][G][HD];
  __shared__ float red_m[DEC_NW][G], red_l[DEC_NW][G];

  // Physical block ids of this chunk, clamped into the pool.
  const int first_blk = t_begin >> bs_log2;
  const int nblk = ((t_end - 1) >> bs_log2) - first_blk + 1;
  {
    const int32_t *bt = btab + (int64_t)b * maxb + first_blk;
    const int hi = (int)(num_blocks - 1 < 0x7fffffff ? num_blocks - 1 : 0x7fffffff);
    for (int i = tid; i < nblk; i += DEC_NW * 64) {
      int v = bt[i];
      blk_lds[i] = v < 0 ? 0 : (v > hi ? hi : v);
    }
  }

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
  __syncthreads();

  float m_run[G], l_part[4], acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m_run[h] = -INFINITY;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) l_part[j] = 0.f;

  const int64_t slot_stride = (int64_t)Hkv * HD;  // elements between slots
  const uint16_t *kbase = kcache + (int64_t)g * HD;
  const uint16_t *vbase = vcache + (int64_t)g * HD;
  auto slot_of = [&](int t) -> int64_t {
    const int64_t phys = blk_lds[(t >> bs_log2) - first_blk];
    return (phys << bs_log2) + (t & (bs - 1));
  };

  // ---- loads of one tile into registers ----
  auto load_tile = [&](int t0, half8 (&kb)[2][4], u32x4 (&vv)[8]) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      int t = t0 + 16 * u + lr;
      t = t < t_end ? t : t_end - 1;
      const uint16_t *kp = kbase + slot_of(t) * slot_stride + lg * 8;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        kb[u][i] = __builtin_bit_cast(
            half8, *reinterpret_cast<const u32x4 *>(kp + i * 32));
    }
    // lane group lg owns tokens t0 + 8 lg .. +7 (one block: bs >= 8)
    int tv = t0 + 8 * lg;
    tv = tv < t_end ? tv : t0;
    const uint16_t *vp = vbase + slot_of(tv) * slot_stride + lr * 8;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      vv[s] = *reinterpret_cast<const u32x4 *>(vp + s * slot_stride);
  };

  // ---- compute of one tile ----
  auto compute_tile = [&](int t0, const half8 (&kb)[2][4], u32x4 (&vv)[8]) {
    floatx4 sacc[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      sacc[u] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sacc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[i], kb[u][i],
                                                         sacc[u], 0, 0, 0);
    }
    float s[2][4];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const bool valid = t0 + 16 * u + lr < t_end;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        s[u][j] = valid ? sacc[u][j] * scale_log2 : -INFINITY;
    }
    float mx[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) mx[j] = row16_max(fmaxf(s[0][j], s[1][j]));

    float alpha[G];
    bool rescale = false;
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float tmax = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mx[h & 3]),
                                           16 * (h >> 2)));
      const float mn = fmaxf(m_run[h], tmax);
      alpha[h] = fast_exp2(m_run[h] - mn);
      rescale |= mn != m_run[h];
      m_run[h] = mn;
    }
    // p for the head held in register j of this lane (head 4 lg + j)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float mj = 0.f, a = 1.f;
#pragma unroll
      for (int h = 0; h < G; ++h)
        if ((h & 3) == j && lg == (h >> 2)) {
          mj = m_run[h];
          a = alpha[h];
        }
      const float p0 = fast_exp2(s[0][j] - mj), p1 = fast_exp2(s[1][j] - mj);
      l_part[j] = l_part[j] * a + p0 + p1;
      // even lanes store (p[t], p[t + 1]) for tokens t = lr and 16 + lr
      const float p0n = dpp_f<0xB1>(p0), p1n = dpp_f<0xB1>(p1);
      const int h = 4 * lg + j;
      if (h < G && (lr & 1) == 0) {
        const int pair = lr >> 1;
        p_lds[w][h][pair >> 2][pair & 3] = pack2<F16T>(p0, p0n);
        p_lds[w][h][2 + (pair >> 2)][pair & 3] = pack2<F16T>(p1, p1n);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    if (rescale) {
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] *= alpha[h];
    }
    // tokens past the end: zero their V rows (p is 0, V may be NaN garbage)
    const int tv = t0 + 8 * lg;
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8)
      if (tv + s8 >= t_end) vv[s8] = u32x4{0, 0, 0, 0};
    // ---- acc += P V over token pairs with v_dot2_f32_f16 ----
    u32x4 pr[G];
#pragma unroll
    for (int h = 0; h < G; ++h)
      pr[h] = p_lds[w][h][lg];
#pragma unroll
    for (int sp = 0; sp < 4; ++sp)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const h2 lo = __builtin_bit_cast(
            h2, __builtin_amdgcn_perm(vv[2 * sp + 1][k], vv[2 * sp][k], 0x05040100u));
        const h2 hi = __builtin_bit_cast(
            h2, __builtin_amdgcn_perm(vv[2 * sp + 1][k], vv[2 * sp][k], 0x07060302u));
#pragma unroll
        for (int h = 0; h < G; ++h) {
          // (explicit conversion: bit_cast of an ext-vector element picks element 0
          // in this compiler)
          const h2 ph = __builtin_bit_cast(h2, (uint32_t)pr[h][sp]);
          acc[h][2 * k] = __builtin_amdgcn_fdot2(lo, ph, acc[h][2 * k], false);
          acc[h][2 * k + 1] = __builtin_amdgcn_fdot2(hi, ph, acc[h][2 * k + 1], false);
        }
      }
    __builtin_amdgcn_wave_barrier();
  };

  // ---- software-pipelined tile loop: next tile's loads before compute ----
  const int ntile = (t_end - t_begin + TILE - 1) / TILE;
  half8 kA[2][4], kB[2][4];
  u32x4 vA[8], vB[8];
  int j = w;
  if (j < ntile) load_tile(t_begin + TILE * j, kA, vA);
  while (j < ntile) {
    int jn = j + DEC_NW;
    if (jn < ntile) load_tile(t_begin + TILE * jn, kB, vB);
    compute_tile(t_begin + TILE * j, kA, vA);
    j = jn;
    if (j >= ntile) break;
    jn = j + DEC_NW;
    if (jn < ntile) load_tile(t_begin + TILE * jn, kA, vA);
    compute_tile(t_begin + TILE * j, kB, vB);
    j = jn;
  }

  // ---- per-wave reduction ----
#pragma unroll
  for (int jj = 0; jj < 4; ++jj) l_part[jj] = row16_sum(l_part[jj]);
  float l_tot[G];
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
  const int64_t row0 = (int64_t)b * Hq + head0;
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
    if (nchunks == 1) {
      out[(row0 + h) * HD + d] = F16T::from_float(A / L);
    } else {
      const int64_t pr = (row0 + h) * max_chunks + c;
      ws.acc[pr * HD + d] = A;
      if (d == 0) {
        ws.ml[pr * 2] = M;
        ws.ml[pr * 2 + 1] = L;
      }
    }
  }
}

// Log-sum-exp merge of split-K partials: one 128-lane workgroup per
// (query head, sequence); lane d owns output dim d.  Chunks are merged 128 at
// a time: lane i loads chunk i's (m, l), the block max rescales them into LDS
// weights, and every lane then streams its dim of the partial outputs with
// independent (unrolled) loads.
__global__ __launch_bounds__(HD) void paged_decode_merge_kernel(
    DecodeWs ws, const int32_t *__restrict__ ctx_lens, uint16_t *__restrict__ out,
    int Hq, int maxb, int bs_log2, int chunk, int max_chunks) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  int ctx = ctx_lens[b];
  const int cap = maxb << bs_log2;
  ctx = ctx > cap ? cap : ctx;
  const int n = ctx > 0 ? (ctx + chunk - 1) / chunk : 0;
  if (n <= 1) return;
  __shared__ float w_lds[HD], wl_lds[HD], mx_lds[2];
  const int64_t row = (int64_t)b * Hq + h;
  const float *ml = ws.ml + row * max_chunks * 2;
  const float *ac = ws.acc + row * max_chunks * HD + d;
  float M = -INFINITY, L = 0.f, A = 0.f;
  for (int c0 = 0; c0 < n; c0 += HD) {
    const int cn = min(HD, n - c0);
    const float mi = d < cn ? ml[2 * (c0 + d)] : -INFINITY;
    const float li = d < cn ? ml[2 * (c0 + d) + 1] : 0.f;
    const float wm = wave_max(mi);
    if ((d & 63) == 0) mx_lds[d >> 6] = wm;
    __syncthreads();
    const float m_new = fmaxf(M, fmaxf(mx_lds[0], mx_lds[1]));
    const float wi = d < cn ? fast_exp2(mi - m_new) : 0.f;
    w_lds[d] = wi;
    wl_lds[d] = wi * li;
    __syncthreads();
    const float sc = fast_exp2(M - m_new);  // 0 on the first pass
    A *= sc;
    L *= sc;
    int i = 0;
    for (; i + 8 <= cn; i += 8) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = ac[(int64_t)(c0 + i + k) * HD];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        A += w_lds[i + k] * v[k];
        L += wl_lds[i + k];
      }
    }
    for (; i < cn; ++i) {
      A += w_lds[i] * ac[(int64_t)(c0 + i) * HD];
      L += wl_lds[i];
    }
    M = m_new;
    __syncthreads();
  }
  out[row * HD + d] = F16T::from_float(A / L);
}

// Chunk length (tokens per workgroup): the largest of 1024/512/256/128 that
// still gives >= 2048 (kv head, chunk, sequence) units for the worst-case
// context, so short batches spread over all CUs and long ones amortise the
// per-workgroup prologue/epilogue.  Depends only on host-known sizes.
static int pick_chunk(int batch, int num_kv_heads, int max_blocks_per_seq,
                      int block_size) {
  const int64_t cap = (int64_t)max_blocks_per_seq * block_size;
  const int64_t pairs = (int64_t)batch * num_kv_heads;
  for (int ch = MAX_CHUNK; ch > 128; ch /= 2)
    if (pairs * ((cap + ch - 1) / ch) >= 2048) return ch;
  return 128;
}

struct DecodeLayout {
  int chunk, max_chunks;
  size_t ml_off, acc_off, total;
};

static DecodeLayout decode_layout(int batch, int num_heads, int num_kv_heads,
                                  int max_blocks_per_seq, int block_size) {
  DecodeLayout L{};
  L.chunk = pick_chunk(batch, num_kv_heads, max_blocks_per_seq, block_size);
  const int64_t cap = (int64_t)max_blocks_per_seq * block_size;
  L.max_chunks = (int)((cap + L.chunk - 1) / L.chunk);
  if (L.max_chunks <= 1) return L;  // no workspace needed
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  L.ml_off = 0;
  L.acc_off = up((size_t)batch * num_heads * L.max_chunks * 2 * sizeof(float));
  L.total = L.acc_off + (size_t)batch * num_heads * L.max_chunks * HD * sizeof(float);
  return L;
}

}  // namespace mce

using namespace mce;

extern "C" size_t mce_paged_attention_decode_workspace_size(
    int batch, int num_heads, int num_kv_heads, int max_blocks_per_seq,
    int block_size) {
  if (batch <= 0 || num_heads <= 0 || num_kv_heads <= 0 ||
      max_blocks_per_seq <= 0 || block_size <= 0)
    return 0;
  return decode_layout(batch, num_heads, num_kv_heads, max_blocks_per_seq,
                       block_size).total;
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
  MCE_REQUIRE(is_pow2(block_size) && block_size >= MIN_BS && block_size <= 256,
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
  MCE_REQUIRE((int64_t)max_blocks_per_seq * block_size <= ((int64_t)1 << 30),
              "mce_paged_attention_decode: context capacity too large");
  const DecodeLayout Lay = decode_layout(batch, num_heads, num_kv_heads,
                                         max_blocks_per_seq, block_size);
  MCE_REQUIRE(Lay.max_chunks <= 65535, "mce_paged_attention_decode: context too long");
  MCE_REQUIRE(batch <= 65535, "mce_paged_attention_decode: batch too large");
  if (Lay.total > 0 && (workspace == nullptr || workspace_bytes < Lay.total ||
                        (reinterpret_cast<uintptr_t>(workspace) & 255) != 0))
    return set_error(MCE_ERR_WORKSPACE,
                     "mce_paged_attention_decode: a 256-byte aligned workspace of %zu bytes "
                     "is required (%zu given)",
                     Lay.total, workspace_bytes);
  DecodeWs ws{};
  if (Lay.total > 0) {
    char *base = (char *)workspace;
    ws.ml = (float *)(base + Lay.ml_off);
    ws.acc = (float *)(base + Lay.acc_off);
  }
  const float scale_log2 = scale * 1.4426950408889634f;
  const int bs_log2 = ilog2(block_size);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t *q = (const uint16_t *)query;
  const uint16_t *kc = (const uint16_t *)key_cache;
  const uint16_t *vc = (const uint16_t *)value_cache;
  uint16_t *out = (uint16_t *)output;
  dim3 grid(num_kv_heads, Lay.max_chunks, batch);
#define MCE_DEC_CASE(GG)                                                       \
  case GG:                                                                     \
    paged_decode_kernel<GG><<<grid, DEC_NW * 64, 0, st>>>(                     \
        q, kc, vc, block_tables, context_lens, out, ws, num_heads,             \
        num_kv_heads, max_blocks_per_seq, bs_log2, num_blocks, scale_log2,     \
        Lay.chunk, Lay.max_chunks);                                            \
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
  if (Lay.max_chunks > 1)
    paged_decode_merge_kernel<<<dim3(num_heads, batch), HD, 0, st>>>(
        ws, context_lens, out, num_heads, max_blocks_per_seq, bs_log2, Lay.chunk,
        Lay.max_chunks);
  return check_launch("mce_paged_attention_decode");
}
