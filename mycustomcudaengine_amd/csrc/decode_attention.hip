// Paged decode attention for gfx950 (reference semantics:
// csrc/kernels/flash_attn_paged.cu:25-142, host wrapper :144-168).
//
// Work decomposition: balanced split-K (flash-decoding) over the whole batch.
//   Every sequence's context is cut into 16-token tiles and the tiles of all
//   sequences are laid end to end (sequence b owns tiles [pre[b], pre[b+1]),
//   the first SEG_TILES of them virtual: they weight the cost of a segment).
//   The grid has J workgroups per group of kv heads (about one workgroup per
//   CU in total) and workgroup j takes the contiguous tile range
//   [j NT / J, (j+1) NT / J): every workgroup gets the same split weight
//   (streamed tiles plus segment starts) whatever the mix of context
//   lengths, so there is no tail of short chunks.  A range may cover the end of one sequence and the start of the
//   next; each such piece ("segment") is reduced separately.
//   A workgroup has 8 waves and covers up to 8 kv heads of its tile range:
//   wave w works on kv head w % HPG (HPG = heads per workgroup) and on every
//   WPH-th tile (WPH = 8 / HPG waves per head).  With 8 kv heads, the waves
//   of a workgroup together sweep whole contiguous 16-token x 2 KB pages, and
//   each wave owns a head outright (no cross-wave merge).  Reading one head's
//   256-byte slice per workgroup instead measured ~15% slower on MI355X.
//   All G = num_heads / num_kv_heads query heads of a kv head are handled by
//   the same wave, so every K/V byte is read from HBM exactly once (the
//   reference launches one warp per query head and reads each KV row G times).
//   K/V are streamed with non-temporal loads (each byte is used once).
//   Short contexts (capacity <= PER_SEQ_MAX_TOKENS) skip the split: the grid
//   is one 8-wave workgroup per (kv head, sequence), the waves share the
//   tiles of that head and merge in LDS, and the rows are written directly
//   by a single kernel (the split's merge pass and its latency chain cost
//   more than the few hundred KB each workgroup then streams).
//   A sequence that lies inside one workgroup is normalised and written
//   directly; otherwise each segment writes its partial softmax state (max m,
//   sum l, unnormalised acc[128]) to the workspace and a second kernel merges
//   the partials of each (sequence, query head) by log-sum-exp.  Partial slots
//   are compact: workgroup j writes its piece of sequence b to slot j + b of
//   each query head's row of J + B slots.  (The pieces of b sit in workgroups
//   j_first(b) .. j_last(b) and j_first(b') >= j_last(b) for b' > b, so the
//   slot ranges [j_first(b) + b, j_last(b) + b] never overlap.)  Workgroup 0
//   records each sequence's first slot and part count for the merge.  (Merging in
//   the last-arriving workgroup would need agent-scope release/acquire
//   fences, which on gfx950 write back the L2 per workgroup; the kernel
//   boundary gives the same visibility for free.)
//
// Per wave and 16-token tile; a wave issues its next tile's loads once the
// current tile's scores are computed, so they land while its P V runs.  One 8
// KB tile in flight per wave (with a workgroup of 8
// waves on every CU, ~16 MB across the chip) covers the memory latency and
// streams faster than more: 32-token tiles, or a second tile in flight per
// wave, measured slower, and 8-token tiles slower again:
//   * the segment's physical block ids are staged in LDS; each wave's first
//     tile reads its ids straight from the table row, so its K/V loads
//     leave before the staging's LDS writes and barrier;
//   * lane group lg (16 lanes) owns tokens TPG lg .. TPG lg + TPG - 1 of the
//     tile and lane lr owns dims 8 lr .. 8 lr + 7: every K and V load
//     instruction reads four whole 256-byte token rows (the pattern that streams fastest on
//     MI355X; loading K in an MFMA-operand layout, 64-byte pieces of 16 rows
//     per instruction, measured ~6% slower);
//   * scores: v_dot2_f32_f16 (v_dot2_f32_bf16 for bf16) over the lane's dims
//     and a 16-lane DPP sum, so every lane of a group holds its tokens'
//     scores for all G query heads;
//   * online softmax in base 2 (p = exp2((s - m) c), c = scale log2 e);
//   * P V with v_dot2 over token pairs (p packed as fp16 / bf16), from the
//     same registers -- no LDS round trip for p.
#include <mutex>

#include "mce_common.h"

namespace mce {

constexpr int HD = 128;           // head_dim
constexpr int TILE = 16;          // tokens per wave iteration
constexpr int TPG = TILE / 4;     // tokens per 16-lane group
constexpr int DEC_NW = 8;         // waves per workgroup
constexpr int NT_THREADS = DEC_NW * 64;
constexpr int MIN_BS = 8;
constexpr int MAX_IDS = 2048;     // block ids staged in LDS at a time
constexpr int MAX_BATCH = 2048;   // sequences per call (LDS prefix array)
constexpr int MIN_TILES_PER_WG = 4;
// Split weight of a sequence start, in tiles: starting a segment (query and
// block-id loads, pipeline refill, one more partial) costs two to four tiles of
// streaming, so every non-empty sequence is preceded by SEG_TILES virtual
// tiles in the split space and a workgroup that takes a boundary gets that
// many fewer real tiles.
constexpr int SEG_TILES = 2;
// Context capacities up to this many tokens take the per-sequence mode.
constexpr int PER_SEQ_MAX_TOKENS = 1024;


struct DecodeArgs {
  const uint16_t *query;    // [B, Hq, HD] rows q_stride_b elements apart
  const uint16_t *kcache;   // [NB, BS, Hkv, HD]
  const uint16_t *vcache;
  const int32_t *btab;      // [B, maxb]
  const int32_t *ctx_lens;  // [B]
  uint16_t *out;            // [B, Hq, HD]
  float *ws_ml;             // [Hq, S, 2]
  float *ws_acc;            // [Hq, S, HD]
  int *ws_meta;             // [B, 2]: first slot and part count of each sequence
  int B, Hq, Hkv, maxb, bs_log2, J;
  int S;                    // part slots per query head: J + B
  int hpg, wph;             // kv heads per workgroup, waves per kv head
  int per_seq;              // 1: workgroup (group, b) covers all of sequence b
  int64_t q_stride_b;       // elements between the query rows of two sequences
  // Fused RoPE + KV append (per-sequence mode; knew == nullptr: off): the
  // query is rotated in registers, and k (rotated) and v of the new token are
  // written to the page slot before the attention reads the sequence.
  const uint16_t *knew, *vnew;  // [B, Hkv, HD] rows new_stride_b elements apart
  int64_t new_stride_b;
  const float *rope_cos, *rope_sin;  // [table_rows, HD / 2]
  const int32_t *positions, *slots;  // [B]
  int64_t table_rows, num_slots;
  int64_t num_blocks;
  float scale_log2;
};

__device__ inline int clamp_ctx(int c, int cap) { return c < 0 ? 0 : (c > cap ? cap : c); }

// One stage of row16_sum applied to every value of v.
template <int CTRL, int N, int M>
__device__ __forceinline__ void row16_sum_stage(float (&v)[N][M]) {
#pragma unroll
  for (int i = 0; i < N; ++i)
#pragma unroll
    for (int j = 0; j < M; ++j) v[i][j] += dpp_f<CTRL>(v[i][j]);
}

// Exclusive prefix sum of per-sequence split weights (tiles + SEG_TILES for a
// non-empty sequence) into pre[0..B], and the clamped context lengths into
// ctx_out[0..B) (so the segments do not load them again); returns NT.  Sequence b's real tiles
// are [pre[b] + SEG_TILES, pre[b+1]).
template <int NW>
__device__ int build_tile_prefix(const DecodeArgs &a, int *pre, int *wave_tot, int *ctx_out) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int cap = a.maxb << a.bs_log2;
  int carry = 0;
  for (int base = 0; base < a.B; base += NW * 64) {
    const int b = base + tid;
    const int cb = b < a.B ? clamp_ctx(a.ctx_lens[b], cap) : 0;
    if (b < a.B) ctx_out[b] = cb;
    int v = (cb + TILE - 1) / TILE;
    if (v > 0) v += SEG_TILES;
    const int incl = wave_incl_scan(v);
    if (lane == 63) wave_tot[w] = incl;
    lds_barrier();
    int before = carry;
    for (int ww = 0; ww < w; ++ww) before += wave_tot[ww];
    if (b < a.B) pre[b] = before + incl - v;
    int total = 0;
    for (int ww = 0; ww < NW; ++ww) total += wave_tot[ww];
    carry += total;
    lds_barrier();
  }
  if (tid == 0) pre[a.B] = carry;
  lds_barrier();
  return carry;
}

__device__ inline int partition_count(int NT, int J) {
  int je = (NT + MIN_TILES_PER_WG - 1) / MIN_TILES_PER_WG;
  return je < 1 ? 1 : (je > J ? J : je);
}
__device__ inline int range_start(int j, int NT, int je) {
  return (int)((int64_t)j * NT / je);
}
// workgroup index that owns tile t
__device__ inline int owner_of(int t, int NT, int je) {
  return (int)(((int64_t)(t + 1) * je - 1) / NT);
}

__device__ inline u32x4 ld_nt(const uint16_t *p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}

// cos / sin of the lane's four rotation pairs (dims 8 (lr & 7) .. +7 of the
// first half), fetched apart from the rotation so the loads can be issued early
struct RopeCS {
  floatx4 c0, c1, s0, s1;
};

__device__ inline RopeCS rope_fetch(const DecodeArgs &a, int pos, int lr) {
  const int i0 = 8 * (lr & 7);  // rotation index of the lane's first dim
  const float *cp = a.rope_cos + (int64_t)pos * (HD / 2) + i0;
  const float *sp = a.rope_sin + (int64_t)pos * (HD / 2) + i0;
  RopeCS r;
  r.c0 = *reinterpret_cast<const floatx4 *>(cp);
  r.c1 = *reinterpret_cast<const floatx4 *>(cp + 4);
  r.s0 = *reinterpret_cast<const floatx4 *>(sp);
  r.s1 = *reinterpret_cast<const floatx4 *>(sp + 4);
  return r;
}

// RoPE of one 128-dim head row spread over a 16-lane group: lane lr holds
// dims 8 lr .. 8 lr + 7; the rotation pairs dim i < 64 with i + 64, i.e. lane
// lr with lane lr ^ 8 (all 64 lanes take part in the exchange).  Returns the
// lane's rotated 8 values, rounded as rope_inplace rounds them.
template <class T>
__device__ inline u32x4 rope_apply(const u32x4 x, const RopeCS &r, int lr) {
  u32x4 pt;
#pragma unroll
  // lane lr ^ 8 of the same 16-lane row: DPP row_ror:8 (no LDS round trip)
  for (int k = 0; k < 4; ++k)
    pt[k] = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x[k], 0x128, 0xf, 0xf, false);
  const bool lo_half = lr < 8;
  u32x4 o;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float cl = k < 2 ? r.c0[2 * k] : r.c1[2 * k - 4], ch = k < 2 ? r.c0[2 * k + 1] : r.c1[2 * k - 3];
    const float sl = k < 2 ? r.s0[2 * k] : r.s1[2 * k - 4], sh = k < 2 ? r.s0[2 * k + 1] : r.s1[2 * k - 3];
    // (x0, x1) = (dim i, dim i + 64) of this element pair
    const float a0 = T::lo(lo_half ? x[k] : pt[k]), a1 = T::lo(lo_half ? pt[k] : x[k]);
    const float b0 = T::hi(lo_half ? x[k] : pt[k]), b1 = T::hi(lo_half ? pt[k] : x[k]);
    float ra0, ra1, rb0, rb1;
    rope_pair(a0, a1, cl, sl, ra0, ra1);
    rope_pair(b0, b1, ch, sh, rb0, rb1);
    o[k] = lo_half ? pack2<T>(ra0, rb0) : pack2<T>(ra1, rb1);
  }
  return o;
}

// Two waves per SIMD: one NW = 8-wave workgroup per CU.  (GQA groups of 7 or
// 8 query heads per kv head spill a few registers at this occupancy.)
// FUSED: RoPE + KV append of the new token (per-sequence mode only; a.knew
// set), a separate instantiation so the plain kernels carry none of its state.
template <class T, int G, int NW, bool FUSED>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(NW / 4)))
void paged_decode_kernel(DecodeArgs a) {
  constexpr int NTH = NW * 64;
  // per-sequence mode: blockIdx.x = slice * Hkv + kv head (the gsplit
  // workgroups of one kv head share an XCD when Hkv is a multiple of 8)
  const int gsub = a.per_seq ? (int)blockIdx.x / a.Hkv : 0;  // query-head slice
  const int hgrp = a.per_seq ? (int)blockIdx.x % a.Hkv : (int)blockIdx.x, j = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int bs_log2 = a.bs_log2, bs = 1 << bs_log2;
  const int cap = a.maxb << bs_log2;
  const int hpg = a.hpg, wph = a.wph;
  const int hl = w % hpg, rlane = w / hpg;       // head in group, tile lane
  const int g = hgrp * hpg + hl;                 // this wave's kv head
  const bool active = rlane < wph && g < a.Hkv;  // uniform per wave
  const int gq = a.Hq / a.Hkv;                   // query heads per kv head
  const int head0 = g * gq + gsub * G;           // this wave's G query heads

  __shared__ int pre[MAX_BATCH + 1];
  __shared__ int wave_tot[NW];
  __shared__ int blk_lds[MAX_IDS];
  __shared__ int ctx_lds[MAX_BATCH];
  const int nb_hi = (int)(a.num_blocks - 1 < 0x7fffffff ? a.num_blocks - 1 : 0x7fffffff);
  __shared__ float red_acc[NW][G][HD];
  __shared__ float red_m[NW][G], red_l[NW][G];

  int NT, je, seg0;  // seg0: virtual tiles at the start of each sequence
  int ctx_j = 0;     // per-sequence mode: the context length, kept for the tile loop
  // fused RoPE + KV append (per-sequence mode): the new token's state
  int pos_j = 0;
  int64_t slot_j = -1;  // -1: no store, nothing to substitute
  bool rope_ok = false;
  RopeCS cs_new{};
  u32x4 kx_new{}, vx_new{}, q_pre[G];
  __shared__ u32x4 knv_lds[32];  // rotated k (lanes 0-15) and v (16-31) of the new token
  u32x4 kA[TPG], vA[TPG];  // the wave's first tile (fused mode: fetched in the prologue)
  int64_t phys_f = 0;      // fused mode: physical block and first row of those rows
  int tv_f = 0;
  if (a.per_seq) {
    seg0 = 0;
    // one workgroup per (head group, sequence j): a one-sequence tile space
    // [0, tiles of j), so the segment loop below runs once with nparts == 1
    // and the rows are written directly (no merge pass).  The sequence's
    // block ids (at most PER_SEQ_MAX_TOKENS / MIN_BS of them) are fetched
    // together with its context length.
    // (maxb <= PER_SEQ_MAX_TOKENS / MIN_BS <= NTH: one block id per thread)
    const int32_t *btj = a.btab + (int64_t)j * a.maxb;
    // Fused mode: the wave's first tile (tile rlane) does not wait for the
    // staging.  Each lane group reads its block id straight from the table
    // row (the first load issued), and the tile's K/V loads leave once the
    // prologue's other loads are issued (position first, so the cos / sin
    // fetch goes out before the K/V).  Tokens past the context are masked by
    // the tile computation; the row index stays in the table.  (The plain
    // kernel measured no faster this way: it stages first.)
    const int tvf = TILE * rlane + TPG * lg;
    const int idf = FUSED ? btj[min(tvf >> bs_log2, a.maxb - 1)] : 0;
    if constexpr (FUSED) pos_j = a.positions[j];
    const int bt_v = tid < a.maxb ? btj[tid] : 0;
    ctx_j = clamp_ctx(a.ctx_lens[j], cap);
    if constexpr (FUSED) {
      // Fused RoPE + KV append: the new token's position, slot and k / v rows
      // and this wave's query rows are fetched with the block ids, the
      // cos / sin rows as soon as the position is known.  The rotations, the
      // slot stores and an LDS copy of the new k / v row follow once the first
      // tile's loads are issued (tile loop below).  The stores are not waited
      // for: every K / V row the workgroup loads from the new slot is taken
      // from the LDS copy, which is what reading after the store returns.
      const int64_t sl = a.slots[j];
      slot_j = sl >= 0 && sl < a.num_slots ? sl : -1;
      rope_ok = pos_j >= 0 && pos_j < a.table_rows;
      const int64_t row = (int64_t)j * a.new_stride_b + (int64_t)g * HD + lr * 8;
      kx_new = *reinterpret_cast<const u32x4 *>(a.knew + row);
      vx_new = *reinterpret_cast<const u32x4 *>(a.vnew + row);
#pragma unroll
      for (int h = 0; h < G; ++h)
        q_pre[h] = *reinterpret_cast<const u32x4 *>(a.query + (int64_t)j * a.q_stride_b +
                                                    (int64_t)(head0 + h) * HD + lr * 8);
      if (rope_ok) cs_new = rope_fetch(a, pos_j, lr);
    }
    if constexpr (FUSED) {
      const int64_t phys = idf < 0 ? 0 : (idf > nb_hi ? nb_hi : idf);
      phys_f = phys;
      tv_f = tvf;
      const int64_t ss = (int64_t)a.Hkv * HD;
      const int64_t off = ((phys << bs_log2) + (tvf & (bs - 1))) * ss + (int64_t)g * HD + lr * 8;
#pragma unroll
      for (int s8 = 0; s8 < TPG; ++s8) kA[s8] = ld_nt(a.kcache + off + s8 * ss);
#pragma unroll
      for (int s8 = 0; s8 < TPG; ++s8) vA[s8] = ld_nt(a.vcache + off + s8 * ss);
    }
    if (tid < a.maxb) blk_lds[tid] = bt_v < 0 ? 0 : (bt_v > nb_hi ? nb_hi : bt_v);
    if (tid == 0) {
      pre[j] = 0;
      pre[j + 1] = (ctx_j + TILE - 1) / TILE;
    }
    lds_barrier();
    NT = pre[j + 1];
    je = 1;
    if (NT == 0) {
      for (int i = tid; i < G * HD; i += NTH)
        a.out[((int64_t)j * a.Hq + head0) * HD + i] = 0;
      if (FUSED && w == 0) {  // an empty sequence still gets its new k / v
        const u32x4 kx = rope_ok ? rope_apply<T>(kx_new, cs_new, lr) : kx_new;
        if (lg == 0 && slot_j >= 0) {
          const int64_t dst = (slot_j * a.Hkv + g) * HD + lr * 8;
          *reinterpret_cast<u32x4 *>(const_cast<uint16_t *>(a.kcache) + dst) = kx;
          *reinterpret_cast<u32x4 *>(const_cast<uint16_t *>(a.vcache) + dst) = vx_new;
        }
      }
      return;
    }
  } else {
    seg0 = SEG_TILES;
    NT = build_tile_prefix<NW>(a, pre, wave_tot, ctx_lds);
    je = partition_count(NT, a.J);
  }
  if (!a.per_seq && j == 0) {
    // rows of empty sequences are zeros; workgroup 0 of each head group
    // writes them for its heads
    const int h_lo = hgrp * hpg * G, h_hi = min(a.Hkv, (hgrp + 1) * hpg) * G;
    for (int b = 0; b < a.B; ++b)
      if (pre[b + 1] == pre[b])
        for (int i = tid; i < (h_hi - h_lo) * HD; i += NTH)
          a.out[((int64_t)b * a.Hq + h_lo) * HD + i] = 0;
    if (hgrp == 0)
      for (int b = tid; b < a.B; b += NTH) {
        int first = 0, n = 0;
        if (pre[b + 1] != pre[b]) {
          const int jf = owner_of(pre[b] + seg0, NT, je);
          first = jf + b;
          n = owner_of(pre[b + 1] - 1, NT, je) - jf + 1;
        }
        *reinterpret_cast<int2 *>(a.ws_meta + 2 * b) = int2{first, n};
      }
  }
  if (!a.per_seq && j >= je) return;
  const int t_lo = a.per_seq ? 0 : range_start(j, NT, je);
  const int t_hi = a.per_seq ? NT : range_start(j + 1, NT, je);
  if (t_lo >= t_hi) return;

  // first sequence whose tiles reach past t_lo
  int b = j;
  if (!a.per_seq) {
    int lo = 0, hi = a.B;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (pre[mid + 1] <= t_lo) lo = mid + 1; else hi = mid;
    }
    b = lo;
  }

  const int64_t slot_stride = (int64_t)a.Hkv * HD;  // elements between slots
  const uint16_t *kbase = a.kcache + (int64_t)g * HD;
  const uint16_t *vbase = a.vcache + (int64_t)g * HD;

  for (; b < a.B && pre[b] < t_hi; ++b) {
    const int r0 = pre[b] + seg0;  // first real tile of b in the split space
    if (pre[b + 1] == pre[b] || max(t_lo, r0) >= min(t_hi, pre[b + 1])) continue;
    const int ctx = a.per_seq ? ctx_j : ctx_lds[b];
    const int seg_lo = max(t_lo, r0) - r0;             // tile index in b
    const int seg_hi = min(t_hi, pre[b + 1]) - r0;
    const int tok_lo = seg_lo * TILE;
    const int tok_end = min(seg_hi * TILE, ctx);
    const int j_first = owner_of(r0, NT, je);
    const int nparts = owner_of(pre[b + 1] - 1, NT, je) - j_first + 1;

    // This lane's slice of each query head: dims 8 lr .. 8 lr + 7 as packed
    // 16-bit pairs -- the same dims the lane loads from every K and V row.
    u32x4 qv[G];
#pragma unroll
    for (int h = 0; h < G; ++h)
      qv[h] = FUSED ? q_pre[h]  // fetched in the prologue, rotated in the tile loop
                     : active ? *reinterpret_cast<const u32x4 *>(
                                    a.query + (int64_t)b * a.q_stride_b + (int64_t)(head0 + h) * HD + lr * 8)
                              : u32x4{0, 0, 0, 0};

    // m_run: running max of the raw scores (uniform over the wave);
    // l_grp: softmax denominator of this lane group's tokens;
    // acc:   unnormalised output, dims 8 lr .. 8 lr + 7, this group's tokens.
    float m_run[G], l_grp[G], acc[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      m_run[h] = -INFINITY;
      l_grp[h] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
    }
    const float c = a.scale_log2;

    const int32_t *bt = a.btab + (int64_t)b * a.maxb;
    // Sub-ranges of the segment whose block ids fit in LDS (one for every
    // workload that fits MAX_IDS blocks per workgroup).
    const int sub_tokens = max(TILE, ((MAX_IDS - 1) << bs_log2) / TILE * TILE);
    for (int s_lo = tok_lo; s_lo < tok_end; s_lo += sub_tokens) {
      const int t_end = min(s_lo + sub_tokens, tok_end);
      // ids[blk - first_blk]: physical block of logical block blk of b (the
      // per-sequence mode staged the whole row at the start)
      const int first_blk = a.per_seq ? 0 : s_lo >> bs_log2;
      const int ntile = (t_end - s_lo + TILE - 1) / TILE;

      // ---- loads of one tile: lane group lg owns tokens t0 + TPG lg .. + TPG - 1
      // (one block, since bs >= 8); each K and V row is one 256-byte run read by
      // 16 lanes x 16 bytes ----
      auto load_rows = [&](int phys, int tv, u32x4 (&kk)[TPG], u32x4 (&vv)[TPG]) {
        // the token's slot in the pool: below 2^32 (checked on the host), so
        // one 32 x 32 -> 64-bit multiply-add gives the element offset
        const uint32_t slot = ((uint32_t)phys << bs_log2) + (uint32_t)(tv & (bs - 1));
        const int64_t off = (int64_t)((uint64_t)slot * (uint32_t)slot_stride) + lr * 8;
#pragma unroll
        for (int s8 = 0; s8 < TPG; ++s8) kk[s8] = ld_nt(kbase + off + s8 * slot_stride);
#pragma unroll
        for (int s8 = 0; s8 < TPG; ++s8) vv[s8] = ld_nt(vbase + off + s8 * slot_stride);
      };
      // Fused append: the row (0 .. TPG - 1) of the lane group's rows tv ..
      // tv + TPG - 1 of physical block phys that is the new token's slot, or
      // -1 (the rows lie in one block: bs >= TPG and TPG | tv).  Found when
      // the tile is loaded, so the tile's compute only tests it.
      auto patch_row = [&](int64_t phys, int tv) {
        if (!FUSED || slot_j < 0 || phys != (slot_j >> bs_log2)) return -1;
        const int dd = (int)(slot_j & (bs - 1)) - (tv & (bs - 1));
        return dd >= 0 && dd < TPG ? dd : -1;
      };
      auto load_tile = [&](int t0, u32x4 (&kk)[TPG], u32x4 (&vv)[TPG], int &sub) {
        int tv = t0 + TPG * lg;
        tv = tv < t_end ? tv : t0;
        const int phys = blk_lds[(tv >> bs_log2) - first_blk];
        load_rows(phys, tv, kk, vv);
        sub = patch_row(phys, tv);
      };
      int k = rlane;
      if (!a.per_seq) {
        const int nblk = ((t_end - 1) >> bs_log2) - first_blk + 1;
        lds_barrier();  // previous users of blk_lds are done
        // The wave's first tile does not wait for the staging: each lane
        // group reads its block id straight from the table row, issued before
        // the segment's ids (loads return in order), and its K / V loads leave
        // before the staging's LDS writes and barrier.
        const int t0f = k < ntile ? s_lo + TILE * k : s_lo;
        int tv0 = t0f + TPG * lg;
        tv0 = tv0 < t_end ? tv0 : t0f;
        const int id0 = bt[tv0 >> bs_log2];
        const int st0 = bt[first_blk + (tid < nblk ? tid : nblk - 1)];
        if (active && k < ntile) load_rows(id0 < 0 ? 0 : (id0 > nb_hi ? nb_hi : id0), tv0, kA, vA);
        if (tid < nblk) blk_lds[tid] = st0 < 0 ? 0 : (st0 > nb_hi ? nb_hi : st0);
        for (int i = tid + NTH; i < nblk; i += NTH) {
          const int v = bt[first_blk + i];
          blk_lds[i] = v < 0 ? 0 : (v > nb_hi ? nb_hi : v);
        }
        lds_barrier();
      }
      if (!active) continue;
      // ---- compute of one tile, in two parts: scores and softmax (p packed
      // into pp), then P V ----
      using Pk = uint32_t[TPG / 2][G];
      auto tile_scores = [&](int t0, u32x4 (&kk)[TPG], Pk &pp) {
        // The score and softmax phase issues at raised wave priority, so the
        // wave that reaches it (and then the next tile's loads) goes first on
        // a SIMD shared with another wave: engine shape 9.81 -> 9.62 us, cfg2
        // -0.7 %, cfg4 -0.2 % (bit-identical).
        __builtin_amdgcn_s_setprio(1);
        const int tv = t0 + TPG * lg;
        // the tile reaches the end of the range (wave-uniform): only such a
        // tile masks tokens
        const bool tail = t0 + TILE > t_end;
        // scores: 4 v_dot2 over the lane's 8 dims, then a 16-lane DPP sum;
        // every lane of a group ends with the scores of the group's 8 tokens
        float sc[TPG][G];
#pragma unroll
        for (int s8 = 0; s8 < TPG; ++s8)
#pragma unroll
          for (int h = 0; h < G; ++h) {
            float d = 0.f;
#pragma unroll
            for (int k = 0; k < 4; ++k)
              // (explicit conversions: bit_cast of an ext-vector element picks
              // element 0 in this compiler)
              d = T::dot2((uint32_t)kk[s8][k], (uint32_t)qv[h][k], d);
            sc[s8][h] = d;
          }
        // the 16-lane sums (row16_sum), one DPP stage at a time across all
        // TPG G values: the chains interleave instead of waiting out each
        // other's DPP read-after-write hazards
        row16_sum_stage<0xB1>(sc);
        row16_sum_stage<0x4E>(sc);
        row16_sum_stage<0x141>(sc);
        row16_sum_stage<0x140>(sc);
        if (tail) {
#pragma unroll
          for (int s8 = 0; s8 < TPG; ++s8)
#pragma unroll
            for (int h = 0; h < G; ++h) sc[s8][h] = tv + s8 < t_end ? sc[s8][h] : -INFINITY;
        }
        // online softmax in base 2: p = exp2(s c - m c)
        float alpha[G];
        bool rescale = false;
#pragma unroll
        for (int h = 0; h < G; ++h) {
          float mx = sc[0][h];
#pragma unroll
          for (int s8 = 1; s8 < TPG; ++s8) mx = max_nq(mx, sc[s8][h]);
          mx = xor32_max(xor16_max(mx));
          mx = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, mx)));
          const float mn = max_nq(m_run[h], mx);
          alpha[h] = fast_exp2((m_run[h] - mn) * c);
          rescale |= mn != m_run[h];
          m_run[h] = mn;
        }
        // p packed in the element type for P V (v_dot2 over token pairs); the
        // row sum is taken from the same packed values (v_dot2 against 1.0),
        // so numerator and denominator use the one rounded p
        const uint32_t ones = T::pack_p(1.0f, 1.0f);
#pragma unroll
        for (int h = 0; h < G; ++h) {
          // (s - m) c rather than one FMA: exactly 0 at the max, so a single
          // token gets p = 1 and the output is v itself
          float ps = 0.f;
#pragma unroll
          for (int sp = 0; sp < TPG / 2; ++sp) {
            pp[sp][h] = T::pack_p(fast_exp2((sc[2 * sp][h] - m_run[h]) * c),
                                  fast_exp2((sc[2 * sp + 1][h] - m_run[h]) * c));
            ps = T::dot2(pp[sp][h], ones, ps);
          }
          l_grp[h] = l_grp[h] * alpha[h] + ps;
        }
        if (rescale) {
#pragma unroll
          for (int h = 0; h < G; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] *= alpha[h];
        }
        __builtin_amdgcn_s_setprio(0);
      };
      auto tile_pv = [&](int t0, u32x4 (&vv)[TPG], const Pk &pp) {
        const int tv = t0 + TPG * lg;
        const bool tail = t0 + TILE > t_end;
        // tokens past the end: zero their V rows (p is 0, V may be NaN garbage)
        if (tail) {
#pragma unroll
          for (int s8 = 0; s8 < TPG; ++s8)
            if (tv + s8 >= t_end) vv[s8] = u32x4{0, 0, 0, 0};
        }
        // acc += P V over token pairs with v_dot2
#pragma unroll
        for (int sp = 0; sp < TPG / 2; ++sp) {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            const uint32_t lo = __builtin_amdgcn_perm(vv[2 * sp + 1][k], vv[2 * sp][k], 0x05040100u);
            const uint32_t hi = __builtin_amdgcn_perm(vv[2 * sp + 1][k], vv[2 * sp][k], 0x07060302u);
#pragma unroll
            for (int h = 0; h < G; ++h) {
              acc[h][2 * k] = T::dot2(lo, pp[sp][h], acc[h][2 * k]);
              acc[h][2 * k + 1] = T::dot2(hi, pp[sp][h], acc[h][2 * k + 1]);
            }
          }
        }
      };
      // Fused append: the row the tile read from the new token's slot (sub,
      // found when the tile was loaded) is replaced by the LDS copy.
      // Wave-uniform branch: only the tile holding
      // the slot is patched, in place, every row by a select (a conditional
      // write of one row would become an indexed register write, which puts
      // the tile in scratch memory).
      auto patch_tile = [&](u32x4 (&kk)[TPG], u32x4 (&vv)[TPG], const int sub) {
        if (FUSED && __builtin_expect(__ballot(sub >= 0) != 0, 0)) {
          const u32x4 kn = knv_lds[lr], vn = knv_lds[16 + lr];
#pragma unroll
          for (int s8 = 0; s8 < TPG; ++s8) {
            const bool hit = s8 == sub;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              kk[s8][e] = hit ? kn[e] : kk[s8][e];
              vv[s8][e] = hit ? vn[e] : vv[s8][e];
            }
          }
        }
      };

      // ---- tile loop: the next tile's loads leave once the current tile's
      // scores are done, and land while its P V runs (one query head per
      // wave: the tiles alternate between two register sets) ----
      int subA = -1;  // patch row of the tile in kA / vA
      if (!FUSED && a.per_seq && k < ntile) load_tile(s_lo + TILE * k, kA, vA, subA);
      if constexpr (FUSED) {
        // (per-sequence mode: every wave of the workgroup is active and
        // reaches this barrier)  RoPE of the query rows and, by wave 0, of the
        // new k (same rounding as rope_inplace); wave 0 writes the new k / v
        // to the slot and to LDS.
        if (rope_ok) {
#pragma unroll
          for (int h = 0; h < G; ++h) qv[h] = rope_apply<T>(qv[h], cs_new, lr);
        }
        if (w == 0) {
          const u32x4 kx = rope_ok ? rope_apply<T>(kx_new, cs_new, lr) : kx_new;
          if (lg == 0) {
            knv_lds[lr] = kx;
            knv_lds[16 + lr] = vx_new;
            if (slot_j >= 0) {
              const int64_t dst = (slot_j * a.Hkv + g) * HD + lr * 8;
              *reinterpret_cast<u32x4 *>(const_cast<uint16_t *>(a.kcache) + dst) = kx;
              *reinterpret_cast<u32x4 *>(const_cast<uint16_t *>(a.vcache) + dst) = vx_new;
            }
          }
        }
        lds_barrier();
      }
      if constexpr (FUSED) subA = patch_row(phys_f, tv_f);
      Pk pp;
      if constexpr (G == 1) {
        u32x4 kB[TPG], vB[TPG];
        int subB = -1;
        while (k < ntile) {
          patch_tile(kA, vA, subA);
          tile_scores(s_lo + TILE * k, kA, pp);
          const int kn = k + wph;
          if (kn < ntile) load_tile(s_lo + TILE * kn, kB, vB, subB);
          tile_pv(s_lo + TILE * k, vA, pp);
          if (kn >= ntile) break;
          patch_tile(kB, vB, subB);
          tile_scores(s_lo + TILE * kn, kB, pp);
          k = kn + wph;
          if (k < ntile) load_tile(s_lo + TILE * k, kA, vA, subA);
          tile_pv(s_lo + TILE * kn, vB, pp);
        }
      } else {
        // (more query heads per wave: one register set measured faster; the
        // compiler keeps the tile's V rows in copies while the next loads land)
        while (k < ntile) {
          patch_tile(kA, vA, subA);
          tile_scores(s_lo + TILE * k, kA, pp);
          tile_pv(s_lo + TILE * k, vA, pp);
          k += wph;
          if (k < ntile) load_tile(s_lo + TILE * k, kA, vA, subA);
        }
      }
    }

    // ---- per-wave reduction over the four lane groups ----
    // (one exchange stage at a time across all values, so the exchanges of
    // different values interleave)
    float l_tot[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      l_tot[h] = xor16_add(l_grp[h]);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] = xor16_add(acc[h][e]);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      l_tot[h] = xor32_add(l_tot[h]);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] = xor32_add(acc[h][e]);
    }
    const int64_t row0 = (int64_t)b * a.Hq + head0;
    const int slot = j + b;  // this piece's partial slot (compact layout)
    if (wph == 1) {
      // the wave owns its kv head: write the final rows or this segment's
      // partial state directly (lanes 0-15 hold dims 8 lr .. 8 lr + 7)
      if (active && lg == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
          if (nparts == 1) {
            const float inv = 1.0f / l_tot[h];
            u32x4 o;
#pragma unroll
            for (int k = 0; k < 4; ++k)
              o[k] = pack2<T>(acc[h][2 * k] * inv, acc[h][2 * k + 1] * inv);
            *reinterpret_cast<u32x4 *>(a.out + (row0 + h) * HD + lr * 8) = o;
          } else {
            const int64_t pr = (int64_t)(head0 + h) * a.S + slot;
            float *dst = a.ws_acc + pr * HD + lr * 8;
            *reinterpret_cast<floatx4 *>(dst) =
                floatx4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
            *reinterpret_cast<floatx4 *>(dst + 4) =
                floatx4{acc[h][4], acc[h][5], acc[h][6], acc[h][7]};
            if (lr == 0) {
              a.ws_ml[pr * 2] = m_run[h] * c;  // base-2 units
              a.ws_ml[pr * 2 + 1] = l_tot[h];
            }
          }
        }
      }
      continue;
    }
    // several waves share a kv head: merge their states through LDS
    lds_barrier();  // previous segment's readers of red_* are done
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
        red_m[w][h] = m_run[h] * c;  // base-2 units
        red_l[w][h] = l_tot[h];
      }
    }
    lds_barrier();
    const int nheads = min(hpg, a.Hkv - hgrp * hpg);
    for (int idx = tid; idx < nheads * G * HD; idx += NTH) {
      const int hh = idx / (G * HD), rem = idx - hh * G * HD;
      const int h = rem / HD, d = rem - h * HD;
      float M = -INFINITY;
      for (int r = 0; r < wph; ++r) M = fmaxf(M, red_m[hh + r * hpg][h]);
      float L = 0.f, A = 0.f;
      for (int r = 0; r < wph; ++r) {
        const float sc = fast_exp2(red_m[hh + r * hpg][h] - M);
        L += red_l[hh + r * hpg][h] * sc;
        A += red_acc[hh + r * hpg][h][d] * sc;
      }
      const int hidx = (hgrp * hpg + hh) * gq + gsub * G + h;
      const int64_t row = (int64_t)b * a.Hq + hidx;
      if (nparts == 1) {
        a.out[row * HD + d] = T::from_float(A / L);
      } else {
        const int64_t pr = (int64_t)hidx * a.S + slot;
        a.ws_acc[pr * HD + d] = A;
        if (d == 0) {
          a.ws_ml[pr * 2] = M;
          a.ws_ml[pr * 2 + 1] = L;
        }
      }
    }
  }
}

// Log-sum-exp merge of split-K partials: one 128-lane workgroup per
// (query head, sequence); lane d owns output dim d.  Parts are merged 128 at
// a time: lane i loads part i's (m, l), the block max rescales them into LDS
// weights, and every lane then streams its dim of the partial outputs with
// independent (unrolled) loads.
template <class T>
__global__ __launch_bounds__(HD) void paged_decode_merge_kernel(DecodeArgs a) {
  const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
  const int64_t row = (int64_t)b * a.Hq + h;
  const int2 meta = *reinterpret_cast<const int2 *>(a.ws_meta + 2 * b);
  const int n = __builtin_amdgcn_readfirstlane(meta.y);
  if (n <= 1) return;
  const int first = __builtin_amdgcn_readfirstlane(meta.x);
  const float *ml = a.ws_ml + ((int64_t)h * a.S + first) * 2;
  const float *ac = a.ws_acc + ((int64_t)h * a.S + first) * HD + d;
  // The first HD parts' (m, l) and this lane's dim of the first SPEC parts'
  // partial outputs are loaded together (one memory round trip).
  constexpr int SPEC = 16;
  const float2 ml0 = d < n ? *reinterpret_cast<const float2 *>(ml + 2 * d) : float2{0.f, 0.f};
  float v0[SPEC];
#pragma unroll
  for (int k = 0; k < SPEC; ++k) v0[k] = k < n ? ac[(int64_t)k * HD] : 0.f;
  __shared__ float w_lds[HD], wl_lds[HD], mx_lds[2];
  float M = -INFINITY, L = 0.f, A = 0.f;
  for (int c0 = 0; c0 < n; c0 += HD) {
    const int cn = min(HD, n - c0);
    float mi = -INFINITY, li = 0.f;
    if (d < cn) {
      if (c0 == 0) {
        mi = ml0.x;
        li = ml0.y;
      } else {
        mi = ml[2 * (c0 + d)];
        li = ml[2 * (c0 + d) + 1];
      }
    }
    const float wm = wave_max(mi);
    if ((d & 63) == 0) mx_lds[d >> 6] = wm;
    lds_barrier();
    const float m_new = fmaxf(M, fmaxf(mx_lds[0], mx_lds[1]));
    const float wi = d < cn ? fast_exp2(mi - m_new) : 0.f;
    w_lds[d] = wi;
    wl_lds[d] = wi * li;
    lds_barrier();
    const float sc = fast_exp2(M - m_new);  // 0 on the first pass
    A *= sc;
    L *= sc;
    int i = 0;
    if (c0 == 0) {  // the prefetched parts (selects, not products: unused slots may hold NaN)
#pragma unroll
      for (int k = 0; k < SPEC; ++k)
        if (k < cn) {
          A += w_lds[k] * v0[k];
          L += wl_lds[k];
        }
      i = min(SPEC, cn);
    }
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
    lds_barrier();
  }
  a.out[row * HD + d] = T::from_float(A / L);
}

struct DecodeLayout {
  int J, S, hpg, wph, groups;
  size_t ml_off, acc_off, meta_off, total;
};

// S = J + B part slots per query head (compact layout: piece of sequence b in
// workgroup j at slot j + b), then two ints per sequence (first slot, parts).
static DecodeLayout decode_layout(int batch, int num_heads, int num_kv_heads) {
  DecodeLayout L{};
  L.hpg = num_kv_heads < DEC_NW ? num_kv_heads : DEC_NW;
  L.wph = DEC_NW / L.hpg;
  L.groups = (num_kv_heads + L.hpg - 1) / L.hpg;
  int J = cu_count() / L.groups;
  L.J = J < 1 ? 1 : (J > 512 ? 512 : J);
  L.S = L.J + batch;
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  const size_t rows = (size_t)num_heads * L.S;
  L.ml_off = 0;
  L.acc_off = up(rows * 2 * sizeof(float));
  L.meta_off = up(L.acc_off + rows * HD * sizeof(float));
  L.total = L.meta_off + up((size_t)batch * 2 * sizeof(int));
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
  // short contexts run the per-sequence mode, which needs no workspace
  if ((int64_t)max_blocks_per_seq * block_size <= PER_SEQ_MAX_TOKENS) return 0;
  return decode_layout(batch, num_heads, num_kv_heads).total;
}

namespace {
struct FusedRope {  // fused RoPE + KV append operands (null knew: off)
  const void *knew = nullptr, *vnew = nullptr;
  int64_t q_stride_b = 0, new_stride_b = 0;
  const float *cos = nullptr, *sin = nullptr;
  const int32_t *positions = nullptr, *slots = nullptr;
  int64_t table_rows = 0;
};

int decode_impl(int dtype, const void *query, const void *key_cache, const void *value_cache,
                const int32_t *block_tables, const int32_t *context_lens, void *output, int batch,
                int num_heads, int num_kv_heads, int head_dim, int max_blocks_per_seq,
                int block_size, int64_t num_blocks, float scale, void *workspace,
                size_t workspace_bytes, void *stream, const FusedRope &fr) {
  clear_error();
  MCE_REQUIRE(dtype == MCE_F16 || dtype == MCE_BF16,
              "mce_paged_attention_decode: unknown dtype %d", dtype);
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
  if (batch > MAX_BATCH)
    return set_error(MCE_ERR_UNSUPPORTED,
                     "mce_paged_attention_decode: batch %d > %d unsupported", batch, MAX_BATCH);
  MCE_REQUIRE(is_pow2(block_size) && block_size >= MIN_BS && block_size <= 256,
              "mce_paged_attention_decode: block_size must be a power of two in [8, 256] (got %d)",
              block_size);
  MCE_REQUIRE(max_blocks_per_seq >= 1, "mce_paged_attention_decode: max_blocks_per_seq must be >= 1");
  MCE_REQUIRE(num_blocks >= 1, "mce_paged_attention_decode: empty KV pool");
  MCE_REQUIRE(num_blocks <= ((int64_t)1 << 32) / block_size,
              "mce_paged_attention_decode: KV pool above 2^32 token slots");
  MCE_REQUIRE((int64_t)max_blocks_per_seq * block_size <= ((int64_t)1 << 26),
              "mce_paged_attention_decode: context capacity above 2^26 tokens");
  if (batch == 0) return MCE_OK;
  MCE_REQUIRE(query && key_cache && value_cache && block_tables &&
                  context_lens && output,
              "mce_paged_attention_decode: null pointer");
  MCE_REQUIRE(aligned16(query) && aligned16(key_cache) &&
                  aligned16(value_cache),
              "mce_paged_attention_decode: query and caches must be 16-byte aligned");
  // all sequences' tiles per kv head must fit an int
  MCE_REQUIRE((int64_t)batch * ((int64_t)max_blocks_per_seq * block_size / TILE + 1) <
                  ((int64_t)1 << 30),
              "mce_paged_attention_decode: batch x context too large");
  const DecodeLayout Lay = decode_layout(batch, num_heads, num_kv_heads);
  const bool per_seq = (int64_t)max_blocks_per_seq * block_size <= PER_SEQ_MAX_TOKENS;
  if (!per_seq && (workspace == nullptr || workspace_bytes < Lay.total ||
                   (reinterpret_cast<uintptr_t>(workspace) & 255) != 0))
    return set_error(MCE_ERR_WORKSPACE,
                     "mce_paged_attention_decode: a 256-byte aligned workspace of %zu bytes "
                     "is required (%zu given)",
                     Lay.total, workspace_bytes);
  DecodeArgs a{};
  a.query = (const uint16_t *)query;
  a.q_stride_b = fr.knew ? fr.q_stride_b : (int64_t)num_heads * head_dim;
  a.knew = (const uint16_t *)fr.knew;
  a.vnew = (const uint16_t *)fr.vnew;
  a.new_stride_b = fr.new_stride_b;
  a.rope_cos = fr.cos;
  a.rope_sin = fr.sin;
  a.positions = fr.positions;
  a.slots = fr.slots;
  a.table_rows = fr.table_rows;
  a.num_slots = num_blocks * block_size;
  a.kcache = (const uint16_t *)key_cache;
  a.vcache = (const uint16_t *)value_cache;
  a.btab = block_tables;
  a.ctx_lens = context_lens;
  a.out = (uint16_t *)output;
  char *base = (char *)workspace;  // unused (may be null) in per-sequence mode
  a.ws_ml = per_seq ? nullptr : (float *)(base + Lay.ml_off);
  a.ws_acc = per_seq ? nullptr : (float *)(base + Lay.acc_off);
  a.ws_meta = per_seq ? nullptr : (int *)(base + Lay.meta_off);
  a.B = batch;
  a.Hq = num_heads;
  a.Hkv = num_kv_heads;
  a.maxb = max_blocks_per_seq;
  a.bs_log2 = ilog2(block_size);
  a.J = Lay.J;
  a.S = Lay.S;
  a.hpg = Lay.hpg;
  a.wph = Lay.wph;
  // Short contexts: one workgroup per (kv head, sequence) streams the whole
  // sequence (at most PER_SEQ_MAX_TOKENS x 512 bytes of K/V) and writes the
  // final rows, so the launch is one kernel with no partials.  Longer
  // contexts use the balanced split over the concatenated tile space.
  a.per_seq = per_seq ? 1 : 0;
  // Per-sequence mode on a grid that leaves CUs idle (few sequences x kv
  // heads): the query heads of a kv head are split over gsplit workgroups
  // (the largest divisor of G that still fits the CUs).  Each reads the same
  // K/V pages (the repeats come from L2 / the infinity cache) and does 1/gsplit
  // of the score and P V work, which is what bounds this mode.
  int gsplit = 1;
  if (per_seq) {
    a.hpg = 1;
    a.wph = DEC_NW;
    for (int d = G; d > 1; --d)
      if (G % d == 0 && (int64_t)batch * num_kv_heads * d <= cu_count()) {
        gsplit = d;
        break;
      }
  }
  const int Gw = G / gsplit;  // query heads per wave
  a.num_blocks = num_blocks;
  a.scale_log2 = scale * 1.4426950408889634f;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = per_seq ? dim3(num_kv_heads * gsplit, batch) : dim3(Lay.groups, Lay.J);
#define MCE_DEC_CASE(TT, GG)                                                   \
  case GG:                                                                     \
    if (a.knew)                                                                \
      paged_decode_kernel<TT, GG, DEC_NW, true><<<grid, NT_THREADS, 0, st>>>(a); \
    else                                                                       \
      paged_decode_kernel<TT, GG, DEC_NW, false><<<grid, NT_THREADS, 0, st>>>(a); \
    break;
#define MCE_DEC_LAUNCH(TT)                                                     \
  switch (Gw) {                                                                \
    MCE_DEC_CASE(TT, 1)                                                        \
    MCE_DEC_CASE(TT, 2)                                                        \
    MCE_DEC_CASE(TT, 3)                                                        \
    MCE_DEC_CASE(TT, 4)                                                        \
    MCE_DEC_CASE(TT, 5)                                                        \
    MCE_DEC_CASE(TT, 6)                                                        \
    MCE_DEC_CASE(TT, 7)                                                        \
    MCE_DEC_CASE(TT, 8)                                                        \
  }                                                                            \
  if (!per_seq) paged_decode_merge_kernel<TT><<<dim3(num_heads, batch), HD, 0, st>>>(a);
  if (dtype == MCE_F16) {
    MCE_DEC_LAUNCH(F16T)
  } else {
    MCE_DEC_LAUNCH(BF16T)
  }
#undef MCE_DEC_LAUNCH
#undef MCE_DEC_CASE
  return check_launch("mce_paged_attention_decode");
}
}  // namespace

extern "C" int mce_paged_attention_decode(
    int dtype, const void *query, const void *key_cache,
    const void *value_cache, const int32_t *block_tables,
    const int32_t *context_lens, void *output, int batch, int num_heads,
    int num_kv_heads, int head_dim, int max_blocks_per_seq, int block_size,
    int64_t num_blocks, float scale, void *workspace, size_t workspace_bytes,
    void *stream) {
  return decode_impl(dtype, query, key_cache, value_cache, block_tables, context_lens, output,
                     batch, num_heads, num_kv_heads, head_dim, max_blocks_per_seq, block_size,
                     num_blocks, scale, workspace, workspace_bytes, stream, FusedRope{});
}

// ---------------------------------------------------------------------------
// Allocation-free variant: the split-K partials live in a file-scope device
// array instead of a caller workspace.  Every GPU the library runs on holds
// its own copy (DECODE_SCRATCH_BYTES) until the process ends; its address on
// each device is fetched once, with that device current, by
// hipGetSymbolAddress, and only that address is handed to kernels (the
// array's name is a host-side stand-in in host code).  The partials need no
// initialisation (workgroup 0 writes the per-sequence part counts before the
// merge kernel reads them), so nothing is cleared between calls.  Calls that
// overlap on one GPU share the array and race.
constexpr size_t DECODE_SCRATCH_BYTES = MCE_DECODE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[DECODE_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[MAX_DEVICES] = {};

// Device address of `scratch` on the current device (looked up on the first
// call per device).
int scratch_address(void **out) {
  int dev = -1;
  const hipError_t ge = hipGetDevice(&dev);
  if (ge != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
    return set_error(MCE_ERR_LAUNCH, "mce_paged_attention_decode_noalloc: no current device (%s)",
                     hipGetErrorString(ge));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return set_error(MCE_ERR_LAUNCH,
                       "mce_paged_attention_decode_noalloc: hipGetSymbolAddress(scratch) failed "
                       "on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return MCE_OK;
}
}  // namespace

extern "C" int mce_paged_attention_decode_noalloc(
    int dtype, const void *query, const void *key_cache, const void *value_cache,
    const int32_t *block_tables, const int32_t *context_lens, void *output, int batch,
    int num_heads, int num_kv_heads, int head_dim, int max_blocks_per_seq, int block_size,
    int64_t num_blocks, float scale, void *stream) {
  clear_error();
  const size_t need = mce_paged_attention_decode_workspace_size(
      batch, num_heads, num_kv_heads, max_blocks_per_seq, block_size);
  if (need > DECODE_SCRATCH_BYTES)
    return set_error(MCE_ERR_UNSUPPORTED,
                     "mce_paged_attention_decode_noalloc: this shape needs %zu bytes of split-K "
                     "scratch, above the library's static %zu (use mce_paged_attention_decode "
                     "with a workspace)",
                     need, DECODE_SCRATCH_BYTES);
  void *ws = nullptr;
  if (need > 0) {
    const int rc = scratch_address(&ws);
    if (rc != MCE_OK) return rc;
  }
  return decode_impl(dtype, query, key_cache, value_cache, block_tables, context_lens, output,
                     batch, num_heads, num_kv_heads, head_dim, max_blocks_per_seq, block_size,
                     num_blocks, scale, ws, need > 0 ? DECODE_SCRATCH_BYTES : 0, stream,
                     FusedRope{});
}

extern "C" int mce_paged_attention_decode_rope(
    int dtype, const void *query, const void *key, const void *value, void *key_cache,
    void *value_cache, const float *cos_table, const float *sin_table, const int32_t *positions,
    const int32_t *slot_mapping, const int32_t *block_tables, const int32_t *context_lens,
    void *output, int batch, int num_heads, int num_kv_heads, int head_dim,
    int max_blocks_per_seq, int block_size, int64_t num_blocks, int64_t table_rows,
    int64_t q_stride, int64_t kv_stride, float scale, void *stream) {
  clear_error();
  if ((int64_t)max_blocks_per_seq * block_size > PER_SEQ_MAX_TOKENS)
    return set_error(MCE_ERR_UNSUPPORTED,
                     "mce_paged_attention_decode_rope: table capacity %lld tokens > %d (use "
                     "mce_rope_kv_store + mce_paged_attention_decode)",
                     (long long)max_blocks_per_seq * block_size, PER_SEQ_MAX_TOKENS);
  MCE_REQUIRE(batch == 0 || (key && value && cos_table && sin_table && positions && slot_mapping),
              "mce_paged_attention_decode_rope: null pointer");
  MCE_REQUIRE(table_rows >= 0, "mce_paged_attention_decode_rope: bad table_rows");
  MCE_REQUIRE(q_stride >= (int64_t)num_heads * head_dim && q_stride % 8 == 0 &&
                  kv_stride >= (int64_t)num_kv_heads * head_dim && kv_stride % 8 == 0,
              "mce_paged_attention_decode_rope: bad row strides");
  MCE_REQUIRE(batch == 0 || (aligned16(key) && aligned16(value) && aligned16(cos_table) &&
                             aligned16(sin_table)),
              "mce_paged_attention_decode_rope: k, v and the tables must be 16-byte aligned");
  FusedRope fr;
  fr.knew = key;
  fr.vnew = value;
  fr.q_stride_b = q_stride;
  fr.new_stride_b = kv_stride;
  fr.cos = cos_table;
  fr.sin = sin_table;
  fr.positions = positions;
  fr.slots = slot_mapping;
  fr.table_rows = table_rows;
  return decode_impl(dtype, query, key_cache, value_cache, block_tables, context_lens, output,
                     batch, num_heads, num_kv_heads, head_dim, max_blocks_per_seq, block_size,
                     num_blocks, scale, nullptr, 0, stream, fr);
}
