// Causal flash prefill attention for gfx950 (reference semantics:
// csrc/kernels/prefill_attention.cu:15-269, host wrapper :271-309).
//
// Rows: the G = Hq / Hkv query heads that share a kv head are packed into the
// M dimension.  For batch b and kv head g, row r = position * G + (query head
// - g G), so one workgroup's rows cover consecutive positions of all G heads
// and every K/V tile staged in LDS serves all of them (the reference stages
// K/V once per query head).
//
// Work items: a workgroup takes BM = 32 * NRB consecutive rows of one (b, g).
// Causal cost grows with the row index, so workgroups are numbered heaviest
// item first.  Small grids run two key streams per item (even / odd key
// tiles) merged through LDS at the end: 128-row items on 8-wave workgroups,
// or, when those would leave CUs idle, 64-row items on 4-wave workgroups, two
// per CU.
//
// Each wave owns 32 rows and uses v_mfma_f32_32x32x16_f16 throughout:
//   S^T[32 keys x 32 rows] = K . Q^T   (A = K from LDS, B = Q^T in registers)
//     -> lane l holds the scores of row (l % 32) for 16 of the 32 keys, so the
//        row softmax is in-lane plus one exchange with lane l ^ 32.
//   O^T[128 dims x 32 rows] += V^T . P^T (A = V^T from LDS, B = P^T straight
//     from the S^T registers, converted to f16): lane l again holds row
//     (l % 32), so the online-softmax rescale is a per-lane multiply.
// The k-index permutation used for P^T (keys 8(v/4) + 4(l/32) + v%4 of the
// S^T output layout) is mirrored by the V^T operand reads: V is staged
// row-major like K and read with the transposing ds_read_b64_tr_b16, two per
// fragment (keys 4(l/32) + 0..3 and 8 + 4(l/32) + 0..3 of a 16-key group), so
// no transpose runs on the VALU.  Tiles sit in LDS in 4-row blocks with
// permuted 16-byte chunks (layout below), filled by direct-to-LDS buffer
// loads.
//
// Software pipeline: the scores of key tile k+1 are computed in the same
// straight-line block as the softmax and P V of tile k, so the exp/convert
// VALU work of one tile runs while the matrix cores work on the other.  K and
// V^T are double-buffered in LDS (K one tile ahead of V) with one barrier per
// tile; the loads of a tile are issued one step before the barrier that
// publishes it.
//
// Softmax in the log2 domain: Q is pre-scaled by c = scale log2(e) when it is
// loaded, and each score accumulator starts at -m (the row's running max, in
// the same units), so the MFMA output is already the exp2 argument.  The
// running max is only raised (O, l and the pending scores shifted) when a
// row's max grows by more than 2^8 in p units, so most tiles skip it and p
// stays below 256, well inside fp16.  Row sums are taken with v_dot2 over the
// same f16 P values that enter P V.
//
// Paged mode (chunked prefill): K / V rows come from the page pool through
// the block table (page byte offsets staged in LDS), the queries being each
// sequence's last S positions.  Its key split (small grids behind long cached
// prefixes) gives every query block up to nsplit workgroups over disjoint key
// ranges, each leaving an unnormalised partial state that
// prefill_merge_kernel combines by log-sum-exp.
#include "mce_common.h"

#include <algorithm>
#include <type_traits>

namespace mce {

constexpr int PF_HD = 128;
constexpr int PF_BN = 32;
// A 32-key K or V tile in LDS: 8 blocks of 4 key rows of 256 bytes (no row
// padding: one direct-to-LDS load instruction, 64 lanes x 16 bytes, fills one
// block), the blocks PF_BLK bytes apart so that consecutive blocks start 64
// bytes further along the banks.  Inside a block the 16-byte chunks of row a
// (0..3) are permuted: chunk c of a K row sits at position c ^ a, of a V row
// at c ^ 4a (whole 64-byte segments).  Then the K fragment reads (16 lanes:
// 16 keys x one chunk) and the transposing V reads (32 lanes: 4 rows x 64
// bytes) touch every bank once, and each lane's read offsets differ from one
// another by constants (immediate offsets).
constexpr int PF_BLK = 1088;         // bytes between 4-row blocks
constexpr int PF_TILE = 8 * PF_BLK;  // bytes of 32 keys of K or V (a tile half)
constexpr float RESCALE_TAU = 8.0f;  // log2 headroom before raising the max
// Buffer descriptor word 3 for raw (stride 0) dword loads on gfx9-family
// parts: data format 32, no swizzle, range-checked against num_records.
constexpr int BUF_RSRC_WORD3 = 0x00020000;

// v_mfma_f32_32x32x16 on raw 16-bit operands of the element type.
template <class T>
__device__ __forceinline__ floatx16 mfma32(u32x4 a, u32x4 b, floatx16 c) {
  if constexpr (T::code == MCE_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a),
                                                  __builtin_bit_cast(half8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

// Buffer load of 16 bytes per lane straight into LDS: lane l's bytes land at
// LDS address m0 + 16 l (m0 wave-uniform).  Written as inline asm rather than
// the builtin: the compiler orders the builtin's LDS write before every later
// read of the same LDS array with a vmcnt wait, which would stall the step's
// fragment reads (of the other buffer) until the load landed.  The waits the
// kernel needs are explicit (s_waitcnt vmcnt before the publishing barrier);
// loads the compiler does not see only make its own vmcnt waits stricter.
// The asm also carries the wait state that gfx9-family parts need between a
// scalar write of M0 (which the constraint produces just before it) and an
// LDS-DMA load: the compiler inserts it before the builtin but cannot insert
// it into inline asm.  (The scalar offset must come from scalar code or a
// constant: a v_readfirstlane result would need five more wait states.)
__device__ __forceinline__ void buffer_load_lds16(i32x4 rsrc, int voff, int soff, unsigned m0) {
  asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" : : "v"(voff), "s"(rsrc),
               "s"(soff), "{m0}"(m0));
}

// Raw buffer descriptor (stride 0, range-checked against `bytes`).
__device__ inline i32x4 buffer_rsrc(const void *base, int bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  return i32x4{(int)(uint32_t)p, (int)(uint32_t)(p >> 32) & 0xffff, bytes, BUF_RSRC_WORD3};
}

// ds_read_b64_tr_b16: within each 16-lane group, lane s supplies the address
// of 4 consecutive 16-bit values (row s / 4, columns 4 (s % 4) .. +3 of a
// 4 x 16 block) and lane d receives column d of the block's 4 rows.
__device__ __forceinline__ u32x2 ds_read_tr16(const uint16_t *p) {
  return __builtin_bit_cast(
      u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)p));
}


struct PrefillArgs {
  const uint16_t *q, *k, *v;
  uint16_t *out;
  int B, S, Hq, Hkv, G;  // S: query rows (positions) per sequence
  int n_items;
  float scale_log2;
  // paged mode: K / V rows from the page pool [num_blocks, bs, Hkv, 128]
  // through block_tables [B, maxb]; sequence b has ctx_b = context_lens[b]
  // keys and its S queries are its last S positions (ctx_b - S ..).
  const int32_t *block_tables, *context_lens;
  int maxb, bs_log2;
  int64_t num_blocks;
  uint32_t cache_bytes;  // bytes of one cache (< 2^31)
  // key split across workgroups (paged mode, SPLITK): every item's key tiles
  // are cut into nsplit parts, one workgroup each; part p of query row r
  // leaves its output ws_o[p][r][128] and (max, sum) ws_ml[p][r] (log2
  // units; max -inf for a part without keys of that row) for the merge.  The
  // fp16 kernels store that output normalised by the part's sum, in fp16
  // (half the bytes); the bf16 kernels store it unnormalised in fp32 (a bf16
  // copy would round too coarsely).
  int nsplit;
  int64_t rows_all;  // B S Hq
  float *ws_o, *ws_ml;
};

constexpr int PF_MAX_BLOCKS = 8192;  // paged mode: block-table row staged in LDS
constexpr int PF_NRB_MERGE = 4;      // row blocks per item of the paged launches (PF_NRB)
constexpr int PF_MAX_SPLIT = 8;      // key parts per item (SPLITK)
// SPLITK: at least this many key tiles per part (a part's start-up, epilogue
// and partial-state traffic cost about as much as streaming 8 to 16 tiles)
constexpr int PF_MIN_PART_TILES = 16;

// Keys of sequence b in the paged mode (its context length clamped into
// [S, table capacity]).
__device__ inline int paged_key_count(const PrefillArgs &a, int b) {
  const int cap_keys = min(a.maxb << a.bs_log2, 1 << 30);
  return min(max(a.context_lens[b], a.S), cap_keys);
}
// SPLITK: parts of query block `item` (rows item BM .. of one (sequence, kv
// head)): its key tiles / PF_MIN_PART_TILES, at least 1 and at most nsplit.
// One part means the workgroup of part 0 writes the output itself.
__device__ inline int prefill_parts(const PrefillArgs &a, int key_S, int item, int BM) {
  const int p0 = key_S - a.S;
  const int n_ktiles = (p0 + min(a.S - 1, (item * BM + BM - 1) / a.G)) / PF_BN + 1;
  return max(1, min(a.nsplit, n_ktiles / PF_MIN_PART_TILES));
}

// NRB row blocks of 32 rows per workgroup and KSPLIT key streams: wave w owns
// row block w % NRB and key stream kh = w / NRB, which takes key tiles kh,
// kh + KSPLIT, kh + 2 KSPLIT, ...  With KSPLIT = 2 every SIMD runs two waves
// of the same rows and the longest serial chain (the causal diagonal item) is
// halved; the streams keep separate online-softmax states that are merged
// through LDS at the end.  KSPLIT = 1 suits grids with several workgroups
// per CU, where the co-resident workgroups already fill the SIMDs.
//
// PAGED: K / V come from the page pool (chunked prefill: the queries are the
// last S positions of each sequence and attend to all its cached keys); the
// contiguous mode is PAGED = false with ctx_b = S.
// SPLITK (paged, two key streams): the workgroup takes part `part` of its
// item's key tiles and writes that part's partial softmax state instead of
// the output; prefill_merge_kernel combines the parts.
//
// BN keys per tile (32 or 64): a tile is NH = BN / 32 halves of 8 blocks, and
// one iteration of a key stream handles a whole tile -- NH score chains, one
// row max, one barrier -- so a 64-key tile pays the step's dependent chain
// (barrier -> fragment reads -> scores -> max -> exp -> P V) once per 64 keys.
template <class T, int NRB, int KSPLIT, bool PAGED, bool SPLITK, int BN>
// Two waves per SIMD (at most 256 registers each): one 8-wave workgroup per
// CU, or two 4-wave workgroups.
__global__ __launch_bounds__(NRB * KSPLIT * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_causal_kernel(PrefillArgs a) {
  static_assert(!SPLITK || (PAGED && KSPLIT == 2), "key parts: paged mode, two key streams");
  static_assert(!SPLITK || BN == PF_BN, "key parts are counted in 32-key tiles");
  static_assert(BN == 32 || BN == 64, "32- or 64-key tiles");
  constexpr int NH = BN / 32;            // 32-key halves per tile
  constexpr int TILE = NH * PF_TILE;     // bytes of one K or V tile
  constexpr int BM = 32 * NRB;
  // blocks of every K and V tile each wave of a key stream stages
  constexpr int KP = 8 / NRB;
  static_assert(KP * NRB == 8, "whole tiles per key stream");
  // Epilogue (reuses the tile buffers): exchanged O halves and (m, l) of the
  // two key streams, then each wave's finished 32 rows x OUT_DIMS before the
  // row-contiguous stores (pitch OUT_DIMS + 8 halfs: 16-byte aligned rows).
  constexpr int OUT_DIMS = PF_HD / KSPLIT;  // dims of a row a wave finishes
  constexpr int YS_PITCH = OUT_DIMS + 8;
  constexpr int XCH_FLOATS = KSPLIT == 2 ? 2 * NRB * 32 * 64 : 0;
  constexpr int ML_FLOATS = KSPLIT == 2 ? 2 * NRB * 2 * 64 : 0;
  constexpr int EPI_HALFS = 2 * (XCH_FLOATS + ML_FLOATS) + NRB * KSPLIT * 32 * YS_PITCH;
  // [key stream][double buffer] K tiles, then V tiles, then (two key streams,
  // 8 waves) the item's Q rows (NRB 32-row groups in the K tile layout); the
  // epilogue reuses them all.  The other launches load Q straight into
  // registers: their LDS has to leave room for two workgroups per CU.
  constexpr bool Q_LDS = KSPLIT == 2 && NRB == 4;
  constexpr bool PRIO_A = KSPLIT == 2 && !Q_LDS;  // the small-grid launch
  constexpr int TILE_HALFS = (2 * KSPLIT * 2 * TILE + (Q_LDS ? NRB * PF_TILE : 0)) / 2;
  constexpr int LDS_HALFS = TILE_HALFS > EPI_HALFS ? TILE_HALFS : EPI_HALFS;
  __shared__ __attribute__((aligned(16))) uint16_t lds[LDS_HALFS];
  char *const Ks = reinterpret_cast<char *>(lds);
  char *const Vs = Ks + 2 * KSPLIT * TILE;
  char *const Qs = Vs + 2 * KSPLIT * TILE;

  // workgroup -> (slot, batch, kv head); kv head fastest so that the
  // workgroups of one kv head share an XCD (and its L2) when Hkv B == 8.
  const int id = blockIdx.x;
  const int g = id % a.Hkv;
  const int b = (id / a.Hkv) % a.B;
  const int rest = id / (a.Hkv * a.B);
  const int part = SPLITK ? rest % a.nsplit : 0;
  int tb = 0;  // first key tile of this workgroup's part (0 without SPLITK)
  const int G = a.G, S = a.S;
  // keys of this sequence and the position of its first query row
  const int key_S = PAGED ? paged_key_count(a, b) : S;
  const int p0 = key_S - S;
  // SPLITK: parts of this item (from its real key range); workgroups of
  // parts past them have nothing to do
  const int n_parts = SPLITK ? prefill_parts(a, key_S, a.n_items - 1 - rest / a.nsplit, BM) : 1;
  if (SPLITK && part >= n_parts) return;
  __shared__ int bt_lds[PAGED ? PF_MAX_BLOCKS : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rb = w % NRB, kh = w / NRB;
  const int hf = lane >> 5, r32 = lane & 31;
  char *const ks_h = Ks + kh * 2 * TILE;  // this stream's K tiles (2 buffers)
  char *const vs_h = Vs + kh * 2 * TILE;

  const int64_t q_row_stride = (int64_t)a.Hq * PF_HD;
  // this sequence's queries (rows of Hq heads, 256 bytes each; < 2^31 bytes)
  const i32x4 qrsrc = buffer_rsrc(a.q + (int64_t)b * S * q_row_stride, S * a.Hq * PF_HD * 2);
  const int kv_row = a.Hkv * PF_HD;  // elements between consecutive keys
  const uint16_t *kbase = PAGED ? a.k + (int64_t)g * PF_HD : a.k + ((int64_t)b * S * a.Hkv + g) * PF_HD;
  const uint16_t *vbase = PAGED ? a.v + (int64_t)g * PF_HD : a.v + ((int64_t)b * S * a.Hkv + g) * PF_HD;
  if constexpr (PAGED) {
    // byte offset in the pool of each of the sequence's pages (block ids
    // clamped into the pool), before any K / V load
    const int32_t *btr = a.block_tables + (int64_t)b * a.maxb;
    const int nb_hi = (int)min(a.num_blocks - 1, (int64_t)0x7fffffff);
    for (int i = tid; i < a.maxb; i += NRB * KSPLIT * 64) {
      const int v = btr[i];
      bt_lds[i] = ((v < 0 ? 0 : (v > nb_hi ? nb_hi : v)) << a.bs_log2) * kv_row * 2;
    }
    lds_barrier();
  }
  const float c = a.scale_log2;

  // Staging, straight from global memory into LDS (buffer loads with the LDS
  // destination, 16 bytes per lane): wave rb of key stream kh fills blocks
  // KP rb .. KP rb + KP - 1 of every 32-key half of every K and V tile of its
  // stream.  Lane l
  // fetches row a = l / 16 of the block, chunk (l % 16) ^ a of a K row or
  // (l % 16) ^ 4a of a V row, so that the instruction's 64 x 16 bytes land in
  // the permuted block layout; each 16-lane group reads one whole 256-byte
  // row.  No registers hold staged data and no LDS write instructions issue;
  // each wave waits for its own loads (vmcnt) before the barrier that
  // publishes the tile.
  // Unconditional buffer loads: the hardware range check of the descriptor
  // returns zeros for keys at or past the sequence end (the descriptor spans
  // this (batch, kv head)'s rows up to key S).
  // (paged: the descriptor spans the whole pool; keys past the sequence end
  // are clamped to its last key, which the causal mask hides)
  const int kv_bytes = PAGED ? (int)(a.cache_bytes - g * PF_HD * 2) : (S * kv_row - g * PF_HD) * 2;
  const i32x4 krsrc = buffer_rsrc(kbase, kv_bytes), vrsrc = buffer_rsrc(vbase, kv_bytes);
  const int la = lane >> 4, lp = lane & 15;
  const int ck = lp ^ la, cv = lp ^ (4 * la);  // chunk this lane fetches (K / V)
  // contiguous mode: byte offset of this lane's piece of block j inside a half
  int voff_k[KP], voff_v[KP];
#pragma unroll
  for (int j = 0; j < KP; ++j) {
    const int key = 4 * (KP * rb + j) + la;
    voff_k[j] = PAGED ? ck * 16 : (key * kv_row + ck * 8) * 2;
    voff_v[j] = PAGED ? cv * 16 : (key * kv_row + cv * 8) * 2;
  }
  // paged mode: byte offset in the pool of the row of key `key`
  const int bsm = (1 << a.bs_log2) - 1;
  auto page_row = [&](int key) {
    key = min(key, key_S - 1);
    return bt_lds[key >> a.bs_log2] + (key & bsm) * kv_row * 2;
  };
  // stream index u of this key stream <-> key tile KSPLIT u + kh
  // (wave-uniform, passed as the scalar offset of the buffer loads)
  auto tile_off = [&](int u) {
    return __builtin_amdgcn_readfirstlane((KSPLIT * u + kh) * BN * kv_row * 2);
  };
  const int half_bytes = PF_BN * kv_row * 2;  // between the halves of a tile
  // LDS address (m0) of this wave's first block in K / V buffer 0
  const unsigned lds0 = (unsigned)reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) char *)reinterpret_cast<char *>(lds));
  const unsigned k_m0 = __builtin_amdgcn_readfirstlane(lds0 + (unsigned)(ks_h - Ks) + KP * rb * PF_BLK);
  const unsigned v_m0 = __builtin_amdgcn_readfirstlane(lds0 + (unsigned)(vs_h - Ks) + KP * rb * PF_BLK);
  const unsigned q_m0 = __builtin_amdgcn_readfirstlane(lds0 + (unsigned)(Qs - Ks));
  // K and V tiles u of this stream into buffer u % 2.  The loads are issued
  // unconditionally, also the last iteration's (never read): skipping those
  // behind a branch computes the same outputs but measured no faster.
  auto stage_k = [&](int u) {
    const unsigned m0 = k_m0 + (u & 1) * TILE;
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
      if constexpr (PAGED) {
#pragma unroll
        for (int j = 0; j < KP; ++j)
          buffer_load_lds16(krsrc,
                            page_row((tb + KSPLIT * u + kh) * BN + 32 * hh + 4 * (KP * rb + j) + la) +
                                voff_k[j],
                            0, m0 + hh * PF_TILE + j * PF_BLK);
      } else {
        const int off = tile_off(u) + hh * half_bytes;
#pragma unroll
        for (int j = 0; j < KP; ++j)
          buffer_load_lds16(krsrc, voff_k[j], off, m0 + hh * PF_TILE + j * PF_BLK);
      }
    }
  };
  auto stage_v = [&](int u) {
    const unsigned m0 = v_m0 + (u & 1) * TILE;
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
      if constexpr (PAGED) {
#pragma unroll
        for (int j = 0; j < KP; ++j)
          buffer_load_lds16(vrsrc,
                            page_row((tb + KSPLIT * u + kh) * BN + 32 * hh + 4 * (KP * rb + j) + la) +
                                voff_v[j],
                            0, m0 + hh * PF_TILE + j * PF_BLK);
      } else {
        const int off = tile_off(u) + hh * half_bytes;
#pragma unroll
        for (int j = 0; j < KP; ++j)
          buffer_load_lds16(vrsrc, voff_v[j], off, m0 + hh * PF_TILE + j * PF_BLK);
      }
    }
  };
  // this wave's staging loads have landed in LDS (s_waitcnt vmcnt(0))
  auto staged = [] { __builtin_amdgcn_s_waitcnt(0x0F70); };
  // Fragment read offsets inside a 32-key half.  K (scores): lane (r32, hf)
  // reads chunk 2 i + hf of key r32, at 64 (i / 2) + kfo[i % 2].  V^T (P V):
  // lane 16 q + s of group q reads dims 32 dt + 16 (q & 1) + 4 (s & 3) .. + 3
  // of key rows 16 kk + 4 (q >> 1) + s / 4 and + 8, at vfo[dt] + (4 kk) PF_BLK
  // and + (4 kk + 2) PF_BLK.
  int kfo[2], vfo[4];
  {
    const int kb = r32 >> 2, ka = r32 & 3;
#pragma unroll
    for (int t = 0; t < 2; ++t) kfo[t] = kb * PF_BLK + ka * 256 + 16 * ((2 * t + hf) ^ ka);
    const int q4 = lane >> 4, s16 = lane & 15, va = s16 >> 2;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
      vfo[dt] = (q4 >> 1) * PF_BLK + va * 256 +
                16 * (4 * (dt ^ va) + 2 * (q4 & 1) + ((s16 >> 1) & 1)) + 8 * (s16 & 1);
  }

  const int rows_total = S * G;
  // Items of this workgroup.  Without the key split the launch has P
  // workgroups per (sequence, kv head), at most one per CU (two for the
  // 4-wave launch), and workgroup j takes item ranks j and 2 P - 1 - j (ranks
  // count from the heaviest item):
  // the lightest items run behind medium ones on the same CU instead of as a
  // second round of workgroups, which paid a start-up and a drain each.
  // (two-stream launches only: the one-stream launches have a workgroup per
  // item, several per CU, and the key split one per part)
  constexpr int MAX_MINE = KSPLIT == 2 && !SPLITK ? 2 : 1;
  const int P = MAX_MINE == 1 ? 1 : (int)(gridDim.x / (unsigned)(a.Hkv * a.B));
  const int n_mine = MAX_MINE == 2 && 2 * P - 1 - rest < a.n_items ? 2 : 1;
  for (int mi = 0; mi < MAX_MINE && mi < n_mine; ++mi) {
    const int item_rank = SPLITK ? rest / a.nsplit : (mi == 0 ? rest : 2 * P - 1 - rest);
    if (mi > 0) lds_barrier();  // every wave is done with the previous item's LDS
    const int item = a.n_items - 1 - item_rank;  // heaviest items first
    const int r_item = item * BM;
    const int r_wave = r_item + 32 * rb;
    const int row = r_wave + r32;                 // this lane's row
    const int qi = row / G;
    const int pos = p0 + qi;                      // its position among the keys
    const bool row_ok = row < rows_total;
    const int wave_min_pos = p0 + r_wave / G;
    const int item_max_pos = p0 + min(S - 1, (r_item + BM - 1) / G);
    const int n_ktiles = item_max_pos / BN + 1;  // key tiles of the item
    // SPLITK: this part's key tiles [tb, te)
    if constexpr (SPLITK) tb = (int)((int64_t)part * n_ktiles / n_parts);
    const int te = SPLITK ? (int)((int64_t)(part + 1) * n_ktiles / n_parts) : n_ktiles;
    // iterations per key stream, rounded up to even for the ping-pong unroll
    const int n_iter = ((te - tb + KSPLIT - 1) / KSPLIT + 1) / 2 * 2;
    // key tiles this wave's rows need (none for a block of padding rows)
    const int n_wtiles =
        r_wave < rows_total ? (p0 + min(S - 1, min(r_wave + 31, rows_total - 1) / G)) / BN + 1 : 0;
    // tiles [0, n_full) need no mask for this wave: every key <= its first
    // position and < key_S (SPLITK: and below the part's end, so that no key of
    // the next part is ever scored into this part's state)
    const int n_full = SPLITK ? min(min((wave_min_pos + 1) / BN, key_S / BN), te)
                              : min((wave_min_pos + 1) / BN, key_S / BN);
    // masked tiles: key offset limit + n0
    const int lim = (SPLITK ? min(min(pos, key_S - 1), te * BN - 1) : min(pos, key_S - 1)) - 4 * hf;

    // Q^T as MFMA B operand: lane supplies Q[pos, h][16 i + 8 hf + j], for fp16
    // pre-scaled by c (so the accumulators come out in log2 units); bf16 keeps
    // Q exact (its 8-bit mantissa would round c Q too coarsely) and scales the
    // scores instead (PRESCALED false).
    constexpr bool PRESCALED = T::code == MCE_F16;
    //
    // Q, K_0, K_1 and V_0 are fetched together (one memory round trip before
    // the first tile instead of one per dependent stage).  With two key
    // streams on 8 waves Q comes through LDS like K: whole 256-byte rows per
    // 16-lane group (the MFMA operand pattern straight from global memory, 32
    // rows x 32 bytes per load instruction, keeps the address path busy ~3.5x
    // longer), loaded once for both streams; wave w fills 4-row blocks
    // QB w .. QB w + QB - 1 of the item (rows past the end re-read the last
    // row and are zeroed below).
    u32x4 qreg[8];
    if constexpr (Q_LDS) {
      constexpr int QB = 8 / KSPLIT;
#pragma unroll
      for (int j = 0; j < QB; ++j) {
        const int bq = QB * w + j;
        const int qr = min(r_item + 4 * bq + la, rows_total - 1);
        const int qp = qr / G;
        const int qh = g * G + (qr - qp * G);
        buffer_load_lds16(qrsrc, (qp * a.Hq + qh) * PF_HD * 2 + ck * 16, 0,
                          q_m0 + (bq >> 3) * PF_TILE + (bq & 7) * PF_BLK);
      }
    } else {
      const int qh = g * G + (row - qi * G);
      const uint16_t *qp = a.q + ((int64_t)b * S + (row_ok ? qi : 0)) * q_row_stride +
                           (int64_t)(row_ok ? qh : 0) * PF_HD + 8 * hf;
#pragma unroll
      for (int i = 0; i < 8; ++i) qreg[i] = *reinterpret_cast<const u32x4 *>(qp + 16 * i);
    }
    stage_k(0);
    stage_k(1);
    stage_v(0);
    staged();
    lds_barrier();
    if constexpr (Q_LDS) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        qreg[i] = *reinterpret_cast<const u32x4 *>(Qs + rb * PF_TILE + kfo[i & 1] + 64 * (i >> 1));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const u32x4 x = row_ok ? qreg[i] : u32x4{0, 0, 0, 0};
      if constexpr (PRESCALED) {
        const half8 xh = __builtin_bit_cast(half8, x);
        half8 y;
#pragma unroll
        // x c rounded to fp16 (as an fma with a +0 addend, one v_fma_mix per
        // element instead of convert / multiply / convert / pack; only a -0
        // product becomes +0)
        for (int j = 0; j < 8; ++j) y[j] = (_Float16)__builtin_fmaf((float)xh[j], c, 0.0f);
        qreg[i] = __builtin_bit_cast(u32x4, y);
      } else {
        qreg[i] = x;
      }
    }

    // S^T of one tile (NH 32-key halves), accumulators starting at `init`.
    using Scores = floatx16[NH];
    auto scores = [&](const char *kt, float init, Scores &st) {
#pragma unroll
      for (int hh = 0; hh < NH; ++hh) {
#pragma unroll
        for (int e = 0; e < 16; ++e) st[hh][e] = init;
#pragma unroll
        for (int i = 0; i < 8; ++i)
          st[hh] = mfma32<T>(*reinterpret_cast<const u32x4 *>(kt + hh * PF_TILE + kfo[i & 1] + 64 * (i >> 1)),
                             qreg[i], st[hh]);
      }
    };

    // Online-softmax state of this lane's row: running max m_run (log2 units;
    // 0 until the row has seen an unmasked key), growth threshold thr (-inf
    // until then, so the first finite tile max sets m_run; RESCALE_TAU after),
    // l_i = this lane's half of the row sum, O^T in o.
    float m_run = 0.f, thr = -INFINITY, l_i = 0.f;
    floatx16 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int e = 0; e < 16; ++e) o[dt][e] = 0.f;
    Scores s_a, s_b;  // ping-pong: scores ready for exp / next accumulator
    // accumulator start of every tile's scores: -m_run (fp16, pre-scaled Q) or 0
    floatx16 acc0;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc0[e] = 0.f;
    const uint32_t ones = T::pack_p(1.0f, 1.0f);

    // Scores of key tile kt straight from the MFMA -> exp2 arguments: bf16
    // scales them here; tiles past the diagonal (or the sequence end) get -inf
    // on masked keys.
    auto prep = [&](Scores &s, const int kt) {
      if constexpr (!PRESCALED) {
#pragma unroll
        for (int hh = 0; hh < NH; ++hh)
#pragma unroll
          for (int e = 0; e < 16; ++e) s[hh][e] = __builtin_fmaf(s[hh][e], c, -m_run);
      }
      if (kt >= n_full) {
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) {
          const int l2 = lim - kt * BN - 32 * hh;
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (8 * (e >> 2) + (e & 3) > l2) s[hh][e] = -INFINITY;
        }
      }
    };
    // max over this lane's row (both 32-lane halves of the wave hold it)
    auto rowmax = [&](const Scores &s) {
      float mx = -INFINITY;
#pragma unroll
      for (int hh = 0; hh < NH; ++hh)
#pragma unroll
        for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[hh][e]);
      return fmaxf(mx, xor32_max(mx));
    };
    // Raise the running max of the rows whose tile max exceeds thr: O, l and
    // the ready scores move to the new max.  Rare after the first tile (growth
    // beyond 2^TAU in p units).
    auto rescale = [&](const float mx, Scores &s_ready) {
      const bool grow = mx > thr;
      const float d = grow ? mx : 0.f;
      const float alpha = thr > -INFINITY ? fast_exp2(-d) : 0.f;
      l_i *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[dt][e] *= alpha;
#pragma unroll
      for (int hh = 0; hh < NH; ++hh)
#pragma unroll
        for (int e = 0; e < 16; ++e) s_ready[hh][e] -= d;
      m_run += d;
      if constexpr (PRESCALED) {
#pragma unroll
        for (int e = 0; e < 16; ++e) acc0[e] = -m_run;
      }
      thr = grow ? RESCALE_TAU : thr;
    };

    // Prologue (per key stream): K_0, K_1 and V_0 staged above (indices are
    // stream indices u), K_0 scored (prepared in s_a).
    {
      scores(ks_h, 0.f, s_a);
      prep(s_a, tb + kh);
      const float mx = rowmax(s_a);
      if (__ballot(mx > thr) != 0) rescale(mx, s_a);
    }

    // Iteration u (key tile kt = KSPLIT u + kh), one straight-line block after
    // the barrier that publishes K_{u+1} and V_u:
    //   K_{u+2} / V_{u+1} are staged (direct-to-LDS loads, issued after the
    //      first score MFMA) into the buffers that iteration u - 1 finished
    //      reading; they have the rest of the iteration to land;
    //   A: scores of tile u + 1 (K in buffer (u+1)%2, accumulators starting at
    //      -m_run) on the matrix cores while the exp2 / convert / row-sum work
    //      of tile u runs on the VALU;
    //   B: P V of tile u (V^T in buffer u%2) while tile u + 1 is masked (DIAG)
    //      and max-reduced;
    // rows whose max grew are rescaled after the block.  The mask is applied
    // only by the DIAG form (tiles that reach the diagonal or the sequence end),
    // and waves past their last tile only stage (stage_only), so the three
    // loops below keep every step free of branches.  Barriers match by count:
    // every wave runs the same (even) number of iterations.  Staging is
    // unconditional; tiles past the end are zero-filled (or clamped) and land
    // in buffers nobody reads again.
    auto step = [&](const int u, Scores &s_cur, Scores &s_nxt, auto diag) {
      constexpr bool DIAG = decltype(diag)::value;
      staged();
      lds_barrier();
      // LLVM's built-in MFMA / LDS-read interleaving strategy for the step's
      // block (same instructions, another order): 1-2% faster at every shape
      // measured, with fewer registers.
      __builtin_amdgcn_iglp_opt(0);
      // Small-grid launch (two 4-wave workgroups per CU, so each SIMD runs
      // waves of two workgroups, not held in one phase by a common barrier):
      // the score phase issues at raised wave priority, back to normal for
      // P V.  B=1 S=128 / 256 / 512 in 20-call graphs 2 / 3 / 4 % faster; on
      // the 8-wave and one-stream launches it measured neutral to 2 % slower.
      if constexpr (PRIO_A) __builtin_amdgcn_s_setprio(1);
      const int kt = tb + KSPLIT * u + kh;  // key tile
      const char *kb = ks_h + ((u + 1) & 1) * TILE;
      const char *vb = vs_h + (u & 1) * TILE;
      // ---- A: the NH score chains of tile u + 1 on the matrix cores while
      // tile u's exp2 / convert / row-sum work runs on the VALU
#pragma unroll
      for (int hh = 0; hh < NH; ++hh) {
        u32x4 kf[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          kf[i] = *reinterpret_cast<const u32x4 *>(kb + hh * PF_TILE + kfo[i & 1] + 64 * (i >> 1));
        s_nxt[hh] = mfma32<T>(kf[0], qreg[0], acc0);
        // The staging loads leave once the first score MFMA is issued: the
        // fragment reads that feed the matrix cores go first after the
        // barrier (issued before them, the loads and their M0 writes delayed
        // the step's first MFMA; ~2.5 % of cfg3).
        if (hh == 0) {
          stage_k(u + 2);
          stage_v(u + 1);
        }
#pragma unroll
        for (int i = 1; i < 8; ++i) s_nxt[hh] = mfma32<T>(kf[i], qreg[i], s_nxt[hh]);
      }
      u32x4 pk[NH][2];
#pragma unroll
      for (int hh = 0; hh < NH; ++hh)
#pragma unroll
        for (int e2 = 0; e2 < 8; ++e2) {
          const float p0 = fast_exp2(s_cur[hh][2 * e2]);
          const float p1 = fast_exp2(s_cur[hh][2 * e2 + 1]);
          const uint32_t pp = T::pack_p(p0, p1);
          l_i = T::dot2(pp, ones, l_i);
          pk[hh][e2 >> 2][e2 & 3] = pp;
        }
      if constexpr (PRIO_A) __builtin_amdgcn_s_setprio(0);
      // ---- B: P V of tile u while tile u + 1 is masked and max-reduced
#pragma unroll
      for (int hh = 0; hh < NH; ++hh) {
        u32x4 vf[8];
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) {
            const char *vp = vb + hh * PF_TILE + vfo[dt];
            const u32x2 lo = ds_read_tr16(reinterpret_cast<const uint16_t *>(vp + 4 * kk * PF_BLK));
            const u32x2 hi = ds_read_tr16(reinterpret_cast<const uint16_t *>(vp + (4 * kk + 2) * PF_BLK));
            vf[dt * 2 + kk] = u32x4{lo[0], lo[1], hi[0], hi[1]};
          }
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) o[dt] = mfma32<T>(vf[dt * 2 + kk], pk[hh][kk], o[dt]);
      }
      if constexpr (!PRESCALED) {
#pragma unroll
        for (int hh = 0; hh < NH; ++hh)
#pragma unroll
          for (int e = 0; e < 16; ++e) s_nxt[hh][e] = __builtin_fmaf(s_nxt[hh][e], c, -m_run);
      }
      if constexpr (DIAG) {
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) {
          const int l2 = lim - (kt + KSPLIT) * BN - 32 * hh;
#pragma unroll
          for (int e = 0; e < 16; ++e)
            if (8 * (e >> 2) + (e & 3) > l2) s_nxt[hh][e] = -INFINITY;
        }
      }
      const float mx = rowmax(s_nxt);
      if (__builtin_expect(__ballot(mx > thr) != 0, 0)) rescale(mx, s_nxt);
    };
    auto stage_only = [&](const int u) {
      staged();
      lds_barrier();
      stage_k(u + 2);
      stage_v(u + 1);
    };
    // step u needs the mask from u_first on (its next tile KSPLIT (u+1) + kh
    // reaches n_full); tile KSPLIT u + kh is past this wave's rows from u_end on
    const int nf_rel = n_full - tb - kh, nw_rel = min(n_wtiles, te) - tb - kh;
    const int u_first = nf_rel <= KSPLIT ? 0 : (nf_rel + KSPLIT - 1) / KSPLIT - 1;
    const int u_end = nw_rel <= 0 ? 0 : (nw_rel + KSPLIT - 1) / KSPLIT;
    const int u1 = u_first & ~1;                      // <= u_end <= n_iter
    const int u2 = max(u1, min((u_end + 1) & ~1, n_iter));
    const std::integral_constant<bool, false> plain;
    const std::integral_constant<bool, true> diag;
    int u = 0;
    for (; u < u1; u += 2) {
      step(u, s_a, s_b, plain);
      step(u + 1, s_b, s_a, plain);
    }
    for (; u < u2; u += 2) {
      step(u, s_a, s_b, diag);
      step(u + 1, s_b, s_a, diag);
    }
    for (; u < n_iter; u += 2) {
      stage_only(u);
      stage_only(u + 1);
    }

    // ---- epilogue: merge the key streams (KSPLIT = 2), normalise, store.
    // Both streams finish rows: stream kh takes dims OUT_DIMS kh .. +OUT_DIMS-1
    // of its 32 rows and reads the partner stream's O for those dims, and its
    // (m, l), from LDS (16-byte lane-major records, conflict-free).  The
    // finished tile goes through LDS once more so that every store writes whole
    // rows: OUT_DIMS * 2 bytes of a row by consecutive lanes, 16 bytes each.
    staged();       // the last staging loads have landed (the epilogue reuses
    lds_barrier();  // the tile buffers); every wave is done with the K / V^T tiles
    float *const xo = reinterpret_cast<float *>(lds);  // [kh][rb][8][64 lanes][4]
    float *const xm = xo + XCH_FLOATS;                 // [kh][rb][2][64 lanes]
    uint16_t *const ys = reinterpret_cast<uint16_t *>(xm + ML_FLOATS) + w * 32 * YS_PITCH;
    float s_own, s_oth = 0.f;  // weights of this stream's and the partner's O, 1 / l included
    const floatx4 *xr = nullptr;
    if constexpr (KSPLIT == 2) {
      const float m_own = thr > -INFINITY ? m_run : -INFINITY;
      floatx4 *const xw = reinterpret_cast<floatx4 *>(xo) + (kh * NRB + rb) * 8 * 64 + lane;
#pragma unroll
      for (int gq = 0; gq < 8; ++gq) {
        // the partner's half: o[2 + gq / 4] for stream 0, o[gq / 4] for stream 1
        // (selects, not an index that depends on kh, keep o in registers)
        const floatx16 &ox = o[2 + (gq >> 2)], &oy = o[gq >> 2];
        const int e0 = (gq & 3) * 4;
        floatx4 x;
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = kh == 0 ? ox[e0 + j] : oy[e0 + j];
        xw[gq * 64] = x;
      }
      xm[((kh * NRB + rb) * 2 + 0) * 64 + lane] = m_own;
      xm[((kh * NRB + rb) * 2 + 1) * 64 + lane] = l_i;
      lds_barrier();
      const int ko = 1 - kh;
      const float m_oth = xm[((ko * NRB + rb) * 2 + 0) * 64 + lane];
      const float l_oth = xm[((ko * NRB + rb) * 2 + 1) * 64 + lane];
      // a state that never saw an unmasked key (m = -inf, l = 0, O = 0) gets
      // weight 0; stream 0 always sees key 0, so mm is finite on real rows
      const float mm = fmaxf(m_own, m_oth);
      // (a part may hold no key of a row in either stream: mm = -inf)
      const float mmz = SPLITK && mm == -INFINITY ? 0.f : mm;
      const float a_own = fast_exp2(m_own - mmz), a_oth = fast_exp2(m_oth - mmz);
      const float l_row = xor32_add(l_i * a_own + l_oth * a_oth);
      xr = reinterpret_cast<const floatx4 *>(xo) + (ko * NRB + rb) * 8 * 64 + lane;
      if (SPLITK && n_parts > 1) {
        // this part's state of the row: O unnormalised (dims OUT_DIMS kh ..),
        // relative to max mm, and the row sum; straight from the MFMA layout
        const int grow = r_wave + r32;
        if (grow < rows_total) {
          const int p = grow / G, hh = g * G + (grow - p * G);
          const int64_t pr = (int64_t)part * a.rows_all + ((int64_t)b * S + p) * a.Hq + hh;
          const int64_t off = pr * PF_HD + OUT_DIMS * kh + 4 * hf;
          constexpr bool NORM_F16 = T::code == MCE_F16;
          const float sc = NORM_F16 ? (l_row > 0.f ? 1.0f / l_row : 0.f) : 1.0f;
#pragma unroll
          for (int dd = 0; dd < OUT_DIMS / 32; ++dd)
#pragma unroll
            for (int e4 = 0; e4 < 4; ++e4) {
              const floatx4 x = xr[(dd * 4 + e4) * 64];
              floatx4 v;
#pragma unroll
              for (int j = 0; j < 4; ++j) {
                const int e = 4 * e4 + j;
                v[j] = ((kh == 0 ? o[dd][e] : o[2 + dd][e]) * a_own + x[j] * a_oth) * sc;
              }
              if constexpr (NORM_F16) {
                u32x2 h;
                h[0] = pack2<T>(v[0], v[1]);
                h[1] = pack2<T>(v[2], v[3]);
                *reinterpret_cast<u32x2 *>(reinterpret_cast<uint16_t *>(a.ws_o) + off + 32 * dd +
                                           8 * e4) = h;
              } else {
                *reinterpret_cast<floatx4 *>(a.ws_o + off + 32 * dd + 8 * e4) = v;
              }
            }
          if (kh == 0 && hf == 0)
            *reinterpret_cast<float2 *>(a.ws_ml + pr * 2) =
                float2{l_row > 0.f ? mm : -INFINITY, l_row};
        }
        return;
      }
      const float inv = 1.0f / l_row;
      s_own = a_own * inv;
      s_oth = a_oth * inv;
    } else {
      s_own = 1.0f / xor32_add(l_i);
    }
    // lane: row r32 of the wave, dims 32 dd + 8 e4 + 4 hf + 0..3 of its half
#pragma unroll
    for (int dd = 0; dd < OUT_DIMS / 32; ++dd)
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        floatx4 x = {0.f, 0.f, 0.f, 0.f};
        if constexpr (KSPLIT == 2) x = xr[(dd * 4 + e4) * 64];
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int e = 4 * e4 + j;
          const float own = KSPLIT == 2 ? (kh == 0 ? o[dd][e] : o[2 + dd][e]) : o[dd][e];
          v[j] = own * s_own + x[j] * s_oth;
        }
        u32x2 pr;
        pr[0] = pack2<T>(v[0], v[1]);
        pr[1] = pack2<T>(v[2], v[3]);
        *reinterpret_cast<u32x2 *>(&ys[r32 * YS_PITCH + dd * 32 + 8 * e4 + 4 * hf]) = pr;
      }
    // the wave reads back rows written by its other lanes: LDS operations of a
    // wave complete in order, so only the compiler has to keep the order
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    constexpr int CH = OUT_DIMS / 8;  // 16-byte chunks per row
    constexpr int RPI = 64 / CH;      // rows per store instruction
    const int dim0 = KSPLIT == 2 ? OUT_DIMS * kh : 0;
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int rr = i * RPI + lane / CH, ch = lane % CH;
      const u32x4 val = *reinterpret_cast<const u32x4 *>(&ys[rr * YS_PITCH + 8 * ch]);
      const int grow = r_wave + rr;
      if (grow < rows_total) {
        const int p = grow / G, hh = g * G + (grow - p * G);
        // non-temporal: the output is not read again by this kernel
        // (back-to-back cfg3 calls 35.2 -> 34.8 us, S = 1024 -2.5 %)
        __builtin_nontemporal_store(val, reinterpret_cast<u32x4 *>(
                                             a.out + ((int64_t)b * S + p) * q_row_stride +
                                             (int64_t)hh * PF_HD + dim0 + 8 * ch));
      }
    }
  }  // items of this workgroup
}

// Merge of the key parts (SPLITK): 32 threads per query row (4 dims each), 8
// rows per 256-thread workgroup; rows of single-part items were written by
// the attention kernel.  The context length and every slot's (max, sum) and O
// are loaded together (one memory round trip); slots past the row's part
// count hold another call's data and are dropped by selects.  Every row has a
// part with keys (key 0 is in every row's range), so the max M is finite and
// parts without keys weigh 0.
template <class T>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a) {
  const int64_t row = (int64_t)blockIdx.x * 8 + (threadIdx.x >> 5);
  const int d4 = (threadIdx.x & 31) * 4;
  if (row >= a.rows_all) return;
  // row = (b S + qi) Hq + h; its query block: rows qi G + h % G of (b, h / G)
  const int h = (int)(row % a.Hq);
  const int64_t bq = row / a.Hq;
  const int b = (int)(bq / a.S), qi = (int)(bq - (int64_t)b * a.S);
  const int item = (qi * a.G + h % a.G) / (32 * PF_NRB_MERGE);
  const int key_S = paged_key_count(a, b);
  float2 ml[PF_MAX_SPLIT];
  floatx4 o[PF_MAX_SPLIT];
#pragma unroll
  for (int p = 0; p < PF_MAX_SPLIT; ++p) {
    if (p < a.nsplit) {
      const int64_t pr = (int64_t)p * a.rows_all + row;
      ml[p] = *reinterpret_cast<const float2 *>(a.ws_ml + pr * 2);
      if constexpr (T::code == MCE_F16) {  // normalised fp16 partials
        const u32x2 h = *reinterpret_cast<const u32x2 *>(
            reinterpret_cast<const uint16_t *>(a.ws_o) + pr * PF_HD + d4);
        o[p] = floatx4{T::lo(h[0]), T::hi(h[0]), T::lo(h[1]), T::hi(h[1])};
      } else {
        o[p] = *reinterpret_cast<const floatx4 *>(a.ws_o + pr * PF_HD + d4);
      }
    } else {
      ml[p] = float2{-INFINITY, 0.f};
      o[p] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
  }
  const int n_parts = prefill_parts(a, key_S, item, 32 * PF_NRB_MERGE);
  if (n_parts <= 1) return;
  float M = -INFINITY;
#pragma unroll
  for (int p = 0; p < PF_MAX_SPLIT; ++p)
    if (p < n_parts) M = fmaxf(M, ml[p].x);
  float L = 0.f;
  floatx4 A = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int p = 0; p < PF_MAX_SPLIT; ++p) {
    const float w = fast_exp2(ml[p].x - M);
    // normalised fp16 partials carry their sum separately
    const float wo = T::code == MCE_F16 ? w * ml[p].y : w;
#pragma unroll
    for (int j = 0; j < 4; ++j) A[j] = p < n_parts ? A[j] + wo * o[p][j] : A[j];
    L = p < n_parts ? L + w * ml[p].y : L;
  }
  const float inv = 1.0f / L;
  u32x2 v;
  v[0] = pack2<T>(A[0] * inv, A[1] * inv);
  v[1] = pack2<T>(A[2] * inv, A[3] * inv);
  *reinterpret_cast<u32x2 *>(a.out + row * PF_HD + d4) = v;
}

}  // namespace mce

using namespace mce;

namespace {

// Items of 128 rows per (batch, kv head), heaviest first: when there are more
// items than workgroup slots, the dispatcher hands the lighter ones to the
// CUs that free up first (longest-processing-time-first scheduling).  The
// key range is split over two wave sets when the grid alone would not give
// every CU about two workgroups (long causal sequences, small batch).
constexpr int PF_NRB = PF_NRB_MERGE;
// Contiguous two-stream launches whose 128-row grid would not reach about
// 1.2 workgroups per CU take 64-row items (PF_NRB_SMALL row blocks) on 4-wave
// workgroups, two per CU: twice the workgroups over the same rows.  Measured
// on MI355X (B=1, 24 / 8 heads): S=512 13.0 -> 11.1 us, S=1024 19.1 -> 17.2,
// S=1536 26.2 -> 24.9; past the threshold (S=1792: 336 128-row items) the
// halved row block, which stages every K / V tile for half as many rows, is
// 3-9% slower.
constexpr int PF_NRB_SMALL = 2;

int64_t prefill_items(int64_t S, int G, int nrb = PF_NRB) {
  return (S * G + 32 * nrb - 1) / (32 * nrb);
}

// Key parts per item of the paged mode: grids that leave more than half of
// the CUs without a workgroup (few long sequences, a short chunk behind a
// cached prefix) cut every item's keys into at most as many parts as keep all
// workgroups in one wave of one per CU (a second round of workgroups costs
// more than the longer parts); 1 = no split.
int prefill_paged_parts(int batch, int seq_len, int num_heads, int num_kv_heads) {
  if (batch <= 0 || seq_len <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return 1;
  const int64_t grid = prefill_items(seq_len, num_heads / num_kv_heads) * batch * num_kv_heads;
  if (2 * grid > (int64_t)cu_count()) return 1;
  const int64_t n = (int64_t)cu_count() / grid;
  return (int)(n > PF_MAX_SPLIT ? PF_MAX_SPLIT : n);
}

// a.nsplit > 1: key parts (paged mode), partials in a.ws_o / a.ws_ml, then
// the merge launch
template <bool PAGED>
int prefill_launch(int dtype, PrefillArgs &a, void *stream, const char *name) {
  a.n_items = (int)prefill_items(a.S, a.G);
  const int64_t items = (int64_t)a.n_items * a.B * a.Hkv;
  MCE_REQUIRE(items * (a.nsplit > 1 ? a.nsplit : 1) < ((int64_t)1 << 31), "%s: problem too large",
              name);
  hipStream_t st = (hipStream_t)stream;
  const bool two_streams = items < 2 * (int64_t)cu_count();
  // workgroups per (sequence, kv head): one per item, or, on the two-stream
  // path when the items outnumber the CUs, one round of at most one per CU,
  // workgroup j taking item ranks j and 2 per - 1 - j (the kernel derives
  // per from the grid)
  // (small grids, contiguous: 64-row items and two workgroups per CU)
  const bool small = !PAGED && two_streams && 5 * items <= 6 * (int64_t)cu_count();
  if (small) a.n_items = (int)prefill_items(a.S, a.G, PF_NRB_SMALL);
  int64_t per = a.n_items;
  if (two_streams && a.nsplit <= 1) {
    const int64_t c_per =
        std::max<int64_t>(1, (small ? 2 : 1) * cu_count() / ((int64_t)a.B * a.Hkv));
    if (a.n_items > c_per) per = std::max<int64_t>(c_per, (a.n_items + 1) / 2);
  }
  const int64_t grid = per * a.B * a.Hkv * (a.nsplit > 1 ? a.nsplit : 1);
  if constexpr (PAGED) {
    if (a.nsplit > 1) {
      const unsigned mgrid = (unsigned)((a.rows_all + 7) / 8);
      if (dtype == MCE_F16) {
        prefill_causal_kernel<F16T, PF_NRB, 2, true, true, PF_BN><<<(unsigned)grid, PF_NRB * 128, 0, st>>>(a);
        prefill_merge_kernel<F16T><<<mgrid, 256, 0, st>>>(a);
      } else {
        prefill_causal_kernel<BF16T, PF_NRB, 2, true, true, PF_BN><<<(unsigned)grid, PF_NRB * 128, 0, st>>>(a);
        prefill_merge_kernel<BF16T><<<mgrid, 256, 0, st>>>(a);
      }
      return check_launch(name);
    }
  }
  // 32-key tiles: 64-key tiles (241 registers) measured 5% slower at cfg3
  // and 8% at B=8 S=512 with the same staging
  constexpr int BN = PF_BN;
  if constexpr (!PAGED) {
    if (small) {
      if (dtype == MCE_F16)
        prefill_causal_kernel<F16T, PF_NRB_SMALL, 2, false, false, BN><<<(unsigned)grid, PF_NRB_SMALL * 128, 0, st>>>(a);
      else
        prefill_causal_kernel<BF16T, PF_NRB_SMALL, 2, false, false, BN><<<(unsigned)grid, PF_NRB_SMALL * 128, 0, st>>>(a);
      return check_launch(name);
    }
  }
  if (dtype == MCE_F16) {
    if (two_streams)
      prefill_causal_kernel<F16T, PF_NRB, 2, PAGED, false, BN><<<(unsigned)grid, PF_NRB * 128, 0, st>>>(a);
    else
      prefill_causal_kernel<F16T, PF_NRB, 1, PAGED, false, BN><<<(unsigned)grid, PF_NRB * 64, 0, st>>>(a);
  } else {
    if (two_streams)
      prefill_causal_kernel<BF16T, PF_NRB, 2, PAGED, false, BN><<<(unsigned)grid, PF_NRB * 128, 0, st>>>(a);
    else
      prefill_causal_kernel<BF16T, PF_NRB, 1, PAGED, false, BN><<<(unsigned)grid, PF_NRB * 64, 0, st>>>(a);
  }
  return check_launch(name);
}

}  // namespace

extern "C" int mce_prefill_attention(int dtype, const void *query,
                                     const void *key, const void *value,
                                     void *output, int batch, int seq_len,
                                     int num_heads, int num_kv_heads,
                                     int head_dim, float scale, void *stream) {
  clear_error();
  MCE_REQUIRE(dtype == MCE_F16 || dtype == MCE_BF16,
              "mce_prefill_attention: unknown dtype %d", dtype);
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
  // one sequence's queries are addressed with 32-bit byte offsets
  MCE_REQUIRE((int64_t)seq_len * num_heads * head_dim * 2 < ((int64_t)1 << 31),
              "mce_prefill_attention: seq_len * num_heads too large");
  // K/V tiles are addressed with 32-bit byte offsets within one batch entry
  // (including the prefetch of up to 6 64-key tiles past the end)
  MCE_REQUIRE(((int64_t)seq_len + 512) * num_kv_heads * head_dim * 2 < ((int64_t)1 << 31),
              "mce_prefill_attention: seq_len * num_kv_heads too large");
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
  a.scale_log2 = scale * 1.4426950408889634f;
  return prefill_launch<false>(dtype, a, stream, "mce_prefill_attention");
}

extern "C" size_t mce_prefill_attention_paged_workspace_size(int batch, int seq_len,
                                                          int num_heads, int num_kv_heads) {
  const int parts = prefill_paged_parts(batch, seq_len, num_heads, num_kv_heads);
  if (parts <= 1) return 0;
  const size_t rows = (size_t)batch * seq_len * num_heads * parts;
  return ((rows * PF_HD * sizeof(float) + 255) & ~(size_t)255) + rows * 2 * sizeof(float);
}

extern "C" int mce_prefill_attention_paged(int dtype, const void *query, const void *key_cache,
                                           const void *value_cache, const int32_t *block_tables,
                                           const int32_t *context_lens, void *output, int batch,
                                           int seq_len, int num_heads, int num_kv_heads,
                                           int head_dim, int max_blocks_per_seq, int block_size,
                                           int64_t num_blocks, float scale, void *workspace,
                                           size_t workspace_bytes, void *stream) {
  clear_error();
  const char *name = "mce_prefill_attention_paged";
  MCE_REQUIRE(dtype == MCE_F16 || dtype == MCE_BF16, "%s: unknown dtype %d", name, dtype);
  MCE_REQUIRE(head_dim == PF_HD, "%s: head_dim must be 128 (got %d)", name, head_dim);
  MCE_REQUIRE(batch >= 0 && seq_len >= 0 && num_heads >= 1 && num_kv_heads >= 1 &&
                  max_blocks_per_seq >= 0 && num_blocks >= 0,
              "%s: bad shape", name);
  MCE_REQUIRE(num_heads % num_kv_heads == 0, "%s: num_heads %d not a multiple of num_kv_heads %d",
              name, num_heads, num_kv_heads);
  MCE_REQUIRE(is_pow2(block_size) && block_size >= 1 && block_size <= 1024,
              "%s: block_size must be a power of two <= 1024 (got %d)", name, block_size);
  if (batch == 0 || seq_len == 0) return MCE_OK;
  MCE_REQUIRE(query && key_cache && value_cache && block_tables && context_lens && output,
              "%s: null pointer", name);
  MCE_REQUIRE(aligned16(query) && aligned16(key_cache) && aligned16(value_cache) &&
                  aligned16(output),
              "%s: tensors must be 16-byte aligned", name);
  MCE_REQUIRE(max_blocks_per_seq <= PF_MAX_BLOCKS,
              "%s: at most %d blocks per sequence (got %d)", name, PF_MAX_BLOCKS,
              max_blocks_per_seq);
  MCE_REQUIRE((int64_t)max_blocks_per_seq * block_size >= seq_len,
              "%s: the block tables hold %lld tokens, fewer than the %d query positions", name,
              (long long)max_blocks_per_seq * block_size, seq_len);
  MCE_REQUIRE(num_blocks >= 1, "%s: empty page pool", name);
  const int G = num_heads / num_kv_heads;
  MCE_REQUIRE((int64_t)seq_len * G < ((int64_t)1 << 30), "%s: too many query rows", name);
  MCE_REQUIRE((int64_t)seq_len * num_heads * head_dim * 2 < ((int64_t)1 << 31),
              "%s: seq_len * num_heads too large", name);
  const int64_t cache_bytes = num_blocks * block_size * num_kv_heads * head_dim * 2;
  MCE_REQUIRE(cache_bytes < ((int64_t)1 << 31),
              "%s: the page pool must be smaller than 2 GiB (32-bit offsets)", name);
  PrefillArgs a{};
  a.q = (const uint16_t *)query;
  a.k = (const uint16_t *)key_cache;
  a.v = (const uint16_t *)value_cache;
  a.out = (uint16_t *)output;
  a.B = batch;
  a.S = seq_len;
  a.Hq = num_heads;
  a.Hkv = num_kv_heads;
  a.G = G;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.block_tables = block_tables;
  a.context_lens = context_lens;
  a.maxb = max_blocks_per_seq;
  a.bs_log2 = ilog2(block_size);
  a.num_blocks = num_blocks;
  a.cache_bytes = (uint32_t)cache_bytes;
  // the key split runs only when the caller hands in a workspace
  a.nsplit = workspace ? prefill_paged_parts(batch, seq_len, num_heads, num_kv_heads) : 1;
  if (a.nsplit > 1) {
    const size_t need = mce_prefill_attention_paged_workspace_size(batch, seq_len, num_heads,
                                                                   num_kv_heads);
    if (workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255) != 0)
      return set_error(MCE_ERR_WORKSPACE,
                       "%s: a 256-byte aligned workspace of %zu bytes is required (%zu given)",
                       name, need, workspace_bytes);
    a.rows_all = (int64_t)batch * seq_len * num_heads;
    a.ws_o = (float *)workspace;
    a.ws_ml = (float *)((char *)workspace +
                        (((size_t)a.rows_all * a.nsplit * PF_HD * sizeof(float) + 255) & ~(size_t)255));
  }
  return prefill_launch<true>(dtype, a, stream, name);
}
