// Ragged grouped matmul with FP4 (e2m1 + e8m0 block-32) weights, bf16
// activations, f32 accumulation: the tokamax gmm_v2 rhs_fp4_codes path
// (patches/tokamax/0001-gmm_v2-fp4-emulation-v6e.patch:58-66, :100-151).
//
// Work decomposition: a block owns one (local group, 96-row tile) x
// (512-column tile).  Tiles are enumerated on the device from group_sizes (no
// host sync): the tile total is (row tiles of every local group) x (column
// tiles); empty groups own no tile and cost no weight traffic.  Tiles are
// listed by cost class (16-row MFMA blocks holding rows, largest first) so
// the dispatcher, which hands blocks to free CUs in index order, balances
// multi-round launches.  Blocks whose index is equal mod 8 run on one XCD
// (the dispatcher's round robin); each class is cut into one contiguous run
// per XCD -- consecutive column tiles of the same row tile -- so the group's
// lhs rows are shared in that XCD's L2.  When the tiles leave CUs idle (a
// one-round decode launch), the costliest classes run as 256-column tiles.
//
// The block is warp-specialised (see the WsCfg comment): producer waves move
// the lhs tile and the prepacked weights and scales (fp4.hip) from memory to
// a ring of LDS stages with direct global -> LDS loads; consumer waves decode
// the weights in registers with the gfx950 fp4 -> bf16 converter (which
// applies the e8m0 scale exactly) and run bf16 MFMA 16x16x32 for every 16-row
// block that holds rows.  The dequantised weights are exact (e2m1 x power of
// two fits bf16), so the products equal the reference's
// bf16(decode(q)) * bf16(scale) operands; only the f32 summation order differs,
// and it is the same for every row.
#include <algorithm>
#include <atomic>
#include <cstdlib>

#include "gmm_tiles.h"

namespace dwm {

// Per-block timeline, compiled only into the timeline build of the library
// (-DDWTPU_TIMELINE, libdwtpu_moe_timeline.so; the product library has no
// trace of it).  Lane 0 of a wave stores a counter into slot `slot` of its
// block's record of kTlSlots words: s_memrealtime (100 MHz, the same clock
// on every XCD) unless noted.  Slots: 0 block entry; 1 HW_ID | XCC_ID << 32;
// 2 tile found; 3 rows | narrow << 16 (0: no tile); 4, 5, 6 consumer wave
// 0's first barrier passed, K loop done, stores issued; 7 and 20 wave 0's
// s_memtime (shader clock) at entry and exit; 8 + w wave w's exit.
[[maybe_unused]] constexpr int kTlSlots = 24;
#ifdef DWTPU_TIMELINE
static __device__ uint64_t *g_timeline;
static __device__ int64_t g_timeline_blocks;
#define DWM_TL(slot, v)                                                                     \
  do {                                                                                      \
    if ((threadIdx.x & 63) == 0 && g_timeline && (int64_t)blockIdx.x < g_timeline_blocks) \
      g_timeline[(int64_t)blockIdx.x * kTlSlots + (slot)] = (uint64_t)(v);                  \
  } while (0)
#else
#define DWM_TL(slot, v) ((void)0)
#endif

// Per-wave step accounting, also in the timeline build only: every wave of a
// tile block sums its shader cycles (s_memtime) by phase into kGsSlots words
// at (blockIdx.x * 16 + wave) * kGsSlots of a second buffer: 0 from its
// role's start to its first wait, 1 waits before barriers (producers: vmcnt
// for their loads; consumers: their LDS reads), 2 barriers, 3 work between
// barriers, 4 from the last barrier to the role's end (consumers: epilogue
// stores issued), 5 barriers passed, 6 role (1 producer, 2 consumer, 3 idle
// consumer of a narrow tile) | rows << 8 | narrow << 24, 7 and 8
// s_memrealtime at the role's start and end, 9 s_memtime from start to end.
[[maybe_unused]] constexpr int kGsSlots = 10;
#ifdef DWTPU_TIMELINE
static __device__ uint64_t *g_gmm_steps;
static __device__ int64_t g_gmm_steps_waves;
struct GsAcct {
  uint64_t rt0, t0, prev, pro, wait, bar, work;
  int n;
  __device__ void start() {
    rt0 = __builtin_amdgcn_s_memrealtime();
    t0 = prev = __builtin_amdgcn_s_memtime();
    pro = wait = bar = work = 0;
    n = 0;
  }
  // ta before a wait, tb after it, tc after the barrier that follows.
  __device__ void step(uint64_t ta, uint64_t tb, uint64_t tc) {
    if (n == 0) pro = ta - prev;
    else work += ta - prev;
    wait += tb - ta;
    bar += tc - tb;
    prev = tc;
    ++n;
  }
  __device__ void finish() {
    const uint64_t end = __builtin_amdgcn_s_memtime(), rt1 = __builtin_amdgcn_s_memrealtime();
    const int64_t slot = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 6);
    if ((threadIdx.x & 63) == 0 && g_gmm_steps && slot < g_gmm_steps_waves) {
      uint64_t *const p = g_gmm_steps + slot * kGsSlots;
      p[0] = pro;
      p[1] = wait;
      p[2] = bar;
      p[3] = work;
      p[4] = end - prev;
      p[5] = (uint64_t)n;
      p[7] = rt0;
      p[8] = rt1;
      p[9] = end - t0;
    }
  }
};
__device__ __forceinline__ void gs_role(uint64_t info) {
  const int64_t slot = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 6);
  if ((threadIdx.x & 63) == 0 && g_gmm_steps && slot < g_gmm_steps_waves) g_gmm_steps[slot * kGsSlots + 6] = info;
}
#define DWM_GS(...) __VA_ARGS__
#else
#define DWM_GS(...)
#endif

// lhs tile rows hold 8 16-byte chunks; chunk c of row r sits at physical
// chunk c ^ ((r >> 1) & 7), so that the 16 lanes of one LDS cycle (16
// consecutive rows, one logical chunk) hit 16 distinct 16-byte bank groups.
__device__ __forceinline__ int lhs_swizzle(int r) { return (r >> 1) & 7; }

// ---------------------------------------------------------------------------
// Warp-specialised tiles.
//
// A block of 12 waves owns (group, 32*MB rows) x 512 columns (256 in a narrow
// tile, whose last four consumers idle).  Waves 0..7 (consumers, two per
// SIMD) each own 64 columns: they read the lhs tile and their weight codes
// and scales from LDS, decode, and run the MFMAs.
// Waves 8..11 (producers, one per SIMD) only move data: global -> LDS loads
// (global_load_lds) of the lhs tile, weights and scales through a ring of LDS
// stages.  One workgroup barrier per 64-deep K step publishes two steps
// (t and t + 1) to the consumers and hands the stage of step t - 1 back to
// the producers.  Each role issues one kind of memory operation, so the
// compiler's waits stay exact, and the consumers carry no load rings in
// registers.  The consumers read step t + 1's weights, scales and first lhs
// fragments during step t, and each group of MFMAs' lhs fragments during the
// previous group, so no MFMA waits on a fresh LDS read.
//
// Weight layout (64-column groups): for expert e, group g (columns 64 g ..
// 64 g + 63, N padded to a multiple of 64 with zero codes), 64-deep K step t
// and half j: 1 KiB where lane l = c + 32 h holds the 32 codes of column
// 64 g + 32 j + c at k = 64 t + 32 h .. + 31, two per byte, low nibble first.
// Scale layout: for (e, g, 128-deep step kb) 256 bytes; byte 2 f + j of lane
// l = c + 32 h is the e8m0 code of column 64 g + 32 j + c, K-block
// 4 kb + 2 f + h.  Decoded, lane (c, h)'s codes k = 64 t + 32 h + 8 s .. + 7
// are the B operand of a 32x32x16 MFMA step s (the MX kernel's 32x32x64
// operand is the lane's 16 bytes as they are); the consumers here read the
// 4-byte pieces of the 16x16x32 operands from their slots (ws_consumer).
// Block shape: CW consumer waves owning JW 32-column blocks each (a tile of
// 32 JW CW columns = GT 64-column groups), NP producer waves, NS LDS stages.
template <int MB, int CW, int JW, int NP, int NS>
struct WsCfg {
  static constexpr int CONS = CW, JWAVE = JW, NPROD = NP, STAGES = NS;
  static constexpr int GT = JW * CW / 2;                 // 64-column groups per tile
  static constexpr int THREADS = 64 * (CW + NP);
  static constexpr int NT = 64 * GT;
  static constexpr int A = 0;                           // 32 MB rows x 128 bytes (8 swizzled 16-byte chunks)
  static constexpr int W = 32 * MB * 128;               // group i of the tile: 2 KiB at W + 2048 i
  static constexpr int S = W + GT * 2048;               // group i: 256 bytes at S + 256 i
  static constexpr int STAGE = S + GT * 256;
  static constexpr int A_LOADS = 4 * MB / NP;           // 1 KiB lhs loads (8 rows) per producer per step
  static constexpr int G_LOADS = GT / NP;               // groups per producer
  static constexpr int AHEAD = 2;                       // steps published per barrier
  static constexpr int EP_STRIDE = 72;                  // epilogue staging row stride (floats)
  static_assert(A_LOADS * NP == 4 * MB && G_LOADS * NP == GT, "loads split evenly over the producers");
  static_assert(NS - 1 - AHEAD >= 1, "stage count");
  static_assert(JW == 2, "one 64-column group per consumer wave");
  static_assert(CW * 32 * EP_STRIDE * 4 <= NS * STAGE, "epilogue staging fits the stages");
};

// Producer wave pw: NA of its A_LOADS lhs row groups hold rows of the tile;
// the others are zero in every stage and never loaded.  It loads GL of the
// tile's 64-column weight groups (G_LOADS in a wide tile, half in a narrow one).
template <class C, int NA, int GL>
__device__ __forceinline__ void ws_producer(const uint16_t *__restrict__ lhs, const int32_t *__restrict__ row_idx,
                                            int64_t lhs_rows, int64_t row0, int rows, int K, int T,
                                            int KB, const uint8_t *__restrict__ wexp,
                                            const uint8_t *__restrict__ sexp, int g0, int G, uint8_t *s_lds,
                                            int pw) {
  constexpr int NP = C::NPROD, NS = C::STAGES;
  constexpr int LOADS = NA + 3 * GL;
  constexpr int PENDING = LOADS * (NS - 1 - C::AHEAD);
  static_assert(PENDING < 64, "vmcnt range");
  const int lane = threadIdx.x & 63;
  DWM_GS(GsAcct gs; gs.start();)
  // Row groups pw + NP i, i >= NA, lie past the tile's rows: zero them.
#pragma unroll
  for (int i = NA; i < C::A_LOADS; ++i)
#pragma unroll
    for (int st = 0; st < NS; ++st)
      *(u32x4_t *)(s_lds + st * C::STAGE + C::A + (pw + NP * i) * 1024 + lane * 16) = u32x4_t{0u, 0u, 0u, 0u};
  // lhs load i: rows 8 (pw + NP i) .. + 7 of the tile; lane l fills physical
  // chunk l % 8 of row + l / 8 with logical chunk (l % 8) ^ swizzle(row).
  // Rows past the tile repeat its last row.  With row_idx (the fused row
  // gather) tile row r is lhs row row_idx[row0 + r], under JAX gather index
  // semantics; the indices are read once, before any direct-to-LDS load.
  const uint8_t *const abase = (const uint8_t *)(row_idx ? lhs : lhs + row0 * K);
  uint32_t aoff[NA > 0 ? NA : 1];
#pragma unroll
  for (int i = 0; i < NA; ++i) {
    const int r = 8 * (pw + NP * i) + (lane >> 3);
    const int rs = r < rows ? r : rows - 1;
    const int64_t src = row_idx ? gather_index(row_idx[row0 + rs], lhs_rows) : rs;
    aoff[i] = (uint32_t)(src * K * 2) + ((((lane & 7) ^ lhs_swizzle(r))) << 4);
  }
  const uint8_t *wsrc[GL];
  const uint8_t *ssrc[GL];
#pragma unroll
  for (int c = 0; c < GL; ++c) {
    const int g = min(g0 + pw + NP * c, G - 1);  // groups past N feed unstored columns
    wsrc[c] = wexp + (int64_t)g * T * 2048 + lane * 16;
    ssrc[c] = sexp + (int64_t)g * KB * 256 + lane * 4;
  }
  auto issue = [&](int stage, int t) {
    uint8_t *const st = s_lds + stage * C::STAGE;
    const uint8_t *const a = abase + (int64_t)t * 128;
#pragma unroll
    for (int i = 0; i < NA; ++i)
      __builtin_amdgcn_global_load_lds((const void *)(a + aoff[i]),
                                       (lds_void_t *)(st + C::A + (pw + NP * i) * 1024), 16, 0, 0);
#pragma unroll
    for (int c = 0; c < GL; ++c) {
      const int gi = pw + NP * c;
      const uint8_t *const w = wsrc[c] + (int64_t)t * 2048;
      __builtin_amdgcn_global_load_lds((const void *)w, (lds_void_t *)(st + C::W + gi * 2048), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void *)(w + 1024), (lds_void_t *)(st + C::W + gi * 2048 + 1024), 16,
                                       0, 0);
      __builtin_amdgcn_global_load_lds((const void *)(ssrc[c] + (int64_t)(t >> 1) * 256),
                                       (lds_void_t *)(st + C::S + gi * 256), 4, 0, 0);
    }
  };
#pragma unroll
  for (int t = 0; t < NS - 1; ++t) issue(t, min(t, T - 1));
  int refill = NS - 1;  // stage of step t + NS - 1
  for (int t = 0; t < T; ++t) {
    // Steps t .. t + AHEAD - 1 have landed once at most the loads of the
    // later steps are pending.
    DWM_GS(const uint64_t gs_a = __builtin_amdgcn_s_memtime();)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(PENDING));
    DWM_GS(const uint64_t gs_b = __builtin_amdgcn_s_memtime();)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    DWM_GS(gs.step(gs_a, gs_b, __builtin_amdgcn_s_memtime());)
    // The consumers are done with step t - 1: refill its stage with step
    // t + NS - 1 (clamped to the last step, so every step issues the same loads).
    issue(refill, min(t + NS - 1, T - 1));
    refill = refill == NS - 1 ? 0 : refill + 1;
  }
  // Every load has landed before the stages are reused for the epilogue.
  DWM_GS(const uint64_t gs_a = __builtin_amdgcn_s_memtime();)
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  DWM_GS(const uint64_t gs_b = __builtin_amdgcn_s_memtime();)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  DWM_GS(gs.step(gs_a, gs_b, __builtin_amdgcn_s_memtime()); gs.finish();)
}

// A consumer wave runs its 64 columns for NH 16-row blocks of the tile with
// 16x16x32 MFMAs: every row of every tile sums K in the same grouping, so a
// row's result depends on its own lhs row only (not on its place in the
// tile), and MFMA work follows the rows in steps of 16.  In MFMA step v
// (32 of the K step's 64) lane row q = lane / 16 of the B operand of column
// block u holds K chunk (h = q / 2, s = 2v + q % 2) of column 16 u + lane %
// 16: 8 codes that the prepack stores as 4 bytes of the column's slot (slot
// c + 32 h of half j holds k = 32 h .. + 31, chunk s at byte 4 s), read from
// LDS and decoded in place (two such dwords per column block and K step, one
// ds_read2).  The lhs fragment of MFMA step v reads the same K chunk, so the
// sum over K is the same in another order.  Each K step runs 2 x NH x 4
// MFMAs in groups of at most 3 row blocks; a group's lhs fragments are read
// during the previous group.
template <class C, int NH, bool ACT>
__device__ __forceinline__ void ws_consumer(int T, uint8_t *s_lds, int cw, int64_t row0, int rows,
                                            int64_t col0, int N, void *__restrict__ out, int out_f32,
                                            const void *bias, const GmmEpilogue &ep) {
  constexpr int NS = C::STAGES;
  constexpr int RG = NH > 3 ? 2 : 1;      // row groups of at most three 16-row blocks
  constexpr int H0 = NH > 3 ? 3 : NH;     // blocks of row group 0 (row group 1: NH - H0)
  static_assert(C::JWAVE == 2 && NH >= 1 && NH <= 6, "64 columns and 16 .. 96 rows per consumer");
  const int lane = threadIdx.x & 63, q = lane >> 4;
  DWM_GS(GsAcct gs; gs.start();)
  f32x4_t acc[NH][4];
#pragma unroll
  for (int hb = 0; hb < NH; ++hb)
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[hb][u] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const int arow = C::A + (lane & 15) * 128;  // row 16 hb + lane % 16: + 2048 hb
  const int x = lhs_swizzle(lane & 15);       // every row 16 hb + lane % 16 shares it
  const int qk = 4 * (q >> 1) + (q & 1);      // K chunk of MFMA step v: qk + 2 v
  // The B operand of column block u (columns 16 (u & 1) + c16 of half
  // j = u >> 1) in lane (c16, q) of MFMA step v: the 8 codes of K chunk
  // (h = q >> 1, s = 2 v + (q & 1)), i.e. bytes 8 v + 4 (q & 1) .. + 3 of
  // slot c32 + 32 h of half j; its scale, byte 2 f + j of that slot's dword.
  const int slot = (lane & 15) + 32 * (q >> 1);
  const int woff = C::W + cw * 2048 + slot * 16 + 4 * (q & 1);  // + 1024 j + 256 (u & 1) + 8 v
  const int soff = C::S + cw * 256 + slot * 4;                   // + 64 (u & 1)
  // Next step's weights and scales, and the lhs fragments of the next MFMA group.
  u32x2_t wn[4];
  u32x4_t an[3];
  uint32_t sn[2];
  auto read_w = [&](const uint8_t *st) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const uint32_t *const p = (const uint32_t *)(st + woff + 1024 * (u >> 1) + 256 * (u & 1));
      wn[u] = u32x2_t{p[0], p[2]};
    }
    sn[0] = *(const uint32_t *)(st + soff);
    sn[1] = *(const uint32_t *)(st + soff + 64);
  };
  auto read_a = [&](const uint8_t *st, int v, int rg) {
    const int ach = ((qk + 2 * v) ^ x) << 4;
    const int nb = rg ? NH - H0 : H0;
#pragma unroll
    for (int i = 0; i < nb; ++i) an[i] = *(const u32x4_t *)(st + arow + (3 * rg + i) * 2048 + ach);
  };
  if constexpr (NH >= 3 && NH <= 5) {
  // Decode ahead (3 to 5 row blocks, where the registers allow it): the B
  // operands of each half step (MFMA step v) are decoded during the previous
  // half step.  Its last MFMA group -- three row blocks, so three MFMAs
  // cover each column block's decode -- runs column block by column block,
  // and right after the last MFMA that reads bop[u] the next half step's
  // bop[u] is decoded in its place, so after a barrier the MFMAs start at
  // once.  The next K step's weights and scales are read at the end of this
  // step's v = 0 half.  Row groups: blocks [0, G0) then [G0, NH).
  constexpr int G0 = NH - 3, DRG = G0 > 0 ? 2 : 1;
  u32x4_t bop[4];
  auto decode = [&](int u, int v, int parity) {
    const float sc = __builtin_bit_cast(float, __builtin_amdgcn_ubfe(sn[u & 1], 16 * parity + 8 * (u >> 1), 8) << 23);
    bop[u][0] = cvt_fp4x2_bf16<0>(wn[u][v], sc);
    bop[u][1] = cvt_fp4x2_bf16<1>(wn[u][v], sc);
    bop[u][2] = cvt_fp4x2_bf16<2>(wn[u][v], sc);
    bop[u][3] = cvt_fp4x2_bf16<3>(wn[u][v], sc);
  };
  // lhs fragments of row group g of MFMA step v
  auto read_g = [&](const uint8_t *st, int v, int g) {
    const int ach = ((qk + 2 * v) ^ x) << 4;
    const int b0 = (DRG == 2 && g == 1) ? G0 : 0;
    const int nb = (DRG == 2 && g == 0) ? G0 : 3;
#pragma unroll
    for (int i = 0; i < nb; ++i) an[i] = *(const u32x4_t *)(st + arow + (b0 + i) * 2048 + ach);
  };
  // One MFMA group (row group rg of MFMA step v) on stage cs; ns is the next
  // step's stage (read by the last group only).  par0 / par1: the scale
  // parity of this step and of the next.
  auto run_group = [&](const uint8_t *cs, const uint8_t *ns, auto vc, auto rgc, int par0, int par1) {
    constexpr int v = decltype(vc)::value, rg = decltype(rgc)::value;
    constexpr int nb = (DRG == 2 && rg == 0) ? G0 : 3;
    constexpr int b0 = (DRG == 2 && rg == 1) ? G0 : 0;
    u32x4_t a[3];
#pragma unroll
    for (int i = 0; i < nb; ++i) a[i] = an[i];
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (rg + 1 < DRG) read_g(cs, v, rg + 1);
    else if constexpr (v == 0) read_g(cs, 1, 0);
    else read_g(ns, 0, 0);
    if constexpr (rg + 1 < DRG) {
#pragma unroll
      for (int i = 0; i < nb; ++i)
#pragma unroll
        for (int u = 0; u < 4; ++u)
          acc[b0 + i][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, a[i]), __builtin_bit_cast(bf16x8_t, bop[u]), acc[b0 + i][u], 0, 0, 0);
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int i = 0; i < nb; ++i)
          acc[b0 + i][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf16x8_t, a[i]), __builtin_bit_cast(bf16x8_t, bop[u]), acc[b0 + i][u], 0, 0, 0);
        decode(u, v == 0 ? 1 : 0, v == 0 ? par0 : par1);
        __builtin_amdgcn_sched_barrier(0);  // keep each decode after the MFMAs that read the old bop[u]
      }
      if constexpr (v == 0) read_w(ns);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // With two row groups, the first group of step t + 1 runs before barrier
  // t + 1: that step was published at barrier t, and its lhs fragments and
  // B operands are already in registers, so the wave that finishes step t
  // first keeps the SIMD's MFMA unit busy instead of waiting.  Every
  // accumulator still takes its MFMAs in step order.
  static_assert(NS % 2 == 0, "t & 1 == cur & 1");
  for (int t0 = 0; t0 < T; t0 += NS) {
#pragma unroll
  for (int cur = 0; cur < NS; ++cur) {
    const int t = t0 + cur;
    if (t >= T) break;
    asm volatile("" ::: "memory");
    DWM_GS(const uint64_t gs_a = __builtin_amdgcn_s_memtime();)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    DWM_GS(const uint64_t gs_b = __builtin_amdgcn_s_memtime();)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    DWM_GS(gs.step(gs_a, gs_b, __builtin_amdgcn_s_memtime());)
    const uint8_t *const st = s_lds + cur * C::STAGE;
    const int nxt = cur == NS - 1 ? 0 : cur + 1;
    // Step t + 1 was published at this barrier (stale contents in the last step, never used).
    const uint8_t *const sx = s_lds + nxt * C::STAGE;
    if (t == 0) {
      if (cw == 0) DWM_TL(4, __builtin_amdgcn_s_memrealtime());
      read_w(st);
      read_g(st, 0, 0);
#pragma unroll
      for (int u = 0; u < 4; ++u) decode(u, 0, 0);
    }
    const int p0 = cur & 1, p1 = (cur + 1) & 1;
    if (DRG == 1 || t == 0) run_group(st, sx, IntC<0>{}, IntC<0>{}, p0, p1);
    if constexpr (DRG == 2) run_group(st, sx, IntC<0>{}, IntC<1>{}, p0, p1);
    run_group(st, sx, IntC<1>{}, IntC<0>{}, p0, p1);
    if constexpr (DRG == 2) {
      run_group(st, sx, IntC<1>{}, IntC<1>{}, p0, p1);
      if (t + 1 < T) run_group(sx, sx, IntC<0>{}, IntC<0>{}, p1, p0);
    }
  }
  }
  } else {
  // Steps in runs of NS, one per stage, so that every stage address is a
  // constant offset (cur = t % NS is known in each copy of the body).
  static_assert(NS % 2 == 0, "t & 1 == cur & 1");
  for (int t0 = 0; t0 < T; t0 += NS) {
#pragma unroll
  for (int cur = 0; cur < NS; ++cur) {
    const int t = t0 + cur;
    if (t >= T) break;
    asm volatile("" ::: "memory");
    DWM_GS(const uint64_t gs_a = __builtin_amdgcn_s_memtime();)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    DWM_GS(const uint64_t gs_b = __builtin_amdgcn_s_memtime();)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    DWM_GS(gs.step(gs_a, gs_b, __builtin_amdgcn_s_memtime());)
    const uint8_t *const st = s_lds + cur * C::STAGE;
    const int nxt = cur == NS - 1 ? 0 : cur + 1;
    // Step t + 1 was published at this barrier and its stage is not refilled
    // before the next one.  In the last step the reads of "step T" fetch
    // stale stage contents that are never used.
    const uint8_t *const sx = s_lds + nxt * C::STAGE;
    if (t == 0) {
      if (cw == 0) DWM_TL(4, __builtin_amdgcn_s_memrealtime());
      read_w(st);
      read_a(st, 0, 0);
    }
    float sc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      sc[u] = __builtin_bit_cast(float, __builtin_amdgcn_ubfe(sn[u & 1], 16 * (cur & 1) + 8 * (u >> 1), 8) << 23);
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      u32x4_t bop[4];  // B operands of column blocks u = 0 .. 3
#pragma unroll
      for (int rg = 0; rg < RG; ++rg) {
        const int nb = rg ? NH - H0 : H0;
        u32x4_t a[3];
#pragma unroll
        for (int i = 0; i < nb; ++i) a[i] = an[i];
        __builtin_amdgcn_sched_barrier(0);
        if (rg + 1 < RG) read_a(st, v, rg + 1);
        else if (v == 0) read_a(st, 1, 0);
        else read_a(sx, 0, 0);
        if (rg == 0) {
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            bop[u][0] = cvt_fp4x2_bf16<0>(wn[u][v], sc[u]);
            bop[u][1] = cvt_fp4x2_bf16<1>(wn[u][v], sc[u]);
            bop[u][2] = cvt_fp4x2_bf16<2>(wn[u][v], sc[u]);
            bop[u][3] = cvt_fp4x2_bf16<3>(wn[u][v], sc[u]);
          }
          // the next step's weights and scales, once this step's are decoded
          // (the step's remaining MFMA groups cover the reads)
          if (v == 1) read_w(sx);
        }
#pragma unroll
        for (int i = 0; i < nb; ++i)
#pragma unroll
          for (int u = 0; u < 4; ++u)
            acc[3 * rg + i][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8_t, a[i]), __builtin_bit_cast(bf16x8_t, bop[u]), acc[3 * rg + i][u], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  }
  }
  // One more barrier: every wave is done with the stages and every load has
  // landed, so each consumer stages its results in a private LDS region and
  // writes whole 8-column runs of a row.
  if (cw == 0) DWM_TL(5, __builtin_amdgcn_s_memrealtime());
  asm volatile("" ::: "memory");
  DWM_GS(const uint64_t gs_a = __builtin_amdgcn_s_memtime();)
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  DWM_GS(const uint64_t gs_b = __builtin_amdgcn_s_memtime();)
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  DWM_GS(gs.step(gs_a, gs_b, __builtin_amdgcn_s_memtime());)
  store_halves<NH, ACT, C::EP_STRIDE>(acc, (float *)(s_lds + cw * 32 * C::EP_STRIDE * 4), row0, rows, col0, N, out,
                                      out_f32, bias, ep.bias_bf16, ep.act);
  if (cw == 0) DWM_TL(6, __builtin_amdgcn_s_memrealtime());
  DWM_GS(gs.finish();)
}

// A consumer wave with no columns in a narrow tile: it only keeps the
// barrier count (T + 1) of the others.
__device__ __forceinline__ void ws_idle_consumer(int T) {
  DWM_GS(GsAcct gs; gs.start();)
  for (int t = 0; t <= T; ++t) {
    asm volatile("" ::: "memory");
    DWM_GS(const uint64_t gs_a = __builtin_amdgcn_s_memtime();)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    DWM_GS(gs.step(gs_a, gs_a, __builtin_amdgcn_s_memtime());)
  }
  DWM_GS(gs.finish();)
}

// Producer dispatch on the number of lhs row groups that hold rows.
template <class C, int GL>
__device__ __forceinline__ void ws_produce(int na, const uint16_t *lhs, const int32_t *row_idx, int64_t lhs_rows,
                                           int64_t row0, int rows, int K, int T, int KB, const uint8_t *wexp,
                                           const uint8_t *sexp, int g0, int G, uint8_t *s_lds, int pw) {
  constexpr int AL = C::A_LOADS;
  if (na >= AL) ws_producer<C, AL, GL>(lhs, row_idx, lhs_rows, row0, rows, K, T, KB, wexp, sexp, g0, G, s_lds, pw);
  else if (na == 2) ws_producer<C, (AL > 2 ? 2 : AL), GL>(lhs, row_idx, lhs_rows, row0, rows, K, T, KB, wexp, sexp, g0, G, s_lds, pw);
  else if (na == 1) ws_producer<C, (AL > 1 ? 1 : AL), GL>(lhs, row_idx, lhs_rows, row0, rows, K, T, KB, wexp, sexp, g0, G, s_lds, pw);
  else ws_producer<C, 0, GL>(lhs, row_idx, lhs_rows, row0, rows, K, T, KB, wexp, sexp, g0, G, s_lds, pw);
}

// NARROW: the tile list may cut its costliest classes into 256-column tiles
// (find_tile) when the 512-column tiles leave some of the ncu CUs idle.
template <class C, int MB, bool ACT, bool NARROW>
__global__ __launch_bounds__(C::THREADS) void gmm_fp4_ws_kernel(
    const uint16_t *__restrict__ lhs, const int32_t *__restrict__ row_idx, int64_t lhs_rows, int64_t M, int K,
    const uint8_t *__restrict__ wpk,
    const uint8_t *__restrict__ spk, const int32_t *__restrict__ group_sizes, int num_groups,
    const int32_t *__restrict__ group_offset, int64_t e_local, int N, void *__restrict__ out,
    int out_f32, GmmEpilogue ep, int ncu, int bal) {
  constexpr int CW = C::CONS;
  constexpr int NC = 2 * MB;  // tile classes: 16-row blocks holding rows
  static_assert(MB == 3, "consumer variants are written for 96-row tiles");
  static_assert(C::STAGES * C::STAGE >= (kMaxGroups + NC * kClsStride) * 4, "tile classes alias the stages");
  static_assert(C::GT % (2 * C::NPROD) == 0, "a narrow tile's groups split evenly over the producers");
  __shared__ __attribute__((aligned(1024))) uint8_t s_lds[C::STAGES * C::STAGE];
  __shared__ int s_info[kTileInfo];
  int *s_rowstart = (int *)s_lds;
  int *s_cls = s_rowstart + kMaxGroups;

  const int tid = threadIdx.x, wave = tid >> 6;
  if (wave == 0) {
    DWM_TL(0, __builtin_amdgcn_s_memrealtime());
    DWM_TL(7, __builtin_amdgcn_s_memtime());
    DWM_TL(1, (uint32_t)__builtin_amdgcn_s_getreg(4 | (31 << 11)) |
                  ((uint64_t)(uint32_t)__builtin_amdgcn_s_getreg(20 | (31 << 11)) << 32));
  }
  // Every wave's exit (timeline build only).
  auto tl_exit = [&]() {
#ifdef DWTPU_TIMELINE
    __builtin_amdgcn_s_waitcnt(0);
    DWM_TL(8 + wave, __builtin_amdgcn_s_memrealtime());
    if (wave == 0) DWM_TL(20, __builtin_amdgcn_s_memtime());
#endif
  };
  const int go = group_offset ? group_offset[0] : 0;
  const int G = (N + 63) >> 6;
  const int n_tiles = (G + C::GT - 1) / C::GT;
  const int n_tiles_n = NARROW ? (G + C::GT / 2 - 1) / (C::GT / 2) : 0;
  TileRef ref;
  if (!find_tile<MB, 16, C::THREADS>(group_sizes, num_groups, go, e_local, M, n_tiles, n_tiles_n, ncu, bal,
                                     s_rowstart, s_cls, s_info, ref)) {
    tl_exit();
    return;
  }
  if (wave == 0) {
    DWM_TL(2, __builtin_amdgcn_s_memrealtime());
    DWM_TL(3, (uint32_t)ref.rows | ((uint32_t)ref.narrow << 16));
  }
  const int g = ref.g, nt = ref.nt, rows = ref.rows;
  const bool narrow = NARROW && ref.narrow;
  const int64_t row0 = ref.row0;
  const int64_t e = g - go;
  const int T = K >> 6, KB = K >> 7;
  const int g0 = nt * (narrow ? C::GT / 2 : C::GT);  // first 64-column group of the tile
  if (wave >= CW) {
    const int pw = wave - CW;
    const uint8_t *const wexp = wpk + e * G * T * 2048;
    const uint8_t *const sexp = spk + e * G * KB * 256;
    // Row groups pw + NP i with 8 (pw + NP i) < rows are loaded.
    const int na = min(C::A_LOADS, (rows + 8 * C::NPROD - 1 - 8 * pw) / (8 * C::NPROD));
    if (NARROW && narrow)
      ws_produce<C, C::G_LOADS / 2>(na, lhs, row_idx, lhs_rows, row0, rows, K, T, KB, wexp, sexp, g0, G, s_lds, pw);
    else
      ws_produce<C, C::G_LOADS>(na, lhs, row_idx, lhs_rows, row0, rows, K, T, KB, wexp, sexp, g0, G, s_lds, pw);
    DWM_GS(gs_role(1u | (uint64_t)rows << 8 | (uint64_t)narrow << 24);)
    tl_exit();
    return;
  }
  // Every consumer runs exactly T + 1 barriers (the producers' count),
  // whatever its row-block count.
  if (narrow && wave >= C::GT / 2) {
    ws_idle_consumer(T);
    DWM_GS(gs_role(3u | (uint64_t)rows << 8 | (uint64_t)narrow << 24);)
    tl_exit();
    return;
  }
  const int nh = (rows + 15) >> 4;  // 16-row blocks holding rows
  const int64_t col0 = (int64_t)(g0 + wave) * 64;
  const void *const bias = expert_bias(ep, e, N);
  switch (nh) {
    case 1: ws_consumer<C, 1, ACT>(T, s_lds, wave, row0, rows, col0, N, out, out_f32, bias, ep); break;
    case 2: ws_consumer<C, 2, ACT>(T, s_lds, wave, row0, rows, col0, N, out, out_f32, bias, ep); break;
    case 3: ws_consumer<C, 3, ACT>(T, s_lds, wave, row0, rows, col0, N, out, out_f32, bias, ep); break;
    case 4: ws_consumer<C, 4, ACT>(T, s_lds, wave, row0, rows, col0, N, out, out_f32, bias, ep); break;
    case 5: ws_consumer<C, 5, ACT>(T, s_lds, wave, row0, rows, col0, N, out, out_f32, bias, ep); break;
    default: ws_consumer<C, 6, ACT>(T, s_lds, wave, row0, rows, col0, N, out, out_f32, bias, ep); break;
  }
  DWM_GS(gs_role(2u | (uint64_t)rows << 8 | (uint64_t)narrow << 24);)
  tl_exit();
}

// zero_initialize: zero rows outside [start(go), start(go + E_local)).
__global__ __launch_bounds__(256) void gmm_zero_rows_kernel(const int32_t *group_sizes, int num_groups,
                                                            const int32_t *group_offset, int64_t e_local,
                                                            int64_t M, int64_t N, void *out,
                                                            int elem_bytes) {
  __shared__ int64_t s_lohi[2];
  const int lane = threadIdx.x & 63;
  if ((threadIdx.x >> 6) == 0) {
    const int go = group_offset ? group_offset[0] : 0;
    int64_t lo = 0, hi = 0;
    for (int base = 0; base < num_groups; base += 64) {
      const int g = base + lane;
      int sz = g < num_groups ? group_sizes[g] : 0;
      sz = sz > 0 ? sz : 0;
      lo += wave_sum(g < go ? sz : 0);
      hi += wave_sum((int64_t)g < (int64_t)go + e_local ? sz : 0);
    }
    if (lane == 0) {
      s_lohi[0] = lo;
      s_lohi[1] = hi;
    }
  }
  __syncthreads();
  const int64_t lo = s_lohi[0], hi = s_lohi[1];
  const int64_t r0 = (int64_t)blockIdx.x * 64;
  const int64_t row_words = N * elem_bytes / 4;  // N % 16 == 0: whole 32-bit words
  for (int64_t r = r0; r < r0 + 64 && r < M; ++r) {
    if (r >= lo && r < hi) continue;
    uint32_t *p = (uint32_t *)((char *)out + r * N * elem_bytes);
    for (int64_t i = threadIdx.x; i < row_words; i += blockDim.x) p[i] = 0u;
  }
}

int launch_gmm_zero_rows(const int32_t *group_sizes, int num_groups, const int32_t *group_offset, int64_t e_local,
                         int64_t M, int64_t n_out, void *out, int elem_bytes, hipStream_t st) {
  hipLaunchKernelGGL(gmm_zero_rows_kernel, dim3((unsigned)((M + 63) / 64)), dim3(256), 0, st, group_sizes, num_groups,
                     group_offset, e_local, M, n_out, out, elem_bytes);
  return launch_status("gmm zero rows");
}

// Compute units of the current device (looked up once per device).  It only
// sizes the narrow split; any positive value gives correct results.
static int device_cu_count() {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cache[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) {
    (void)hipGetLastError();
    return 256;
  }
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    n = 256;
  }
  cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

template <int MB, int CW, int JW, int NP, int NS, bool ACT, bool NARROW>
static int launch_gmm_ws(const uint16_t *lhs, const int32_t *row_idx, int64_t lhs_rows, int64_t M, int64_t K,
                         const uint8_t *w, const uint8_t *s,
                         const int32_t *gs, int ng, const int32_t *go, int64_t e_local, int64_t N, void *out,
                         int out_f32, const GmmEpilogue &ep, int ncu, int bal, hipStream_t st) {
  using C = WsCfg<MB, CW, JW, NP, NS>;
  constexpr int MT = 32 * MB, NT = C::NT, NC = 2 * MB;
  const int64_t n_tiles = (N + NT - 1) / NT;
  const int64_t max_tiles = ((M + MT - 1) / MT + e_local) * n_tiles;
  // Per XCD at most ceil(n_a / 8) tiles of each class: <= entries / 8 + NC,
  // where a narrow split keeps the entry count within ncu.
  const int64_t entries = NARROW ? std::max<int64_t>(max_tiles, ncu) : max_tiles;
  const int64_t grid = ((entries + 7) / 8 + NC) * 8;
  DWM_UNSUPPORTED_IF(grid > (1ll << 31) - 1, "gmm_fp4: too many tiles (%lld)", (long long)grid);
  DWM_UNSUPPORTED_IF(K > (1 << 24), "gmm_fp4: K <= 2^24 required");
  hipLaunchKernelGGL((gmm_fp4_ws_kernel<C, MB, ACT, NARROW>), dim3((unsigned)grid), dim3(C::THREADS), 0, st, lhs,
                     row_idx, lhs_rows, M, (int)K, w, s, gs, ng, go, e_local, (int)N, out, out_f32, ep, ncu, bal);
  return launch_status("gmm_fp4");
}

// Groups of 2 .. kGmmBalancedTiles row tiles split their rows evenly, and
// their row tiles of one column tile run side by side on one XCD (find_tile).
// DWTPU_GMM_BALANCED_TILES (read at every launch) sets another bound: 0 or 1
// balances no group, a bound past every group's tile count balances all of
// them (each group's row tiles of one column tile then run together, so the
// group's weight slice is read once per XCD).  Only the schedule changes:
// every row's result is the same.
constexpr int kGmmBalancedTiles = 4;

static int balanced_tiles() {
  const char *e = getenv("DWTPU_GMM_BALANCED_TILES");
  if (!e || !*e) return kGmmBalancedTiles;
  char *end = nullptr;
  const long v = strtol(e, &end, 10);
  return (*end == 0 && v >= 0 && v <= (1l << 30)) ? (int)v : kGmmBalancedTiles;
}

// The bf16 grouped matmul (arguments checked by the caller).
int launch_gmm_bf16(const uint16_t *lhs, const int32_t *row_idx, int64_t lhs_rows, int64_t M, int64_t K,
                    const uint8_t *weight, const uint8_t *scale, const int32_t *group_sizes, int num_groups,
                    const int32_t *group_offset, int64_t E_local, int64_t N, void *out, int out_f32, bool gated,
                    const GmmEpilogue &ep, hipStream_t st) {
  // 96-row x 512-column tiles, 8 consumer + 4 producer waves, four 64-deep
  // K stages (120 KB of LDS, under 168 VGPRs: one block of 12 waves per CU).
  // Measured fastest on the decode and prefill workloads among the tile,
  // wave-split and pipeline-depth variants tried.  The narrow-split kernel
  // is launched when even the fewest tiles M rows can make (every group
  // local and full) leave CUs idle; larger launches never split, and run the
  // kernel without the narrow producers.
  const int ncu = device_cu_count();
  const bool narrow = ((M + 95) / 96) * ((N + 511) / 512) < ncu;
#define DWM_GMM_WS(ACT, NARROW)                                                                                   \
  launch_gmm_ws<3, 8, 2, 4, 4, ACT, NARROW>(lhs, row_idx, lhs_rows, M, K, weight, scale, group_sizes, num_groups, \
                                             group_offset, E_local, N, out, out_f32, ep, ncu, balanced_tiles(), st)
  if (gated) return narrow ? DWM_GMM_WS(true, true) : DWM_GMM_WS(true, false);
  return narrow ? DWM_GMM_WS(false, true) : DWM_GMM_WS(false, false);
#undef DWM_GMM_WS
}

// Checks shared by every form of the grouped matmul, then the launch.
// lhs_fp4: the MX lhs is e2m1 codes [rows, K / 2] (MXFP4) instead of e4m3.
static int gmm_run(const dwm_gmm_lhs &L, int64_t M, int64_t K, const uint8_t *weight, const uint8_t *scale,
                   const void *bias, int bias_dtype, const int32_t *group_sizes, int num_groups,
                   const int32_t *group_offset, int64_t E_local, int64_t N, void *out, int out_dtype, int zero_init,
                   int fuse_act, void *stream, bool lhs_fp4 = false) {
  const bool mx = L.scale != nullptr;
  const char *const what = lhs_fp4 ? "gmm_fp4_mxfp4" : mx ? "gmm_fp4_mx" : (L.row_idx ? "gmm_fp4_gather" : "gmm_fp4");
  DWM_CHECK_ARG(M >= 0 && K > 0 && N > 0 && E_local >= 0 && num_groups >= 0 && L.rows >= 0,
                "%s: bad sizes M=%lld K=%lld N=%lld E_local=%lld groups=%d lhs_rows=%lld", what, (long long)M,
                (long long)K, (long long)N, (long long)E_local, num_groups, (long long)L.rows);
  DWM_CHECK_ARG(out_dtype == DWM_BF16 || out_dtype == DWM_F32, "%s: bad out dtype %d", what, out_dtype);
  DWM_CHECK_ARG(fuse_act >= DWM_ACT_NONE && fuse_act <= DWM_ACT_SWIGLUOAI, "%s: bad fuse_act %d", what, fuse_act);
  DWM_CHECK_ARG(!bias || bias_dtype == DWM_F32 || bias_dtype == DWM_BF16, "%s: bias dtype must be f32 or bf16", what);
  DWM_CHECK_ARG(L.row_idx || L.rows == M, "%s: without row_idx lhs must have M rows (%lld != %lld)", what,
                (long long)L.rows, (long long)M);
  DWM_UNSUPPORTED_IF(fuse_act != DWM_ACT_NONE && N % 64 != 0, "%s: fuse_act needs N %% 64 == 0 (N=%lld)", what,
                     (long long)N);
  DWM_UNSUPPORTED_IF(K % 128 != 0 || N % 16 != 0, "%s: K %% 128 == 0 and N %% 16 == 0 required", what);
  DWM_UNSUPPORTED_IF(num_groups > kMaxGroups, "%s: at most %d groups (got %d)", what, kMaxGroups, num_groups);
  DWM_UNSUPPORTED_IF(K > (1 << 24) || N > (1 << 30), "%s: K <= 2^24 and N < 2^30 required", what);
  if (M == 0) return DWM_OK;
  DWM_CHECK_ARG(L.data && out && (num_groups == 0 || group_sizes) && (!L.row_idx || L.rows > 0),
                "%s: null pointer or empty lhs with rows to read", what);
  // The MX kernels and the fused gather address lhs rows with 32-bit byte offsets.
  DWM_UNSUPPORTED_IF((mx || L.row_idx) && L.rows * K * (lhs_fp4 ? 1 : mx ? 2 : 4) >= (1ll << 33),
                     "%s: lhs of %lld rows is too large", what, (long long)L.rows);
  DWM_CHECK_ARG(E_local == 0 || (weight && scale), "%s: null weight pointer", what);
  DWM_CHECK_ARG((uintptr_t)L.data % 16 == 0 && (uintptr_t)weight % 16 == 0 && (uintptr_t)out % 16 == 0 &&
                    (uintptr_t)scale % 4 == 0 && (uintptr_t)L.scale % 4 == 0,
                "%s: lhs, weight and out must be 16-byte aligned, the scales 4-byte aligned", what);
  DWM_CHECK_ARG(!bias || (uintptr_t)bias % 4 == 0, "%s: bias must be 4-byte aligned", what);
  hipStream_t st = as_stream(stream);
  if (zero_init) {
    const int64_t n_out = fuse_act != DWM_ACT_NONE ? N / 2 : N;
    int rc = launch_gmm_zero_rows(group_sizes, num_groups, group_offset, E_local, M, n_out, out,
                                  out_dtype == DWM_F32 ? 4 : 2, st);
    if (rc != DWM_OK) return rc;
  }
  if (E_local == 0 || num_groups == 0) return DWM_OK;
  const GmmEpilogue ep{bias, bias && bias_dtype == DWM_BF16 ? 1 : 0, fuse_act};
  const int out_f32 = out_dtype == DWM_F32;
  const bool gated = fuse_act != DWM_ACT_NONE;
  if (mx)
    return launch_gmm_mx((const uint8_t *)L.data, L.scale, L.row_idx, L.rows, M, K, weight, scale, group_sizes,
                         num_groups, group_offset, E_local, N, out, out_f32, gated, ep, st, lhs_fp4);
  return launch_gmm_bf16((const uint16_t *)L.data, L.row_idx, L.rows, M, K, weight, scale, group_sizes, num_groups,
                         group_offset, E_local, N, out, out_f32, gated, ep, st);
}

}  // namespace dwm

using namespace dwm;

#ifdef DWTPU_TIMELINE
// Timeline build only: record the bf16 gmm kernel's per-wave step accounting
// for waves 0 .. waves - 1 (16 per block) into buf (waves x kGsSlots words,
// zeroed by the caller), or stop (NULL).
extern "C" int dwm_gmm_steps_set(uint64_t *buf, int64_t waves) {
  clear_error();
  DWM_CHECK_ARG(waves >= 0 && (buf || waves == 0), "gmm_steps_set: bad buffer");
  if (hipMemcpyToSymbol(HIP_SYMBOL(dwm::g_gmm_steps), &buf, sizeof(buf)) != hipSuccess ||
      hipMemcpyToSymbol(HIP_SYMBOL(dwm::g_gmm_steps_waves), &waves, sizeof(waves)) != hipSuccess)
    return launch_status("gmm_steps_set");
  return DWM_OK;
}

// Timeline build only: record the bf16 gmm kernel's blocks 0 .. blocks - 1
// into buf (blocks x kTlSlots words, zeroed by the caller), or stop (NULL).
extern "C" int dwm_timeline_set(uint64_t *buf, int64_t blocks) {
  clear_error();
  DWM_CHECK_ARG(blocks >= 0 && (buf || blocks == 0), "timeline_set: bad buffer");
  if (hipMemcpyToSymbol(HIP_SYMBOL(dwm::g_timeline), &buf, sizeof(buf)) != hipSuccess ||
      hipMemcpyToSymbol(HIP_SYMBOL(dwm::g_timeline_blocks), &blocks, sizeof(blocks)) != hipSuccess)
    return launch_status("timeline_set");
  return DWM_OK;
}
#endif

extern "C" int dwm_gmm_fp4_ex(const dwm_gmm_lhs *lhs, int64_t M, int64_t K, const uint8_t *weight,
                              const uint8_t *scale, const void *rhs_bias, int bias_dtype, const int32_t *group_sizes,
                              int num_groups, const int32_t *group_offset, int64_t E_local, int64_t N, void *out,
                              int out_dtype, int zero_init, int fuse_act, void *stream) {
  clear_error();
  DWM_CHECK_ARG(lhs, "gmm_fp4_ex: null lhs descriptor");
  return gmm_run(*lhs, M, K, weight, scale, rhs_bias, bias_dtype, group_sizes, num_groups, group_offset, E_local, N,
                 out, out_dtype, zero_init, fuse_act, stream);
}

extern "C" int dwm_gmm_fp4(const uint16_t *lhs, int64_t M, int64_t K, const uint8_t *weight,
                           const uint8_t *scale, const int32_t *group_sizes, int num_groups,
                           const int32_t *group_offset, int64_t E_local, int64_t N, void *out,
                           int out_dtype, int zero_init, int fuse_act, void *stream) {
  clear_error();
  const dwm_gmm_lhs L{lhs, nullptr, M, nullptr};
  return gmm_run(L, M, K, weight, scale, nullptr, 0, group_sizes, num_groups, group_offset, E_local, N, out,
                 out_dtype, zero_init, fuse_act, stream);
}

extern "C" int dwm_gmm_fp4_gather(const uint16_t *lhs, int64_t lhs_rows, const int32_t *row_idx, int64_t M,
                                  int64_t K, const uint8_t *weight, const uint8_t *scale,
                                  const int32_t *group_sizes, int num_groups, const int32_t *group_offset,
                                  int64_t E_local, int64_t N, void *out, int out_dtype, int zero_init, int fuse_act,
                                  void *stream) {
  clear_error();
  DWM_CHECK_ARG(lhs_rows >= 0 && M >= 0, "gmm_fp4_gather: bad sizes lhs_rows=%lld M=%lld", (long long)lhs_rows,
                (long long)M);
  DWM_CHECK_ARG(M == 0 || (row_idx && lhs_rows > 0), "gmm_fp4_gather: null row_idx or empty lhs with rows to gather");
  const dwm_gmm_lhs L{lhs, nullptr, lhs_rows, row_idx};
  return gmm_run(L, M, K, weight, scale, nullptr, 0, group_sizes, num_groups, group_offset, E_local, N, out,
                 out_dtype, zero_init, fuse_act, stream);
}

extern "C" int dwm_gmm_fp4_mxfp4(const uint8_t *lhs, const uint8_t *lhs_scale, int64_t lhs_rows,
                                 const int32_t *row_idx, int64_t M, int64_t K, const uint8_t *weight,
                                 const uint8_t *scale, const void *rhs_bias, int bias_dtype,
                                 const int32_t *group_sizes, int num_groups, const int32_t *group_offset,
                                 int64_t E_local, int64_t N, void *out, int out_dtype, int zero_init, int fuse_act,
                                 void *stream) {
  clear_error();
  DWM_CHECK_ARG(lhs_scale || M == 0, "gmm_fp4_mxfp4: null lhs_scale");
  const dwm_gmm_lhs L{lhs, lhs_scale ? lhs_scale : (const uint8_t *)lhs, lhs_rows, row_idx};
  return gmm_run(L, M, K, weight, scale, rhs_bias, bias_dtype, group_sizes, num_groups, group_offset, E_local, N,
                 out, out_dtype, zero_init, fuse_act, stream, true);
}

extern "C" int dwm_gmm_fp4_mx(const uint8_t *lhs, const uint8_t *lhs_scale, int64_t lhs_rows, const int32_t *row_idx,
                              int64_t M, int64_t K, const uint8_t *weight, const uint8_t *scale,
                              const int32_t *group_sizes, int num_groups, const int32_t *group_offset, int64_t E_local,
                              int64_t N, void *out, int out_dtype, int zero_init, int fuse_act, void *stream) {
  clear_error();
  DWM_CHECK_ARG(lhs_scale || M == 0, "gmm_fp4_mx: null lhs_scale");
  const dwm_gmm_lhs L{lhs, lhs_scale ? lhs_scale : (const uint8_t *)lhs, lhs_rows, row_idx};
  return gmm_run(L, M, K, weight, scale, nullptr, 0, group_sizes, num_groups, group_offset, E_local, N, out,
                 out_dtype, zero_init, fuse_act, stream);
}
