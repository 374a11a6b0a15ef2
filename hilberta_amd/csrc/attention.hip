// Block-sparse flash-attention forward for HilbertA block tables on gfx950 (MI355X).
//
// Replaces the Triton kernels _paired_fwd (reference hilberta/paired_kernel.py:18-94) and
// _block_sparse_fwd (hilberta/sparse_kernel.py:28-97) with one hand-written CDNA4 kernel:
//
//  * Work item = one query tile (256 queries for quad tables, 128 for paired tables, 64 for
//    unpaired ones) of one (batch, head), or one chunk of a global (text) query tile's all-key
//    sweep.  Global tiles are split into at most MAX_SPLIT chunks of about a workgroup's average
//    work (at least two for sweeps of four rows or more), none shorter than the longest ordinary
//    row or MIN_CHUNK steps, so no item dominates the schedule; chunk
//    partials (unnormalised accumulator, running max, row sum) go to the workspace and
//    merge_kernel combines them after the main kernel.
//  * Persistent workgroups (2 per CU; 3 for paired D = 64 calls with enough items; 1 eight-wave
//    workgroup per CU for quad tables) claim items
//    from 8 work queues, one per XCD (queue x = blockIdx % 8, the XCD under round-robin dispatch,
//    owns a contiguous range of the item list), so items that share K/V blocks run under one L2;
//    idle workgroups steal from other queues, skipping those a drained-queue mask marks empty.
//    Each workgroup's first two items are dealt out without atomics; later claims run one item
//    ahead, and the next item's table entries, first K/V block and Q tile are prefetched while
//    the current item finishes.
//  * Per 64-key block: the K and V tiles stream from HBM straight into one of two LDS stages
//    (buffer loads to LDS, 16 bytes per lane, rows unpadded with an XOR chunk swizzle); the next
//    block's loads are in flight while the current block is computed.  Table entries that neither
//    query half may see are never loaded.
//  * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16: each lane then
//    holds 16 keys of ONE query, so the online-softmax row max is an in-lane max plus one
//    cross-half exchange (v_permlane32_swap), and the output O^T = V^T P^T takes the score
//    registers directly as the B operand; its A operand (V^T) comes out of LDS already
//    transposed through ds_read_b64_tr_b16.
//  * Each wave owns 32 queries; in paired mode waves 0-1 own query half 0 and waves 2-3 half 1;
//    with quad tables (two paired rows merged, flag bit = 64-query block 0..3) waves 2b and
//    2b + 1 own query block b, and the eight waves share each staged K/V tile, so a tile costs
//    half the load instructions and LDS writes per MFMA of a paired item.
//    A block that the flag test (flags >> (half + 2*key_half)) & 1 of paired_kernel.py:65,83-84
//    hides from a wave's half is computed but masked (P = 0), which keeps one code path (a
//    wave-uniform branch around the masked case measured slower, and with this compiler it
//    spills about 280 VGPRs to scratch: the step's state stays live across both paths).
//  * Online softmax in exp2 with fp32 state (paired_kernel.py:82-93) and a lazy rescale; P is
//    rounded to the input type before the PV product and summed unrounded into the row
//    normaliser, as in the reference; an optional fp32 per-row logsumexp (natural log) is written
//    as well.
#include <mutex>

#include "common.h"
#include "../../include/hilberta_hip.h"

namespace hb {
namespace {

constexpr int KEYS = 64;     // keys per staged block
constexpr float LN2 = 0.69314718055994530942f;
constexpr int QUEUES = 8;    // one work queue per XCD
constexpr float RESCALE_LOG2 = 8.0f;  // lazy-rescale threshold (log2 units)
constexpr int MAX_SPLIT = 16;  // chunks per global query tile, at most
constexpr int NOMINAL_GROUPS = 512;  // persistent workgroups on a full MI355X (2 per CU)
constexpr int MIN_CHUNK = 64;  // key-block steps per global chunk, at least (shorter chunks' fixed costs show)
// V operands (ds_read_b64_tr_b16 pairs) in flight ahead of the PV MFMAs: three cover the LDS
// latency under load better than two (2-3 % at 2048 px 16-tile K3), four a little better again
// (0.2-1 % at every configuration, no spills; bitwise-identical results)
constexpr int PFV = 4;
// word 3 of a raw buffer resource (32-bit data format, no swizzle), as for gfx9-family buffers
constexpr int BUFFER_WORD3 = 0x00020000;
// __builtin_amdgcn_sched_group_barrier instruction classes
constexpr int SG_MFMA = 0x008;
constexpr int SG_DS_READ = 0x100;

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  // element strides (b, h, n) of Q, K, V, O; 32-bit (checked on the host) to save scalar registers
  int32_t q_sb, q_sh, q_sn, k_sb, k_sh, k_sn, v_sb, v_sh, v_sn, o_sb, o_sh, o_sn;
  const int32_t* indices;
  const int32_t* flags;
  const int32_t* counts;
  int32_t heads, tokens, global_tokens, bh, width, rows, key_blocks;
  int32_t global_tiles, nsplit, chunk, per_bh;
  float scale_log2;
  int32_t* counters;  // [0, 8) queue heads, [8] exit count, [9] drained-queue mask; zero between launches
  float* part;        // split partial accumulators, fragment order
  float* part_ml;     // split partial (max, sum) per query lane
};

template <bool F16>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (F16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
}

// Round 8 fp32 values to the input type (round to nearest even) and pack them.
template <bool F16>
__device__ __forceinline__ u32x4 pack8(f32x8 x) {
  if constexpr (F16) {
    return __builtin_bit_cast(u32x4, __builtin_convertvector(x, f16x8));
  } else {
    return __builtin_bit_cast(u32x4, __builtin_convertvector(x, bf16x8));
  }
}

template <bool F16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (F16) {
    _Float16 h[2] = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
  } else {
    __bf16 h[2] = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, h);
  }
}

// x combined with the value held by the lane 32 positions away: v_permlane32_swap exchanges the
// two 32-lane halves of a register (no LDS round trip); of its two results, each lane holds its
// own value in one and its partner's in the other.
__device__ __forceinline__ float pair_max(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  // copied out first: this compiler lowers a bit cast of a vector element to element 0
  const unsigned r0 = r[0], r1 = r[1];
  return fmaxf(__builtin_bit_cast(float, r0), __builtin_bit_cast(float, r1));
}
__device__ __forceinline__ float pair_sum(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const unsigned r0 = r[0], r1 = r[1];
  return __builtin_bit_cast(float, r0) + __builtin_bit_cast(float, r1);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef __attribute__((address_space(3))) void* lds_ptr;

// 16 bytes per lane from base + voffset + soffset (bytes) into LDS at dst + 16 * lane, as a
// buffer load to LDS over a raw buffer at base.  The buffer resource type exists only for the
// device target, so the host pass (which compiles the kernels' launch stubs) sees an empty body.
__device__ __forceinline__ void buffer_load_lds16(const void* base, uint16_t* dst, int voffset,
                                                  int soffset) {
#if defined(__HIP_DEVICE_COMPILE__)
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, BUFFER_WORD3);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_ptr)dst, 16, voffset, soffset, 0, 0);
#endif
}

// Entry i of a table row of `width` int32 entries, or 0 past its end: a raw buffer load, whose
// range check returns 0 out of range, addressed by a scalar base and a 32-bit lane offset (no
// per-lane 64-bit pointer to keep in vector registers).
__device__ __forceinline__ int row_entry(const int32_t* row, int width, int i) {
#if defined(__HIP_DEVICE_COMPILE__)
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int32_t*>(row), 0, width * 4, BUFFER_WORD3);
  return __builtin_amdgcn_raw_buffer_load_b32(rsrc, i * 4, 0, 0);
#else
  return 0;
#endif
}

// Chunk permutation of K/V row r in LDS (16-byte chunks, CPR per row): XOR with a row-dependent
// value so that the K reads (8 consecutive rows, one 16-byte chunk each) and the transposing V
// reads (4 consecutive rows, 4 neighbouring chunks each per 32 lanes) hit distinct banks.
template <int CPR>
__device__ __forceinline__ int swz(int r) {
  if constexpr (CPR == 16) return 4 * (r & 3) + ((r >> 2) & 3);
  else return (4 * ((r >> 1) & 1) + ((r >> 2) & 3)) & 7;
}

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i%4 of the 4-element
// (8-byte) words addressed by lanes i/4, i/4 + 4, i/4 + 8, i/4 + 12.
__device__ __forceinline__ u32x2 read_tr(const uint16_t* p) {
  typedef short i16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)p));
}

// Paired workgroups (four waves, one per SIMD) per CU, i.e. waves per SIMD: two for D = 128 (64 KiB
// of K/V stages, about 250 registers per lane), three for D = 64 (32 KiB of stages, at most 168
// registers).  Against two, three made D = 64 calls 5-9 % faster at 2048 and 4096 px.
//  Quad workgroups (eight waves) fill a CU alone at two waves per SIMD.
template <int HALVES, int D>
constexpr int groups_per_cu() { return HALVES == 4 ? 1 : (HALVES == 2 && D == 64 ? 3 : 2); }

template <int HALVES, int D, int KBR, bool F16>
__global__ __launch_bounds__(128 * HALVES, (HALVES == 2 ? groups_per_cu<HALVES, D>() : 1)) void attn_fwd_kernel(AttnArgs a) {
  static_assert(HALVES == 1 || HALVES == 2 || (HALVES == 4 && KBR == 1), "quad tables use 64-key blocks");
  constexpr int WAVES = 2 * HALVES;             // waves per workgroup, 32 queries each
  constexpr int QT = 64 * HALVES;               // queries per work item
  constexpr int NG = 1;                         // 32-query groups per wave
  constexpr int QW = 32 * NG;                   // queries per wave
  constexpr int VW = WAVES * NG;                // 32-query groups per item
  constexpr int CPR = D / 8;                    // 16-byte chunks per K/V row
  constexpr int TILE = KEYS * D;                // elements of one K (or V) tile
  constexpr int STAGE = 2 * TILE;               // K tile then V tile
  constexpr int DT = D / 32;                    // output 32-dim tiles
  constexpr int DS = D / 16;                    // contraction steps over D
  constexpr int FRAG = DT * 16 * 64;            // partial accumulator floats per wave
  static_assert(CPR % WAVES == 0 || WAVES % CPR == 0, "tile loads must split over the waves");

  // Two stages of [K tile | V tile], both row-major (key rows of D elements) with the 16-byte
  // chunks of row r permuted by chunk ^ swz(r); written by direct global->LDS loads.
  __shared__ __attribute__((aligned(1024))) uint16_t lds0[STAGE];
  __shared__ __attribute__((aligned(1024))) uint16_t lds1[STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Two waves share each SIMD, and with equal priorities they tend to reach the MFMA and softmax
  // phases together; a higher issue priority for one of them lets it run ahead.  With two
  // workgroups per CU the upper half of the persistent grid takes it (5-7 % faster at 2048 px
  // 16-tile K3, measured against the symmetric kernel in one process; neutral on dense tables),
  // and a workgroup whose claim finds every queue drained gives it up for its last item (see
  // `step`).  An eight-wave quad workgroup holds both waves of each SIMD (waves w and w + 4
  // under round-robin placement): its upper four waves take it.
  if (HALVES != 4 && blockIdx.x >= gridDim.x / 2) __builtin_amdgcn_s_setprio(1);
  // wave index as a provably uniform (scalar) value, so per-wave tests such as the flag check
  // compile to branches rather than exec-masked code
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (HALVES == 4 && wave >= 4) __builtin_amdgcn_s_setprio(1);
  // query block (64 queries) of this wave: the flag bit it tests
  const int half = HALVES >= 2 ? (wave * QW) / 64 : 0;
  // flags of a block every query block of the item sees (global chunks)
  constexpr int ALL_FLAGS = HALVES == 4 ? 15 : 3;
  const int ql = lane & 31;   // query (column) owned by this lane inside the wave's 32
  const int hl = lane >> 5;   // lane half: selects the 8-element k slice of MFMA operands

  // ------------------------------------------------------------------ persistent work queues
  // Item codes: [0, total_g) are the chunks of global query tiles ((batch, head)-major, then tile,
  // then chunk), [total_g, total_g + total_r) the ordinary rows ((batch, head)-major).  Queue x
  // (= blockIdx % 8, the XCD of the round-robin dispatch) owns the x-th eighth of each list, so
  // the items running on one XCD share heads and neighbouring K/V tiles in its L2, and hands out
  // its global chunks first (longest items first), then its rows.  The first 2*w items of a
  // queue served by w workgroups are dealt out without atomics, items r and r + w to the
  // workgroup of rank r (all workgroups hitting eight counters at once at the launch would
  // serialise there); later items are claimed with the queue's atomic counter, and a workgroup
  // whose queue is empty steals from the others.  The claim for the item after next is issued
  // at the top of an item's last step, right after the next item's first K/V loads, so its round
  // trip (a few thousand cycles: device-scope atomics go past the L2) overlaps that whole step,
  // and it is read at the top of the next item's first step (its table entries are loaded during
  // that step).  The library builds this file without the compiler's atomic optimizer, which
  // would turn the single-lane atomic into a wave-aggregated one that waits for its result right
  // where it is issued.  The last workgroup to leave resets the counters.  The queue count is a constant, so the queue
  // arithmetic is shifts and masks (a grid of fewer than eight workgroups leaves some queues
  // without workgroups of their own; their items are stolen).
  __shared__ int s_claim[2];
  constexpr int nq = QUEUES;
  const int qx = blockIdx.x % nq;
  const int gper = a.global_tiles * a.nsplit;  // global chunks per (batch, head)
  const int total_g = a.bh * gper;
  const int total_r = a.bh * a.rows;
  auto g_lo = [&](int q) { return (int)((int64_t)total_g * q / nq); };
  auto r_lo = [&](int q) { return (int)((int64_t)total_r * q / nq); };
  // tid 0 only: code of the c-th item of queue q, or -1 past its end
  auto item_of = [&](int q, int c) {
    const int gl = g_lo(q + 1) - g_lo(q);
    if (c < gl) return g_lo(q) + c;
    c -= gl;
    return c < r_lo(q + 1) - r_lo(q) ? total_g + r_lo(q) + c : -1;
  };
  // workgroups serving queue q, whose first 2 * dealt(q) items are dealt out
  auto dealt = [&](int q) { return ((int)gridDim.x - q + nq - 1) / nq; };
  // When every queue's items are all dealt out (small problems), there is nothing to claim: no
  // atomics at all, rather than one per queue per workgroup to find every queue empty.
  const bool all_dealt =
      2 * ((int)gridDim.x / nq) >= (total_g + nq - 1) / nq + (total_r + nq - 1) / nq;
  // tid 0 only: code of a claimed item (counter value first_count of this workgroup's queue), or
  // -1 when every queue is drained.
  auto claim_from = [&](int first_count) {
    if (all_dealt) return -1;
    const int own = item_of(qx, 2 * dealt(qx) + first_count);
    if (own >= 0) return own;
    // The own queue is drained: mark it in the launch's drained-queue mask and skip the queues
    // already marked, so the claim that finds every queue empty takes two round trips, not eight.
    unsigned* mask = (unsigned*)&a.counters[QUEUES + 1];
    const unsigned drained = atomicOr(mask, 1u << qx);
    for (int t = 1; t < nq; ++t) {
      const int q = (qx + t) % nq;
      if ((drained >> q) & 1) continue;
      const int c = item_of(q, 2 * dealt(q) + atomicAdd(&a.counters[q], 1));
      if (c >= 0) return c;
    }
    return -1;
  };
  if (tid == 0) {
    // ranks rotated by half: the first items of a queue (its global chunks, the longest) go to
    // the upper half of the grid, which issues at the higher priority (0.3-3 % faster, most at
    // 1024 px 16-tile K3; bitwise identical)
    const int rank = ((int)blockIdx.x / nq + dealt(qx) / 2) % dealt(qx);
    int i0 = item_of(qx, rank), i1 = item_of(qx, rank + dealt(qx));
    // a queue shorter than its dealt share: claim (steal) instead, unless every item is dealt
    if (i0 < 0 && !all_dealt) i0 = claim_from(atomicAdd(&a.counters[qx], 1));
    if (i1 < 0 && !all_dealt) i1 = claim_from(atomicAdd(&a.counters[qx], 1));
    s_claim[0] = i0;
    s_claim[1] = i1;
  }
  __syncthreads();

  struct Item {
    int valid, bh, b, h, global, qfirst, row, gtile, split, first_block, nsteps;
  };
  auto decode = [&](int idx) {
    Item it;
    it.valid = idx >= 0;
    const int i = it.valid ? idx : 0;
    it.global = i < total_g;
    it.row = 0;
    it.gtile = 0;
    it.split = 0;
    it.first_block = 0;
    if (it.global) {
      it.bh = i / gper;
      const int rem = i - it.bh * gper;
      it.gtile = rem / a.nsplit;
      it.split = rem - it.gtile * a.nsplit;
      it.qfirst = it.gtile * QT;
      it.first_block = it.split * a.chunk;
      it.nsteps = min(a.chunk, a.key_blocks - it.first_block);
    } else {
      const int ri = i - total_g;
      it.bh = ri / a.rows;
      it.row = ri - it.bh * a.rows;
      it.qfirst = a.tokens - (a.rows - it.row) * QT;  // ordinary rows follow the global prefix
      it.nsteps = 0;  // from the row count, loaded with the item's table entries
    }
    it.b = it.bh / a.heads;
    it.h = it.bh - it.b * a.heads;
    return it;
  };
  // First 64 table entries (lane i holds entry i) and the entry count of a row item.
  auto load_meta = [&](const Item& it, int& cnt, int& t_id, int& t_fl) {
    cnt = 0;
    t_id = 0;
    t_fl = 0;
    if (!it.valid || it.global) return;
    const int64_t row = (int64_t)it.row * a.width;
    cnt = a.counts[it.row];
    t_id = row_entry(a.indices + row, a.width, lane);
    if (HALVES >= 2) t_fl = row_entry(a.flags + row, a.width, lane);
  };

  Item cur = decode(uniform(s_claim[0]));
  int nxt_idx = uniform(s_claim[1]);  // next item, decoded only when it becomes current
  int c_cnt, t_id, t_fl, n_cnt, n_id, n_fl;
  load_meta(cur, c_cnt, t_id, t_fl);
  load_meta(decode(nxt_idx), n_cnt, n_id, n_fl);
  if (!cur.global) cur.nsteps = max(uniform(c_cnt), 1) * KBR;
  int tbase = 0;
  int pending = 0;       // tid 0: raw counter value of the claim in flight
  bool claiming = false; // a claim was issued at the last item boundary

  // Block index and per-half permission bits (bit h: query half h may see it) of step s of the
  // current item.  Table entries live in lane registers; a step reads its entry with v_readlane,
  // refilling 64 entries at a time for rows longer than 64 entries.
  auto step_info = [&](int s, int& kb, int& fl) {
    if (cur.global) {
      kb = cur.first_block + s;
      fl = ALL_FLAGS;
      return;
    }
    const int e = s / KBR;
    const int sub = s - e * KBR;
    if (e >= tbase + 64) {
      tbase = e & ~63;
      const int64_t row = (int64_t)cur.row * a.width;
      t_id = row_entry(a.indices + row, a.width, tbase + lane);
      t_fl = HALVES >= 2 ? row_entry(a.flags + row, a.width, tbase + lane) : 0;
      // Wait here, inside the refill branch, for the entries read just below: left pending past
      // the branch, the waitcnt pass would stall the next LDS reads on every path (vmcnt(0)).
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    }
    kb = __builtin_amdgcn_readlane(t_id, e - tbase) * KBR + sub;
    if constexpr (HALVES == 4) fl = __builtin_amdgcn_readlane(t_fl, e - tbase) & 15;
    else fl = HALVES == 2 ? (__builtin_amdgcn_readlane(t_fl, e - tbase) >> (2 * sub)) & 3 : 1;
  };
  // First step at or after s that some query half may see.  With one step per table entry every
  // entry qualifies (paired entries carry at least one flag bit), so only 128-key blocks (two
  // steps per entry, one of which may be hidden from both halves) need the search.
  auto next_live = [&](int s) {
    if (KBR == 1) return s;
    for (; s < cur.nsteps; ++s) {
      int kb, fl;
      step_info(s, kb, fl);
      if (fl) break;
    }
    return s;
  };

  u32x4 qreg[NG][DS];
  auto load_q = [&](const Item& it) {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      // (a paired row's first item may start 64 queries before token 0 when G = 0 and the
      // ordinary query count is an odd multiple of 64: that half is never stored, and loads the
      // queries of token 0 instead)
      const int qi = max(it.qfirst + wave * QW + g * 32 + ql, 0);
      const uint16_t* qp = a.q + (int64_t)it.b * a.q_sb + (int64_t)it.h * a.q_sh +
                           (int64_t)qi * a.q_sn + hl * 8;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) qreg[g][ds] = *(const u32x4*)(qp + ds * 16);
    }
  };

  // Stage the K and V tiles of 64-key block kb: wave instruction i covers rows 64*i/CPR.. (64
  // lanes x 16 bytes = one contiguous KiB of LDS); lane l of it fetches the global chunk that the
  // swizzle places at LDS slot 64*i + l.  The loads are buffer loads to LDS (MUBUF, counted on
  // vmcnt only, so the LDS reads that follow keep exact lgkmcnt waits) over a raw buffer of the
  // (batch, head) K or V rows; the per-lane byte offsets inside a block are fixed, the block
  // offset goes in soffset.  The loads complete asynchronously; the top of the next step waits.
  constexpr int NDMA = (CPR + WAVES - 1) / WAVES;
  // When one round of the waves' instructions covers a multiple of 16 rows, the swizzle repeats
  // and instruction n's lane offsets are instruction 0's plus a uniform row offset, which goes
  // in soffset: one offset register per tile instead of NDMA.
  constexpr int ROWS_PER_ROUND = WAVES * 64 / CPR;
  constexpr bool DMA_LINEAR = ROWS_PER_ROUND % 16 == 0;
  constexpr int NOFF = DMA_LINEAR ? 1 : NDMA;
  int dk[NOFF], dv[NOFF];
#pragma unroll
  for (int n = 0; n < NOFF; ++n) {
    const int slot = (n * WAVES + wave) * 64 + lane;
    const int r = slot / CPR;
    const int c = (slot % CPR) ^ swz<CPR>(r);
    dk[n] = (int)(r * a.k_sn + c * 8) * 2;
    dv[n] = (int)(r * a.v_sn + c * 8) * 2;
  }
  // K and V rows of one (batch, head), computed once per item
  auto k_base = [&](const Item& it) { return a.k + (int64_t)it.b * a.k_sb + (int64_t)it.h * a.k_sh; };
  auto v_base = [&](const Item& it) { return a.v + (int64_t)it.b * a.v_sb + (int64_t)it.h * a.v_sh; };
  const int kblk_bytes = KEYS * (int)a.k_sn * 2, vblk_bytes = KEYS * (int)a.v_sn * 2;
  const int kround_bytes = ROWS_PER_ROUND * (int)a.k_sn * 2;
  const int vround_bytes = ROWS_PER_ROUND * (int)a.v_sn * 2;
  auto dma_block = [&](uint16_t* stage, const uint16_t* kbase, const uint16_t* vbase, int kb) {
    const int sk = kb * kblk_bytes, sv = kb * vblk_bytes;
    // The wave index enters the LDS destinations through an opaque copy, so each launch rebuilds
    // them with scalar adds; left visible, the compiler hoists all 16 destinations of both stages
    // out of the loop and, short of scalar registers, reloads them from VGPR lanes every step.
    int w = wave;
    asm volatile("" : "+s"(w));
#pragma unroll
    for (int n = 0; n < NDMA; ++n) {
      const int i = n * WAVES + w;
      if (CPR % WAVES == 0 || i < CPR) {
        const int o = DMA_LINEAR ? 0 : n;
        const int rk = DMA_LINEAR ? n * kround_bytes : 0, rv = DMA_LINEAR ? n * vround_bytes : 0;
        buffer_load_lds16(kbase, stage + i * 512, dk[o], sk + rk);
        buffer_load_lds16(vbase, stage + TILE + i * 512, dv[o], sv + rv);
      }
    }
  };

  // Per-lane LDS element offsets of the MFMA operands (the key-tile and 16-key-step parts are
  // compile-time offsets added at the read):
  //  K (A of S^T = K Q^T): row ql, chunk 2*ds + hl, for each d-step ds.
  //  V (A of O^T = V^T P^T, two transposing reads of 4 keys each): lane (g, j, t) = (lane/16,
  //  lane%16/4, lane%4) addresses keys 4*hl + j (+8 for the second read) at dims
  //  32*dt + 16*(g&1) + 4*t; ds_read_b64_tr_b16 then hands lane l the 4 keys at dim 32*dt + ql.
  int koff[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) koff[ds] = ql * D + (((2 * ds + hl) ^ swz<CPR>(ql)) << 3);
  int voff[DT][2];
  {
    const int g = lane >> 4, j = (lane >> 2) & 3, t = lane & 3;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        const int row = 4 * hl + j + 8 * rb;
        const int d = 32 * dt + 16 * (g & 1) + 4 * t;
        voff[dt][rb] = row * D + (((d >> 3) ^ swz<CPR>(row)) << 3) + (d & 7);
      }
  }

  f32x16 acc[NG][DT];
  float m_run[NG], l_run[NG];
#pragma unroll
  for (int g = 0; g < NG; ++g) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[g][dt] = f32x16{};
    m_run[g] = -__builtin_inff();
    l_run[g] = 0.f;
  }

  // Output of a finished item, packed in the input type, held until it is stored.  The stores of
  // an item are deferred to the next item's first step, after its barrier: the hand-over waits
  // for the next item's loads, and vector memory operations complete in issue order, so stores
  // issued at the hand-over would hold up that wait and the step barrier's fence behind them.
  // The address of a lane's output row is the item's (uniform) base plus a lane offset that
  // never changes, so the pending state costs the packed values and the LSE only.  With 128-key
  // blocks the extra registers would spill, and the D = 64 kernel keeps to 168 registers for
  // three waves per SIMD, so those store at the epilogue.
  static_assert(NG == 1, "one pending output tile per wave");
  constexpr bool DEFER_OUTPUT = KBR == 1 && (HALVES == 4 || groups_per_cu<HALVES, D>() == 2);
  const int o_lane = (wave * QW + ql) * a.o_sn + hl * 8;
  const int l_lane = wave * QW + ql;
  u32x2 ow[DT][4];
  uint16_t* o_item = nullptr;
  float* l_item = nullptr;
  float l_val = 0.f;
  bool out_pending = false;
  auto flush_output = [&]() {
    if (!out_pending) return;
    out_pending = false;
    // Lanes l and l + 32 hold the two 8-byte halves of each 16-byte chunk of a row: one swap
    // per pair of chunks hands lane l the whole even chunk and lane l + 32 the whole odd one, so
    // each lane stores 16 bytes and a store covers 32 bytes of each of the wave's 32 rows.
    uint16_t* op = o_item + o_lane;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int gp = 0; gp < 2; ++gp) {
        const u32x2 ea = ow[dt][2 * gp], ob = ow[dt][2 * gp + 1];
        const auto x = __builtin_amdgcn_permlane32_swap(ea[0], ob[0], false, false);
        const auto y = __builtin_amdgcn_permlane32_swap(ea[1], ob[1], false, false);
        const unsigned x0 = x[0], x1 = x[1], y0 = y[0], y1 = y[1];
        *(u32x4*)(op + dt * 32 + gp * 16) = u32x4{x0, y0, x1, y1};
      }
    if (l_item && hl == 0) l_item[l_lane] = l_val;
  };

  // Epilogue of the current item: normalised output (and LSE), held for flush_output, or, for a
  // chunk of a split global tile, its partial (unnormalised acc, max, sum) in fragment order,
  // stored here; merge_kernel combines the chunks after this kernel (the kernel boundary makes
  // every partial visible on every XCD).
  auto epilogue = [&]() {
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      const float l_tot = pair_sum(l_run[g]);
      if (!cur.global || a.nsplit == 1) {
        // 32 queries outside the item's own range (the half of a paired row that reaches into the
        // global prefix, or of the last global tile past it) are computed but not stored
        const int q0 = cur.qfirst + wave * QW + g * 32;
        if (cur.global ? q0 >= a.global_tokens : q0 < a.global_tokens) continue;
        const float inv = 1.f / l_tot;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq)
            ow[dt][gq] = u32x2{pack2<F16>(acc[g][dt][gq * 4 + 0] * inv, acc[g][dt][gq * 4 + 1] * inv),
                               pack2<F16>(acc[g][dt][gq * 4 + 2] * inv, acc[g][dt][gq * 4 + 3] * inv)};
        o_item = a.o + (int64_t)cur.b * a.o_sb + (int64_t)cur.h * a.o_sh + (int64_t)cur.qfirst * a.o_sn;
        l_item = a.lse ? a.lse + (int64_t)cur.bh * a.tokens + cur.qfirst : nullptr;
        l_val = (m_run[g] + __log2f(l_tot)) * LN2;
        out_pending = true;
        if constexpr (!DEFER_OUTPUT) flush_output();
        continue;
      }
      // partial slots: (tile, chunk)-major, then the item's 32-query group wave * NG + g
      const int tile = cur.bh * a.global_tiles + cur.gtile;
      const int64_t slot = ((int64_t)tile * a.nsplit + cur.split) * VW + wave * NG + g;
      float* pa = a.part + slot * FRAG;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) pa[(dt * 16 + i) * 64 + lane] = acc[g][dt][i];
      float* pml = a.part_ml + slot * 128;
      pml[lane] = m_run[g];
      pml[64 + lane] = l_tot;
    }
  };

  // ------------------------------------------------------------------ main loop
  // Every item starts at its step 0 with that step's own flags (a 128-key entry whose first half
  // neither query half sees is then computed fully masked).  The K/V prefetch runs one step
  // ahead across item boundaries, and the next item's Q is loaded right after the last score
  // MFMAs of the current item.
  const uint16_t* cur_k = k_base(cur);
  const uint16_t* cur_v = v_base(cur);
  // block and flags of the current step, computed while the step before it issued their loads
  int c_kb = 0, c_fl = 0;
  if (cur.valid) {
  load_q(cur);
  step_info(0, c_kb, c_fl);
  dma_block(lds0, cur_k, cur_v, c_kb);
  int s = 0;
  // One step on `stage` while the next block streams into `other`.  The two stages are distinct
  // LDS arrays and the loop below alternates them at compile time, so the compiler can see that
  // reads of `stage` never alias the loads in flight into `other`.  Returns true when done.
  auto step = [&](uint16_t* __restrict__ stage, uint16_t* __restrict__ other) -> bool {
    const int fl = c_fl;
    if (claiming && tid == 0) s_claim[0] = claim_from(pending);
    // every wave's loads of this stage have landed (each wave waits for its own, then the
    // barrier), and every wave is done reading the other stage, which the next block's loads may
    // now overwrite
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    const int sn = next_live(s + 1);
    const bool cross = sn >= cur.nsteps;
    // The claimed item's table entries are loaded after this step's tile loads and output
    // stores, where the held output registers are free, unless this step already crosses to it.
    const bool meta_late = claiming && !cross;
    if (claiming) {
      claiming = false;
      nxt_idx = uniform(s_claim[0]);
      // Every queue is drained, so this item is the workgroup's last: back to the base priority,
      // so a workgroup of the same CU still running its own last items is not held back by it
      // (4 % faster at 1024 px, where every item is dealt out and the second is the last, 1.5-2 %
      // on dense tables, 0.5-1.3 % at 2048 px 16-tile K3; bitwise identical).
      // (A quad workgroup has the CU to itself and keeps its waves' asymmetry.)
      if (HALVES != 4 && nxt_idx < 0) __builtin_amdgcn_s_setprio(0);
      if (!meta_late) load_meta(decode(nxt_idx), n_cnt, n_id, n_fl);
    }
    if (!cross) {
      step_info(sn, c_kb, c_fl);
      dma_block(other, cur_k, cur_v, c_kb);
    } else if (nxt_idx >= 0) {
      // step 0 of the next item: a global chunk's blocks are seen by both query halves; a row's
      // first entry carries its own flags (tables without a global prefix, or G = 0, may start
      // with an entry only one half sees), sub-step 0 of it for 128-key blocks
      const Item nxt = decode(nxt_idx);
      c_kb = nxt.global ? nxt.first_block : __builtin_amdgcn_readlane(n_id, 0) * KBR;
      c_fl = nxt.global ? ALL_FLAGS
                        : (HALVES >= 2 ? __builtin_amdgcn_readlane(n_fl, 0) & ALL_FLAGS : 1);
      dma_block(other, k_base(nxt), v_base(nxt), c_kb);
      // the claim for the item after next: its round trip overlaps this step (read at the next
      // item's first step, after the hand-over's wait); 0.4-1 % faster than issuing it at the
      // hand-over, where it was waited at once
      if (tid == 0 && !all_dealt) pending = atomicAdd(&a.counters[qx], 1);
    }
    flush_output();  // the previous item's output, behind this step's loads
    if (meta_late) load_meta(decode(nxt_idx), n_cnt, n_id, n_fl);
    const bool live = (fl >> half) & 1;
    const bool q_next = cross && nxt_idx >= 0;
    {
      // S^T = K Q^T for two 32-key tiles and each 32-query group.  Every K operand read from LDS
      // feeds NG MFMAs; the K operands of two d-steps stay in flight ahead of the MFMAs (software
      // pipelined LDS reads), so no MFMA waits on a fresh LDS read.
      f32x16 sc[NG][2];
#pragma unroll
      for (int g = 0; g < NG; ++g) sc[g][0] = sc[g][1] = f32x16{};
      u32x4 kr[2 * DS];
#pragma unroll
      for (int ds = 0; ds < 2; ++ds) {
        kr[2 * ds] = *(const u32x4*)(stage + koff[ds]);
        kr[2 * ds + 1] = *(const u32x4*)(stage + koff[ds] + 32 * D);
      }
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        if (ds + 2 < DS) {
          kr[2 * ds + 4] = *(const u32x4*)(stage + koff[ds + 2]);
          kr[2 * ds + 5] = *(const u32x4*)(stage + koff[ds + 2] + 32 * D);
        }
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          sc[g][0] = mfma32<F16>(kr[2 * ds], qreg[g][ds], sc[g][0]);
          sc[g][1] = mfma32<F16>(kr[2 * ds + 1], qreg[g][ds], sc[g][1]);
        }
      }
      // order: 4 K reads, then (2 reads, 2*NG MFMAs) per d-step, the last two d-steps MFMAs only
      __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 4, 0);
#pragma unroll
      for (int ds = 0; ds < DS - 2; ++ds) {
        __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 2, 0);
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, 2 * NG, 0);
      }
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, 4 * NG, 0);
      if (q_next) load_q(decode(nxt_idx));  // the current Q is dead after the score MFMAs
      // the first PFV V operands, read before the softmax so their latency hides under it
      const uint16_t* vt = stage + TILE;
      constexpr int NPV = 4 * DT;
      u32x4 vr[NPV];
      auto vread = [&](int j) {  // operand of MFMA j: d-tile j % DT, key step j / DT
        const int dt = j % DT, ks = j / DT;
        const u32x2 lo = read_tr(vt + voff[dt][0] + ks * 16 * D);
        const u32x2 hi = read_tr(vt + voff[dt][1] + ks * 16 * D);
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
      };
#pragma unroll
      for (int j = 0; j < PFV; ++j) vr[j] = vread(j);
      // online softmax for query ql of each group (this lane holds 32 of its 64 keys)
      float mx[NG];
      bool resc = false;
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        float m = sc[g][0][0];
#pragma unroll
        for (int i = 1; i < 16; ++i) m = fmaxf(m, sc[g][0][i]);
#pragma unroll
        for (int i = 0; i < 16; ++i) m = fmaxf(m, sc[g][1][i]);
        // A block this wave's query half may not see (paired flags) is computed but masked: its
        // row max counts as -inf (no rescale) and its exponent offset is -inf, so P = 0 exactly.
        // This lane's max over its 32 keys of the row decides; the row max (with the other 32
        // keys, held by the lane 32 away, which sees the same test) is taken only to rescale.
        mx[g] = live ? m * a.scale_log2 : -__builtin_inff();
        resc |= mx[g] > m_run[g] + RESCALE_LOG2;
      }
      // Lazy rescale: the exponent reference m_run moves only when some row's max exceeds it by
      // more than 2^8, so P = exp2(s - m_run) < 256 (exact range for fp32 state and bf16 P) and
      // the O rescale runs on few blocks.  O = acc / l does not depend on the choice.
      if (__ballot(resc) != 0) {
#pragma unroll
        for (int g = 0; g < NG; ++g) {
          const float m_new = fmaxf(m_run[g], pair_max(mx[g]));
          const float alpha = fast_exp2(m_run[g] - m_new);
          l_run[g] *= alpha;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) acc[g][dt] *= alpha;
          m_run[g] = m_new;
        }
      }
      u32x4 pk[NG][4];
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        const float neg = live ? -m_run[g] : -__builtin_inff();
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int i = 0; i < 16; ++i) sc[g][t][i] = fast_exp2(__builtin_fmaf(sc[g][t][i], a.scale_log2, neg));
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          pk[g][2 * t] = pack8<F16>(f32x8{sc[g][t][0], sc[g][t][1], sc[g][t][2], sc[g][t][3],
                                          sc[g][t][4], sc[g][t][5], sc[g][t][6], sc[g][t][7]});
          pk[g][2 * t + 1] = pack8<F16>(f32x8{sc[g][t][8], sc[g][t][9], sc[g][t][10], sc[g][t][11],
                                              sc[g][t][12], sc[g][t][13], sc[g][t][14], sc[g][t][15]});
        }
        // Row sum of P in fp32, before rounding, as paired_kernel.py:90 takes it (four chains).
        // A sum of the rounded P would make O's weights sum to exactly one but put up to 2^-9 of
        // relative error into l, i.e. about 2e-3 into the LSE of a row dominated by one key.
        float ls[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int i = 0; i < 16; ++i) ls[i & 3] += sc[g][t][i];
        l_run[g] += (ls[0] + ls[1]) + (ls[2] + ls[3]);
      }
      // O^T += V^T P^T, V operands read PFV MFMAs ahead, each feeding NG MFMAs
#pragma unroll
      for (int j = 0; j < NPV; ++j) {
        if (j + PFV < NPV) vr[j + PFV] = vread(j + PFV);
#pragma unroll
        for (int g = 0; g < NG; ++g) acc[g][j % DT] = mfma32<F16>(vr[j], pk[g][j / DT], acc[g][j % DT]);
      }
#pragma unroll
      for (int j = 0; j < NPV - PFV; ++j) {
        __builtin_amdgcn_sched_group_barrier(SG_DS_READ, 2, 1);
        __builtin_amdgcn_sched_group_barrier(SG_MFMA, NG, 1);
      }
      __builtin_amdgcn_sched_group_barrier(SG_MFMA, PFV * NG, 1);
    }
    if (!cross) {
      s = sn;
      return false;
    }
    epilogue();
    if (nxt_idx < 0) {
      flush_output();
      return true;
    }
    // Wait here, once per item, for the next item's Q (and with it its first K/V block): with
    // no load pending on qreg at the loop head, the steady-state steps keep their K/V prefetch in
    // flight across the whole compute of a step.
    __builtin_amdgcn_s_waitcnt(0);
    // advance to the next item (table entries loaded one item ahead; the claim of the one after
    // it was issued at the top of this step)
    cur = decode(nxt_idx);
    cur_k = k_base(cur);
    cur_v = v_base(cur);
    t_id = n_id;
    t_fl = n_fl;
    tbase = 0;
    if (!cur.global) cur.nsteps = max(uniform(n_cnt), 1) * KBR;
    claiming = true;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[g][dt] = f32x16{};
      m_run[g] = -__builtin_inff();
      l_run[g] = 0.f;
    }
    s = 0;
    return false;
  };
  for (;;) {
    if (step(lds0, lds1)) break;
    if (step(lds1, lds0)) break;
  }
  }
  // the last workgroup to leave resets the queue counters for the next launch
  __syncthreads();
  if (tid == 0 && atomicAdd(&a.counters[QUEUES], 1) == (int)gridDim.x - 1) {
    for (int q = 0; q <= QUEUES + 1; ++q) atomicExch(&a.counters[q], 0);
  }
}

// Combines the chunks of each split global query tile: O = sum_c 2^(m_c - M) acc_c / L with
// M = max_c m_c and L = sum_c 2^(m_c - M) l_c; LSE = (M + log2 L) ln 2.  One workgroup per tile,
// thread (wave, lane) owning the same fragment registers as in attn_fwd_kernel.
template <int HALVES, int D, bool F16>
__global__ __launch_bounds__(128 * HALVES) void merge_kernel(AttnArgs a) {
  constexpr int WAVES = 2 * HALVES;
  constexpr int QT = 64 * HALVES;
  constexpr int DT = D / 32;
  constexpr int FRAG = DT * 16 * 64;
  const int tile = blockIdx.x;
  const int dt = blockIdx.y;  // 32-column slice of the head dimension
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ql = lane & 31, hl = lane >> 5;
  const int bh = tile / a.global_tiles, gtile = tile - bh * a.global_tiles;
  const int b = bh / a.heads, h = bh - b * a.heads;
  const int64_t sl0 = (int64_t)tile * a.nsplit * WAVES + wave;
  // the 64 queries of a last global tile that reach past the global prefix (G an odd multiple of
  // 64, paired tables) belong to the first ordinary row, whose item stores them
  if (gtile * QT + wave * 32 >= a.global_tokens) return;
  const int q = gtile * QT + wave * 32 + ql;
  uint16_t* op = a.o + (int64_t)b * a.o_sb + (int64_t)h * a.o_sh + (int64_t)q * a.o_sn + hl * 4 + dt * 32;
  if (a.nsplit <= 4) {
    // up to four chunks: every load issued at once (indices clamped to the last chunk, whose
    // weight is then zero), one round trip instead of two
    constexpr int NS = 4;
    float m4[NS], l4[NS];
    f32x16 p4[NS];
#pragma unroll
    for (int c = 0; c < NS; ++c) {
      const int cc = c < a.nsplit ? c : a.nsplit - 1;
      const float* ml = a.part_ml + (sl0 + cc * WAVES) * 128 + lane;
      m4[c] = ml[0];
      l4[c] = ml[64];
      const float* pc = a.part + (sl0 + cc * WAVES) * FRAG + dt * 16 * 64 + lane;
#pragma unroll
      for (int i = 0; i < 16; ++i) p4[c][i] = pc[i * 64];
    }
    float mx = m4[0];
#pragma unroll
    for (int c = 1; c < NS; ++c) mx = fmaxf(mx, m4[c]);
    float ls = 0.f;
    f32x16 acc = f32x16{};
#pragma unroll
    for (int c = 0; c < NS; ++c) {
      const float w = c < a.nsplit ? fast_exp2(m4[c] - mx) : 0.f;
      ls += w * l4[c];
      acc += w * p4[c];
    }
    const float iv = 1.f / ls;
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      u32x2 w = {pack2<F16>(acc[gq * 4 + 0] * iv, acc[gq * 4 + 1] * iv),
                 pack2<F16>(acc[gq * 4 + 2] * iv, acc[gq * 4 + 3] * iv)};
      *(u32x2*)(op + gq * 8) = w;
    }
    if (a.lse && dt == 0 && hl == 0) a.lse[(int64_t)bh * a.tokens + q] = (mx + __log2f(ls)) * LN2;
    return;
  }
  float mc[MAX_SPLIT], lc[MAX_SPLIT], mmax = -__builtin_inff();
#pragma unroll
  for (int c = 0; c < MAX_SPLIT; ++c) {
    const float* ml = a.part_ml + (sl0 + c * WAVES) * 128 + lane;
    mc[c] = c < a.nsplit ? ml[0] : -__builtin_inff();
    lc[c] = c < a.nsplit ? ml[64] : 0.f;
  }
#pragma unroll
  for (int c = 0; c < MAX_SPLIT; ++c) mmax = fmaxf(mmax, mc[c]);
  float lsum = 0.f;
#pragma unroll
  for (int c = 0; c < MAX_SPLIT; ++c) {
    mc[c] = c < a.nsplit ? fast_exp2(mc[c] - mmax) : 0.f;
    lsum += mc[c] * lc[c];
  }
  const float inv = 1.f / lsum;
  f32x16 sum = f32x16{};
#pragma unroll
  for (int c = 0; c < MAX_SPLIT; ++c) {
    if (c < a.nsplit) {
      const float* pc = a.part + (sl0 + c * WAVES) * FRAG + dt * 16 * 64 + lane;
#pragma unroll
      for (int i = 0; i < 16; ++i) sum[i] += mc[c] * pc[i * 64];
    }
  }
#pragma unroll
  for (int gq = 0; gq < 4; ++gq) {
    u32x2 w = {pack2<F16>(sum[gq * 4 + 0] * inv, sum[gq * 4 + 1] * inv),
               pack2<F16>(sum[gq * 4 + 2] * inv, sum[gq * 4 + 3] * inv)};
    *(u32x2*)(op + gq * 8) = w;
  }
  if (a.lse && dt == 0 && hl == 0) a.lse[(int64_t)bh * a.tokens + q] = (mmax + __log2f(lsum)) * LN2;
}

struct Plan {
  int halves, d, kbr, f16;
  int global_tiles, nsplit, chunk, per_bh, rows, key_blocks, qt, waves;
  int64_t counters_bytes, part_bytes, ml_bytes;
};

// paired: 0 = unpaired 64-query rows, 1 = paired 128-query rows, 2 = quad 256-query rows
int make_plan(Plan& p, int batch, int heads, int tokens, int head_dim, int global_tokens, int width,
              int key_block_size, int paired, int all_queries) {
  HB_REQUIRE(batch > 0 && heads > 0 && tokens > 0, "batch, heads and tokens must be positive");
  HB_REQUIRE(head_dim == 64 || head_dim == 128, "head_dim must be 64 or 128 (got %d)", head_dim);
  // (a table row is read through a buffer whose byte size is a 32-bit width * 4)
  HB_REQUIRE(width >= 1 && width < (1 << 28), "table width must be in [1, 2^28) (got %d)", width);
  HB_REQUIRE(paired >= 0 && paired <= 2, "table kind must be 0 (unpaired), 1 (paired) or 2 (quad)");
  HB_REQUIRE(paired != 2 || (head_dim == 128 && key_block_size == 64),
             "quad tables take head_dim 128 and 64-key blocks");
  p.halves = paired == 2 ? 4 : (paired ? 2 : 1);
  p.qt = 64 * p.halves;
  p.waves = 2 * p.halves;
  p.d = head_dim;
  HB_REQUIRE(key_block_size == 64 || (paired && key_block_size == 128),
             "key_block_size must be 64 (or 128 with paired tables)");
  p.kbr = key_block_size / 64;
  // Paired tables take N and G in multiples of 64: rows are aligned to the end of the sequence
  // (the first one may reach 64 queries into the global prefix) and global tiles to its start
  // (the last one may reach 64 queries past G); the kernel stores neither overhang.
  const int align = p.halves == 2 ? 64 : p.qt;
  HB_REQUIRE(tokens % align == 0 && global_tokens % align == 0 && global_tokens >= 0 &&
                 global_tokens < tokens,
             "tokens and global_tokens must be multiples of %d with ordinary queries remaining", align);
  p.rows = (tokens - global_tokens + p.qt - 1) / p.qt;
  p.key_blocks = tokens / 64;
  p.global_tiles = all_queries ? (global_tokens + p.qt - 1) / p.qt : 0;
  // A global query tile sweeps every key block.  It is split into at most MAX_SPLIT chunks of
  // about the average work of one workgroup (at the nominal 2 workgroups x 256 CUs), never
  // shorter than the longest ordinary row or than MIN_CHUNK steps, and into at least two when the
  // sweep is four rows long or more: the chunks are claimed first, so each finishes well before
  // the queues drain, while few chunks keep the partials and the merge small.  The average is
  // estimated from the table width, which overstates the row work by up to 2x for tables padded
  // to a bound (rows paired on the device); the two-chunk floor keeps a whole sweep from ending
  // in the tail there.  (Against half the average: 2048 px 0.7-0.9 % faster with two chunks
  // instead of three, or none at 4-tile K1; the padded tables and the other shapes unchanged.)
  const int64_t row_steps = (int64_t)width * p.kbr;
  const int64_t all_steps =
      (int64_t)batch * heads * ((int64_t)p.rows * row_steps + (int64_t)p.global_tiles * p.key_blocks);
  // (quad workgroups are half as many, one per CU)
  const int64_t nominal = p.halves == 4 ? NOMINAL_GROUPS / 2 : NOMINAL_GROUPS;
  int64_t target = (all_steps + nominal - 1) / nominal;
  if (target < row_steps) target = row_steps;
  if (target < MIN_CHUNK) target = MIN_CHUNK;
  int nsplit = (int)((p.key_blocks + target - 1) / target);
  if (nsplit < 2 && p.key_blocks >= 4 * row_steps) nsplit = 2;
  nsplit = nsplit < 1 ? 1 : (nsplit > MAX_SPLIT ? MAX_SPLIT : nsplit);
  p.chunk = (p.key_blocks + nsplit - 1) / nsplit;
  p.nsplit = (p.key_blocks + p.chunk - 1) / p.chunk;
  p.per_bh = p.global_tiles * p.nsplit + p.rows;
  const int64_t bh = (int64_t)batch * heads;
  const int64_t tiles = bh * p.global_tiles;
  p.counters_bytes = 256;
  const int64_t slots = p.nsplit > 1 ? tiles * p.nsplit * p.waves : 0;
  p.part_bytes = slots * (head_dim / 32) * 16 * 64 * 4;
  p.ml_bytes = slots * 128 * 4;
  return HB_OK;
}

// Zeroes the work-queue counters (the first 256 bytes of a workspace) ahead of a launch.  A fill
// kernel rather than hipMemsetAsync, so that a captured HIP graph replays it as a kernel node.
__global__ __launch_bounds__(64) void clear_counters_kernel(int32_t* counters) {
  counters[threadIdx.x] = 0;
}

template <int HALVES, int D, int KBR, bool F16>
void launch(const AttnArgs& a, int groups, hipStream_t stream) {
  hipLaunchKernelGGL((attn_fwd_kernel<HALVES, D, KBR, F16>), dim3(groups), dim3(128 * HALVES), 0,
                     stream, a);
  const int tiles = a.bh * a.global_tiles;
  if (a.nsplit > 1 && tiles > 0)
    hipLaunchKernelGGL((merge_kernel<HALVES, D, F16>), dim3(tiles, D / 32), dim3(128 * HALVES), 0,
                       stream, a);
}

template <int HALVES, int KBR>
int dispatch_d(const AttnArgs& a, int d, int f16, int groups, hipStream_t stream) {
  if (d == 128) {
    if (f16) launch<HALVES, 128, KBR, true>(a, groups, stream);
    else launch<HALVES, 128, KBR, false>(a, groups, stream);
  } else {
    if (f16) launch<HALVES, 64, KBR, true>(a, groups, stream);
    else launch<HALVES, 64, KBR, false>(a, groups, stream);
  }
  return HB_OK;
}

int attention_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                  const int64_t* strides, int32_t batch, int32_t heads, int32_t tokens,
                  int32_t head_dim, int32_t dtype, const int32_t* kv_indices,
                  const int32_t* kv_flags, const int32_t* kv_counts, int32_t table_width,
                  int32_t global_tokens, int32_t key_block_size, int32_t paired,
                  int32_t all_queries, float scale_log2, void* workspace,
                  int64_t workspace_bytes, int32_t num_groups, hipStream_t stream,
                  bool clear_counters = false) {
  Plan p;
  int rc = make_plan(p, batch, heads, tokens, head_dim, global_tokens, table_width, key_block_size,
                     paired, all_queries);
  if (rc) return rc;
  HB_REQUIRE(dtype == HB_DTYPE_BF16 || dtype == HB_DTYPE_F16, "dtype must be bf16 or fp16");
  HB_REQUIRE(q && k && v && out && kv_indices && kv_counts && strides, "null pointer argument");
  HB_REQUIRE(!paired || kv_flags, "paired tables need kv_flags");
  HB_REQUIRE(scale_log2 > 0.f && scale_log2 < 3.0e38f, "scale must be positive and finite");
  const void* ptrs[4] = {q, k, v, out};
  for (int i = 0; i < 4; ++i)
    HB_REQUIRE(((uintptr_t)ptrs[i] & 15) == 0, "Q/K/V/out base pointers must be 16-byte aligned");
  for (int i = 0; i < 12; ++i)
    HB_REQUIRE(strides[i] > 0 && strides[i] % 8 == 0 && strides[i] < (1ll << 31),
               "Q/K/V/out outer strides must be positive multiples of 8 elements below 2^31");
  // a lane's output row inside an item is addressed with a 32-bit element offset
  HB_REQUIRE((int64_t)p.qt * strides[11] + head_dim < (1ll << 31),
             "output token stride too large: %d rows must span fewer than 2^31 elements", p.qt);
  // K/V blocks are addressed with 32-bit byte offsets from each (batch, head) base
  HB_REQUIRE(((int64_t)tokens * (strides[5] > strides[8] ? strides[5] : strides[8])) * 2 < (1ll << 31),
             "K/V token stride too large: one (batch, head) must span less than 2 GiB");
  const int64_t need = p.counters_bytes + p.part_bytes + p.ml_bytes;
  HB_REQUIRE(workspace && workspace_bytes >= need && ((uintptr_t)workspace & 255) == 0,
             "workspace must be 256-byte aligned and hold %lld bytes", (long long)need);
  AttnArgs a;
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)k;
  a.v = (const uint16_t*)v;
  a.o = (uint16_t*)out;
  a.lse = lse;
  a.q_sb = strides[0]; a.q_sh = strides[1]; a.q_sn = strides[2];
  a.k_sb = strides[3]; a.k_sh = strides[4]; a.k_sn = strides[5];
  a.v_sb = strides[6]; a.v_sh = strides[7]; a.v_sn = strides[8];
  a.o_sb = strides[9]; a.o_sh = strides[10]; a.o_sn = strides[11];
  a.indices = kv_indices;
  a.flags = kv_flags ? kv_flags : kv_indices;
  a.counts = kv_counts;
  a.heads = heads;
  a.tokens = tokens;
  a.global_tokens = global_tokens;
  a.bh = batch * heads;
  a.width = table_width;
  a.rows = p.rows;
  a.key_blocks = p.key_blocks;
  a.global_tiles = p.global_tiles;
  a.nsplit = p.nsplit;
  a.chunk = p.chunk;
  a.per_bh = p.per_bh;
  a.scale_log2 = scale_log2;
  a.counters = (int32_t*)workspace;
  a.part = (float*)((char*)workspace + p.counters_bytes);
  a.part_ml = (float*)((char*)workspace + p.counters_bytes + p.part_bytes);
  const int64_t items = (int64_t)a.bh * p.per_bh;
  // three workgroups per CU where the kernel fits them, once each gets two items or more (with
  // fewer, the call finishes sooner on two workgroups per CU, whose items run faster)
  const int cus = device_cu_count();
  const int per_cu = p.halves == 4 ? groups_per_cu<4, 128>()
                     : paired && head_dim == 64 && items >= 2 * 3 * (int64_t)cus ? groups_per_cu<2, 64>() : 2;
  int groups = num_groups > 0 ? num_groups : per_cu * cus;
  if (groups > items) groups = (int)items;
  if (groups < 1) return HB_OK;
  if (clear_counters) {
    static_assert(QUEUES + 2 <= 64, "the counters fit the cleared 256 bytes");
    hipLaunchKernelGGL(clear_counters_kernel, dim3(1), dim3(64), 0, stream, a.counters);
  }
  if (p.halves == 4) {
    if (dtype == HB_DTYPE_F16) launch<4, 128, 1, true>(a, groups, stream);
    else launch<4, 128, 1, false>(a, groups, stream);
  } else if (paired) {
    if (p.kbr == 2) dispatch_d<2, 2>(a, head_dim, dtype == HB_DTYPE_F16, groups, stream);
    else dispatch_d<2, 1>(a, head_dim, dtype == HB_DTYPE_F16, groups, stream);
  } else {
    dispatch_d<1, 1>(a, head_dim, dtype == HB_DTYPE_F16, groups, stream);
  }
  HB_HIP(hipGetLastError());
  return HB_OK;
}

}  // namespace
}  // namespace hb

// Workspace of hb_paired_fwd_noalloc: the work-queue counters and the split partials live in this
// array, one copy per device, held from the library's first use on a device until the process
// ends.  Host code never passes `scratch` itself to a kernel (on the host it names a stand-in, not
// device memory): it passes the device address hipGetSymbolAddress returns for the current device.
static __device__ __align__(256) unsigned char scratch[HB_NOALLOC_SCRATCH_BYTES];

namespace hb {
namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[MAX_DEVICES] = {};

// Device address of `scratch` on the current device, looked up once per device.
int scratch_address(void** out) {
  int dev = 0;
  HB_HIP(hipGetDevice(&dev));
  HB_REQUIRE(dev >= 0 && dev < MAX_DEVICES, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    HB_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    HB_REQUIRE(p != nullptr && ((uintptr_t)p & 255) == 0, "scratch address lookup failed");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return HB_OK;
}

}  // namespace
}  // namespace hb

extern "C" int64_t hb_attention_workspace_bytes(int32_t batch, int32_t heads, int32_t tokens,
                                                int32_t head_dim, int32_t global_tokens,
                                                int32_t table_width, int32_t key_block_size,
                                                int32_t paired, int32_t all_queries) {
  hb::Plan p;
  if (hb::make_plan(p, batch, heads, tokens, head_dim, global_tokens, table_width, key_block_size,
                    paired, all_queries))
    return -1;
  return p.counters_bytes + p.part_bytes + p.ml_bytes;
}

extern "C" int hb_paired_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                             const int64_t* strides, int32_t batch, int32_t heads, int32_t tokens,
                             int32_t head_dim, int32_t dtype, const int32_t* kv_indices,
                             const int32_t* kv_flags, const int32_t* kv_counts,
                             int32_t table_width, int32_t global_tokens, int32_t key_block_size,
                             int32_t all_queries, float scale_log2, void* workspace,
                             int64_t workspace_bytes, int32_t num_groups, hipStream_t stream) {
  return hb::attention_fwd(q, k, v, out, lse, strides, batch, heads, tokens, head_dim, dtype,
                           kv_indices, kv_flags, kv_counts, table_width, global_tokens,
                           key_block_size, 1, all_queries, scale_log2, workspace, workspace_bytes,
                           num_groups, stream);
}

extern "C" int hb_quad_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                           const int64_t* strides, int32_t batch, int32_t heads, int32_t tokens,
                           int32_t head_dim, int32_t dtype, const int32_t* kv_indices,
                           const int32_t* kv_flags, const int32_t* kv_counts, int32_t table_width,
                           int32_t global_tokens, int32_t all_queries, float scale_log2,
                           void* workspace, int64_t workspace_bytes, int32_t num_groups,
                           hipStream_t stream) {
  return hb::attention_fwd(q, k, v, out, lse, strides, batch, heads, tokens, head_dim, dtype,
                           kv_indices, kv_flags, kv_counts, table_width, global_tokens, 64, 2,
                           all_queries, scale_log2, workspace, workspace_bytes, num_groups, stream);
}

extern "C" int hb_block_sparse_fwd(const void* q, const void* k, const void* v, void* out,
                                   float* lse, const int64_t* strides, int32_t batch,
                                   int32_t heads, int32_t tokens, int32_t head_dim, int32_t dtype,
                                   const int32_t* kv_indices, const int32_t* kv_counts,
                                   int32_t table_width, int32_t global_tokens, int32_t block_size,
                                   int32_t all_queries, float scale_log2, void* workspace,
                                   int64_t workspace_bytes, int32_t num_groups,
                                   hipStream_t stream) {
  HB_REQUIRE(block_size == 64, "block_size must be 64");
  return hb::attention_fwd(q, k, v, out, lse, strides, batch, heads, tokens, head_dim, dtype,
                           kv_indices, nullptr, kv_counts, table_width, global_tokens, 64, 0,
                           all_queries, scale_log2, workspace, workspace_bytes, num_groups,
                           stream);
}

extern "C" int hb_paired_fwd_noalloc(const void* q, const void* k, const void* v, void* out,
                                     float* lse, const int64_t* strides, int32_t batch,
                                     int32_t heads, int32_t tokens, int32_t head_dim,
                                     int32_t dtype, const int32_t* kv_indices,
                                     const int32_t* kv_flags, const int32_t* kv_counts,
                                     int32_t table_width, int32_t global_tokens,
                                     int32_t key_block_size, int32_t all_queries, float scale_log2,
                                     int32_t num_groups, hipStream_t stream) {
  // the size check comes first: shapes beyond the static scratch are rejected before any HIP call
  hb::Plan p;
  int rc = hb::make_plan(p, batch, heads, tokens, head_dim, global_tokens, table_width,
                         key_block_size, 1, all_queries);
  if (rc) return rc;
  const int64_t need = p.counters_bytes + p.part_bytes + p.ml_bytes;
  HB_REQUIRE(need <= HB_NOALLOC_SCRATCH_BYTES,
             "hb_paired_fwd_noalloc: these shapes need %lld bytes of scratch, the static scratch "
             "holds %lld; use hb_paired_fwd with a caller workspace",
             (long long)need, (long long)HB_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  rc = hb::scratch_address(&ws);
  if (rc) return rc;
  return hb::attention_fwd(q, k, v, out, lse, strides, batch, heads, tokens, head_dim, dtype,
                           kv_indices, kv_flags, kv_counts, table_width, global_tokens,
                           key_block_size, 1, all_queries, scale_log2, ws, HB_NOALLOC_SCRATCH_BYTES,
                           num_groups, stream, /*clear_counters=*/true);
}
