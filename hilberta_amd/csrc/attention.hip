// Block-sparse flash-attention forward for HilbertA block tables on gfx950 (MI355X).
//
// Replaces the Triton kernels _paired_fwd (reference hilberta/paired_kernel.py:18-94) and
// _block_sparse_fwd (hilberta/sparse_kernel.py:28-97) with one hand-written CDNA4 kernel:
//
//  * Work item = one query tile (128 queries for paired tables, 64 for unpaired ones) of one
//    (batch, head), or one chunk of a global (text) query tile's all-key sweep.  Global tiles are
//    split into chunks of about one table row's length so no item is longer than the longest
//    ordinary row; chunk partials (unnormalised accumulator, running max, row sum) are merged by
//    the last chunk to finish (counter in the workspace).
//  * Persistent workgroups (2 per CU) pull items from 8 queues, one per XCD, each queue owning the
//    heads bh = q, q+8, ...; a workgroup starts with the queue of its own XCD (dispatch is round
//    robin over XCDs) so items that share K/V blocks run under one L2, then steals from the
//    others.  Queue heads reset themselves when the last workgroup leaves.
//  * Per 64-key block: K (row major) and V (transposed, keys permuted to the MFMA operand order)
//    are staged through double-buffered LDS; the next block's global loads are in flight while the
//    current block is computed.  Blocks whose flags allow neither query half are never loaded.
//  * Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16_bf16: each lane then
//    holds 16 keys of ONE query, so the online-softmax row max is an in-lane max plus one
//    permlane32 swap, and the output O^T = V^T P^T reuses the score registers directly as the
//    B operand (no shuffle of P) while the rescale by alpha is a per-lane scalar.
//  * Each wave owns 32 queries; in paired mode waves 0-1 own query half 0 and waves 2-3 half 1, so
//    the flag test (flags >> (half + 2*key_half)) & 1 of paired_kernel.py:65,83-84 is a
//    wave-uniform skip.
//  * Online softmax in exp2 with fp32 state (paired_kernel.py:82-93); P is rounded to the input
//    type before the PV product as in the reference; an optional fp32 per-row logsumexp (natural
//    log) is written as well.
#include "common.h"
#include "../../include/hilberta_hip.h"

namespace hb {
namespace {

constexpr int KEYS = 64;     // keys per staged block
constexpr int PAD = 8;       // LDS row padding in elements (16 bytes) against bank conflicts
constexpr float LN2 = 0.69314718055994530942f;
constexpr int QUEUES = 8;    // one work queue per XCD
// The workspace starts with a fixed counter region (queue heads, exit count, one merge counter
// per split global tile) that every launch leaves at zero, whatever its shapes; partials follow.
constexpr int64_t COUNTER_BYTES = 64 * 1024;
constexpr int64_t MAX_SPLIT_TILES = COUNTER_BYTES / 4 - 16;

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  float* lse;
  int64_t q_sb, q_sh, q_sn, k_sb, k_sh, k_sn, v_sb, v_sh, v_sn, o_sb, o_sh, o_sn;
  const int32_t* indices;
  const int32_t* flags;
  const int32_t* counts;
  int32_t heads, tokens, bh, width, rows, key_blocks;
  int32_t global_tiles, nsplit, chunk, per_bh;
  float scale_log2;
  int32_t* counters;  // [0..7] queue heads, [8] exit count, [16 + tile] split-merge counters
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

// x combined with the value held by the lane 32 positions away (ds_bpermute; `partner` is the
// byte address ((lane ^ 32) << 2)).
__device__ __forceinline__ float pair_max(float x, int partner) {
  const float y = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(partner, __builtin_bit_cast(int, x)));
  return fmaxf(x, y);
}
__device__ __forceinline__ float pair_sum(float x, int partner) {
  const float y = __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(partner, __builtin_bit_cast(int, x)));
  return x + y;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Position of key kappa (0..15) inside a 16-key group of the transposed V tile: the order in
// which a lane's S^T registers present keys to the PV MFMA (lane half hl, slot r -> key
// 8*(r/4) + 4*hl + r%4).
__device__ __forceinline__ int vpos4(int g) {  // first position of keys 4g..4g+3, g in 0..15
  const int k0 = (g & 3) * 4;
  return 16 * (g >> 2) + 8 * ((k0 >> 2) & 1) + 4 * (k0 >> 3);
}

template <int HALVES, int D, int KBR, bool F16>
__global__ __launch_bounds__(128 * HALVES, HALVES) void attn_fwd_kernel(AttnArgs a) {
  constexpr int WAVES = 2 * HALVES;
  constexpr int NT = 64 * WAVES;
  constexpr int QT = 64 * HALVES;               // queries per work item
  constexpr int KS = D + PAD;                   // K tile row stride (elements)
  constexpr int VS = KEYS + PAD;                // V^T tile row stride (elements)
  constexpr int K_ELEMS = KEYS * KS;
  constexpr int STAGE = K_ELEMS + D * VS;
  constexpr int DC = D / 8;                     // 16-byte chunks per row
  constexpr int KCH = KEYS * DC / NT;           // K chunks per thread
  constexpr int VGROUPS = 16 * DC;              // (4 keys x 8 dims) groups per V tile
  constexpr int VG = (VGROUPS + NT - 1) / NT;   // V groups per thread
  constexpr int DT = D / 32;                    // output 32-dim tiles
  constexpr int DS = D / 16;                    // contraction steps over D
  static_assert(KEYS * DC % NT == 0, "K staging must divide evenly");

  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * STAGE];
  __shared__ int s_item;
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = HALVES == 2 ? (wave >> 1) : 0;
  const int ql = lane & 31;   // query (column) owned by this lane inside the wave's 32
  const int hl = lane >> 5;   // lane half: selects the 8-element k slice of MFMA operands
  const int partner = (lane ^ 32) << 2;

  const int q0 = blockIdx.x % QUEUES;
  for (int qi = 0; qi < QUEUES; ++qi) {
    const int queue = (q0 + qi) % QUEUES;
    const int nbh = a.bh > queue ? (a.bh - queue + QUEUES - 1) / QUEUES : 0;
    const int nitems = nbh * a.per_bh;
    for (;;) {
      if (tid == 0) s_item = atomicAdd(&a.counters[queue], 1);
      __syncthreads();
      const int item = uniform(s_item);
      __syncthreads();
      if (item >= nitems) break;

      // ---------------------------------------------------------------- decode the work item
      const int bh = queue + QUEUES * (item / a.per_bh);
      const int rem = item % a.per_bh;
      const int b = bh / a.heads;
      const int h = bh - b * a.heads;
      const bool is_global = rem < a.global_tiles * a.nsplit;
      int qfirst, row = 0, gtile = 0, split = 0, nsteps, first_block = 0;
      if (is_global) {
        gtile = rem / a.nsplit;
        split = rem - gtile * a.nsplit;
        qfirst = gtile * QT;
        first_block = split * a.chunk;
        nsteps = min(a.chunk, a.key_blocks - first_block);
      } else {
        row = rem - a.global_tiles * a.nsplit;
        qfirst = a.tokens - (a.rows - row) * QT;  // ordinary rows follow the global prefix
        nsteps = a.counts[row] * KBR;
      }
      const int32_t* trow_ids = a.indices + (int64_t)row * a.width;
      const int32_t* trow_flags = a.flags + (int64_t)row * a.width;

      // 64-key block index and per-half permission bits of step s (bit h = query half h may see it)
      auto step_info = [&](int s, int& kb, int& fl) {
        if (is_global) {
          kb = first_block + s;
          fl = 3;
        } else if (HALVES == 2) {
          const int e = s / KBR;
          const int sub = s - e * KBR;
          kb = trow_ids[e] * KBR + sub;
          fl = (trow_flags[e] >> (2 * sub)) & 3;
        } else {
          kb = trow_ids[s];
          fl = 1;
        }
      };
      auto next_live = [&](int s) {
        for (; s < nsteps; ++s) {
          int kb, fl;
          step_info(s, kb, fl);
          if (fl) break;
        }
        return s;
      };

      const uint16_t* kbh = a.k + b * a.k_sb + h * a.k_sh;
      const uint16_t* vbh = a.v + b * a.v_sb + h * a.v_sh;

      // ---------------------------------------------------------------- Q^T operand in registers
      u32x4 qreg[DS];
      {
        const uint16_t* qp = a.q + b * a.q_sb + h * a.q_sh +
                             (int64_t)(qfirst + wave * 32 + ql) * a.q_sn + hl * 8;
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) qreg[ds] = *(const u32x4*)(qp + ds * 16);
      }

      f32x16 acc[DT];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16{};
      float m_run = -__builtin_inff();
      float l_run = 0.f;

      u32x4 kst[KCH];
      u32x4 vst[VG][4];
      auto load_block = [&](int kb) {
        const uint16_t* kp = kbh + (int64_t)kb * KEYS * a.k_sn;
        const uint16_t* vp = vbh + (int64_t)kb * KEYS * a.v_sn;
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
          const int idx = tid + j * NT;
          const int r = idx / DC, c = idx % DC;
          kst[j] = *(const u32x4*)(kp + r * a.k_sn + c * 8);
        }
#pragma unroll
        for (int j = 0; j < VG; ++j) {
          const int idx = tid + j * NT;
          if (VGROUPS % NT == 0 || idx < VGROUPS) {
            const int g = idx % 16, c = idx / 16;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
              vst[j][kk] = *(const u32x4*)(vp + (4 * g + kk) * a.v_sn + c * 8);
          }
        }
      };
      auto store_block = [&](uint16_t* stage) {
#pragma unroll
        for (int j = 0; j < KCH; ++j) {
          const int idx = tid + j * NT;
          const int r = idx / DC, c = idx % DC;
          *(u32x4*)(stage + r * KS + c * 8) = kst[j];
        }
        uint16_t* vt = stage + K_ELEMS;
#pragma unroll
        for (int j = 0; j < VG; ++j) {
          const int idx = tid + j * NT;
          if (VGROUPS % NT == 0 || idx < VGROUPS) {
            const int g = idx % 16, c = idx / 16;
            uint16_t* dst = vt + (c * 8) * VS + vpos4(g);
#pragma unroll
            for (int m = 0; m < 4; ++m) {  // word m of each key row holds dims 2m, 2m+1
              const uint32_t w0 = vst[j][0][m], w1 = vst[j][1][m], w2 = vst[j][2][m], w3 = vst[j][3][m];
              u32x2 even = {(w0 & 0xffffu) | (w1 << 16), (w2 & 0xffffu) | (w3 << 16)};
              u32x2 odd = {(w0 >> 16) | (w1 & 0xffff0000u), (w2 >> 16) | (w3 & 0xffff0000u)};
              *(u32x2*)(dst + (2 * m) * VS) = even;
              *(u32x2*)(dst + (2 * m + 1) * VS) = odd;
            }
          }
        }
      };

      // ---------------------------------------------------------------- main loop over key blocks
      int s = next_live(0);
      int buf = 0;
      if (s < nsteps) {
        int kb, fl;
        step_info(s, kb, fl);
        load_block(kb);
      }
      while (s < nsteps) {
        int kb, fl;
        step_info(s, kb, fl);
        uint16_t* stage = lds + buf * STAGE;
        store_block(stage);
        __syncthreads();
        const int sn = next_live(s + 1);
        if (sn < nsteps) {
          int kbn, fln;
          step_info(sn, kbn, fln);
          load_block(kbn);
        }
        if ((fl >> half) & 1) {
          // S^T = K Q^T for two 32-key tiles
          f32x16 s0 = f32x16{}, s1 = f32x16{};
          const uint16_t* kl = stage + ql * KS + hl * 8;
#pragma unroll
          for (int ds = 0; ds < DS; ++ds) {
            const u32x4 k0 = *(const u32x4*)(kl + ds * 16);
            const u32x4 k1 = *(const u32x4*)(kl + 32 * KS + ds * 16);
            s0 = mfma32<F16>(k0, qreg[ds], s0);
            s1 = mfma32<F16>(k1, qreg[ds], s1);
          }
          // online softmax for query ql (this lane holds 32 of its 64 keys)
          float mx = s0[0];
#pragma unroll
          for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s0[i]);
#pragma unroll
          for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s1[i]);
          mx = pair_max(mx, partner) * a.scale_log2;
          const float m_new = fmaxf(m_run, mx);
          const float alpha = fast_exp2(m_run - m_new);
          const float neg = -m_new;
          float lsum = 0.f;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            s0[i] = fast_exp2(__builtin_fmaf(s0[i], a.scale_log2, neg));
            lsum += s0[i];
          }
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            s1[i] = fast_exp2(__builtin_fmaf(s1[i], a.scale_log2, neg));
            lsum += s1[i];
          }
          l_run = l_run * alpha + lsum;
          m_run = m_new;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
          u32x4 pk[4];
          pk[0] = pack8<F16>(f32x8{s0[0], s0[1], s0[2], s0[3], s0[4], s0[5], s0[6], s0[7]});
          pk[1] = pack8<F16>(f32x8{s0[8], s0[9], s0[10], s0[11], s0[12], s0[13], s0[14], s0[15]});
          pk[2] = pack8<F16>(f32x8{s1[0], s1[1], s1[2], s1[3], s1[4], s1[5], s1[6], s1[7]});
          pk[3] = pack8<F16>(f32x8{s1[8], s1[9], s1[10], s1[11], s1[12], s1[13], s1[14], s1[15]});
          // O^T += V^T P^T
          const uint16_t* vl = stage + K_ELEMS + ql * VS + hl * 8;
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
              const u32x4 vop = *(const u32x4*)(vl + dt * 32 * VS + ks * 16);
              acc[dt] = mfma32<F16>(vop, pk[ks], acc[dt]);
            }
          }
        }
        buf ^= 1;
        s = sn;
      }

      // ---------------------------------------------------------------- epilogue
      const float l_tot = pair_sum(l_run, partner);
      const int q = qfirst + wave * 32 + ql;
      uint16_t* op = a.o + b * a.o_sb + h * a.o_sh + (int64_t)q * a.o_sn + hl * 4;
      float* lsep = a.lse ? a.lse + (int64_t)bh * a.tokens + q : nullptr;
      if (!is_global || a.nsplit == 1) {
        const float inv = 1.f / l_tot;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            u32x2 w = {pack2<F16>(acc[dt][gq * 4 + 0] * inv, acc[dt][gq * 4 + 1] * inv),
                       pack2<F16>(acc[dt][gq * 4 + 2] * inv, acc[dt][gq * 4 + 3] * inv)};
            *(u32x2*)(op + dt * 32 + gq * 8) = w;
          }
        if (lsep && hl == 0) *lsep = (m_run + __log2f(l_tot)) * LN2;
      } else {
        // split global tile: publish the partial, the last chunk merges all of them
        const int tile = bh * a.global_tiles + gtile;
        const int64_t slot = (int64_t)tile * a.nsplit + split;
        constexpr int FRAG = DT * 16 * 64;
        float* pa = a.part + (slot * WAVES + wave) * FRAG;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int i = 0; i < 16; ++i) pa[(dt * 16 + i) * 64 + lane] = acc[dt][i];
        float* pml = a.part_ml + (slot * WAVES + wave) * 128;
        pml[lane] = m_run;
        pml[64 + lane] = l_tot;
        __threadfence();
        __syncthreads();
        if (tid == 0) s_last = atomicAdd(&a.counters[16 + tile], 1) == a.nsplit - 1;
        __syncthreads();
        if (s_last) {
          __threadfence();
          float mmax = -__builtin_inff();
          for (int c = 0; c < a.nsplit; ++c) {
            const float* pm = a.part_ml + (((int64_t)tile * a.nsplit + c) * WAVES + wave) * 128;
            mmax = fmaxf(mmax, __builtin_nontemporal_load(pm + lane));
          }
          f32x16 sum[DT];
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) sum[dt] = f32x16{};
          float lsum = 0.f;
          for (int c = 0; c < a.nsplit; ++c) {
            const int64_t sl = ((int64_t)tile * a.nsplit + c) * WAVES + wave;
            const float* pm = a.part_ml + sl * 128;
            const float w = fast_exp2(__builtin_nontemporal_load(pm + lane) - mmax);
            lsum += w * __builtin_nontemporal_load(pm + 64 + lane);
            const float* pc = a.part + sl * FRAG;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
              for (int i = 0; i < 16; ++i)
                sum[dt][i] += w * __builtin_nontemporal_load(pc + (dt * 16 + i) * 64 + lane);
          }
          const float inv = 1.f / lsum;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              u32x2 w = {pack2<F16>(sum[dt][gq * 4 + 0] * inv, sum[dt][gq * 4 + 1] * inv),
                         pack2<F16>(sum[dt][gq * 4 + 2] * inv, sum[dt][gq * 4 + 3] * inv)};
              *(u32x2*)(op + dt * 32 + gq * 8) = w;
            }
          if (lsep && hl == 0) *lsep = (mmax + __log2f(lsum)) * LN2;
          if (tid == 0) atomicExch(&a.counters[16 + tile], 0);
        }
      }
    }
  }
  // the last workgroup to leave resets the queue heads for the next launch on this workspace
  __syncthreads();
  if (tid == 0) {
    __threadfence();
    if (atomicAdd(&a.counters[QUEUES], 1) == (int)gridDim.x - 1) {
      for (int i = 0; i <= QUEUES; ++i) atomicExch(&a.counters[i], 0);
    }
  }
}

struct Plan {
  int halves, d, kbr, f16;
  int global_tiles, nsplit, chunk, per_bh, rows, key_blocks, qt, waves;
  int64_t counters_bytes, part_bytes, ml_bytes;
};

int make_plan(Plan& p, int batch, int heads, int tokens, int head_dim, int global_tokens, int width,
              int key_block_size, int paired, int all_queries) {
  HB_REQUIRE(batch > 0 && heads > 0 && tokens > 0, "batch, heads and tokens must be positive");
  HB_REQUIRE(head_dim == 64 || head_dim == 128, "head_dim must be 64 or 128 (got %d)", head_dim);
  HB_REQUIRE(width >= 1, "table width must be positive");
  p.halves = paired ? 2 : 1;
  p.qt = 64 * p.halves;
  p.waves = 2 * p.halves;
  p.d = head_dim;
  HB_REQUIRE(key_block_size == 64 || (paired && key_block_size == 128),
             "key_block_size must be 64 (or 128 with paired tables)");
  p.kbr = key_block_size / 64;
  HB_REQUIRE(tokens % p.qt == 0 && global_tokens % p.qt == 0 && global_tokens >= 0 &&
                 global_tokens < tokens,
             "tokens and global_tokens must be multiples of %d with ordinary queries remaining", p.qt);
  p.rows = (tokens - global_tokens) / p.qt;
  p.key_blocks = tokens / 64;
  p.global_tiles = all_queries ? global_tokens / p.qt : 0;
  int chunk = width * p.kbr;
  chunk = chunk < 16 ? 16 : chunk;
  const int min_chunk = (p.key_blocks + 63) / 64;
  chunk = chunk < min_chunk ? min_chunk : chunk;
  p.chunk = chunk;
  p.nsplit = (p.key_blocks + chunk - 1) / chunk;
  p.per_bh = p.global_tiles * p.nsplit + p.rows;
  const int64_t bh = (int64_t)batch * heads;
  const int64_t tiles = bh * p.global_tiles;
  HB_REQUIRE(tiles <= MAX_SPLIT_TILES, "too many global query tiles (%lld > %lld)",
             (long long)tiles, (long long)MAX_SPLIT_TILES);
  p.counters_bytes = COUNTER_BYTES;
  const int64_t slots = p.nsplit > 1 ? tiles * p.nsplit * p.waves : 0;
  p.part_bytes = slots * (head_dim / 32) * 16 * 64 * 4;
  p.ml_bytes = slots * 128 * 4;
  return HB_OK;
}

template <int HALVES, int D, int KBR, bool F16>
void launch(const AttnArgs& a, int groups, hipStream_t stream) {
  hipLaunchKernelGGL((attn_fwd_kernel<HALVES, D, KBR, F16>), dim3(groups), dim3(128 * HALVES), 0,
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
                  int64_t workspace_bytes, int32_t num_groups, hipStream_t stream) {
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
    HB_REQUIRE(strides[i] > 0 && strides[i] % 8 == 0,
               "Q/K/V/out outer strides must be positive multiples of 8 elements");
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
  int groups = num_groups > 0 ? num_groups : 2 * device_cu_count();
  if (groups > items) groups = (int)items;
  if (groups < 1) return HB_OK;
  if (paired) {
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
