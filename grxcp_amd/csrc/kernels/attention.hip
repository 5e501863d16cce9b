// grxDNN fused scaled-dot-product attention (forward) on gfx950.
//
// New: the reference plans attention for grxDNN but ships no code
// (ref docs/designs/grxcp_roadmap.md:864-877). Single pass, online softmax,
// O(S) memory:
//
//  * persistent: one workgroup per CU (8 wavefronts, two per SIMD) loops
//    over work items of 256 query rows of one (batch, head); each wave owns
//    32 queries whose Q fragments stay in VGPRs for the item. The K/V loads
//    run across items (an item's last tiles load the next item's first),
//    the next item's Q loads behind the last tile, and O is stored while
//    the next item starts: no workgroup launch, prologue or drain between
//    items (measured ~30K idle cycles per CU between one-shot workgroups,
//    plus ~11K of prologue and epilogue);
//  * K and V stream through LDS in 64-key tiles by direct-to-LDS buffer loads
//    (no staging registers; rows past the sequence read as zero) into three
//    stages, each tile's loads issued two tiles ahead of its use (three
//    stages measured 0.7-2.7 % faster than two with the same waits);
//  * the K fragments of the score MFMAs are read four MFMAs ahead of their
//    use and the two 32-key accumulation chains alternate (pinned with
//    sched_group_barrier; +4 %);
//  * scores are computed TRANSPOSED, S^T = K Q^T (v_mfma_f32_32x32x16): per
//    lane the accumulator holds 32 keys of ONE query, so the softmax row
//    max/sum is an in-register reduction plus one exchange with lane^32;
//  * O^T += V^T P^T: P^T is already in the B-operand layout in the lanes
//    that computed it (no LDS round trip), and the V^T operand is read from
//    the row-major V tile with ds_read_b64_tr_b16 (gfx950's transposing LDS
//    read: 4 keys of one head-dim column per lane), so V is never rewritten;
//  * softmax in the exp2 domain with the running max m tracked in scaled
//    units: p = exp2(s*scale*log2e - m). m is only raised when a tile's max
//    exceeds it by more than 8 (p <= 2^8 otherwise, exact in bf16's relative
//    precision), so the O rescale (and its 128 multiplies) is rare;
//  * P is packed with v_cvt_pk_bf16_f32 (round to nearest even); O is
//    divided by the row sum once at the end, rounded once, and leaves
//    through a per-wave LDS region as whole rows (not 8-byte pieces of 32
//    rows per store instruction);
//  * registers: this file is compiled with MFMA results in VGPRs
//    (-amdgpu-mfma-vgpr-form), which keeps the scores, P and O out of
//    AGPR<->VGPR copies (226 VGPRs, two waves per SIMD);
//  * causal: key tiles past the query tile are never loaded; a 32-query block
//    skips tiles entirely above its diagonal; heads are split over the XCDs
//    (all query tiles of a head on one XCD: K/V shared in its L2), each
//    XCD's items are dealt a block of heads at a time, heaviest first, in a
//    snake order, so every CU gets the same number of key tiles (272 of
//    69632 at B4 H32 S4096) and an XCD's CUs share few heads' K/V at a time.

#include "../launch.h"
#include "device_common.h"

namespace grxk {
namespace {

constexpr int kNW = 8;          // wavefronts per workgroup (two per SIMD)
constexpr int kBQ = 32 * kNW;   // queries per workgroup, 32 per wave
constexpr int kBK = 64;   // keys per tile
constexpr int kNS = 3;    // K/V tile stages in LDS (96 KB at head dim 128)
constexpr int kQkAhead = 4;  // K fragments read ahead of the score MFMAs
static_assert(kNS == 3, "the tile loop below is unrolled for three stages");
constexpr uint32_t kRsrcWord3 = 0x00020000u;
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4* lds_s16x4_t;
template <int N> struct Stage { static constexpr int value = N; };

// Buffer descriptor words: 48-bit base, stride 0, num_records bytes (reads
// past it return zero), raw-buffer format word.
__device__ __forceinline__ i32x4 rsrc_words(const void* base, uint32_t num_records) {
  const uint64_t a = (uint64_t)base;
  return i32x4{(int)(uint32_t)a, (int)(uint32_t)(a >> 32) & 0xffff, (int)num_records, (int)kRsrcWord3};
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_ptr_t)p;
}
// 16 bytes per lane from global memory straight into LDS (lane L writes
// lds + 16*L). Issued as assembly so that the compiler does not see an LDS
// write: it would otherwise make every later transposing LDS read wait for
// ALL outstanding DMA, including the prefetch of the next tile. Ordering is
// explicit instead: each tile ends with s_waitcnt vmcnt(0) and a barrier
// before any wave reads the stage this DMA fills. M0 carries the LDS base:
// gfx950 needs one wait state between an M0 write and the LDS DMA that reads
// it (the s_nop; the compiler's hazard pass does not look inside inline
// assembly). M0 is a register the compiler reserves (a clobber naming it is
// ignored), so each DMA writes it itself; in the gfx950 code of this kernel
// and of gemm_tn128 no other instruction reads or writes M0.
// s_waitcnt vmcnt(0) through the builtin, so that the compiler's own wait
// bookkeeping also sees every earlier load as complete.
__device__ __forceinline__ void wait_vmem_all() {
  __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt 0, expcnt 7, lgkmcnt 15: wait on vmcnt only
  asm volatile("" ::: "memory");
}
__device__ __forceinline__ void dma16(i32x4 rsrc, uint32_t lds, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(lds), "v"(voff), "s"(rsrc) : "memory");
}
// The same with a wave-uniform byte offset in the instruction's soffset. The
// buffer's range check sees only the per-lane offset, so this form is for
// rows known to lie inside the tensor.
__device__ __forceinline__ void dma16_so(i32x4 rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds), "v"(voff), "s"(rsrc), "s"(soff) : "memory");
}

template <AttnType T> struct AIo;
template <> struct AIo<AttnType::BF16> {
  __device__ static f32x16 mma(i32x4 a, i32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // two fp32 -> packed bf16 (RNE, v_cvt_pk_bf16_f32)
  __device__ static uint32_t pack2(float a, float b) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
  // acc + the two packed values (v_dot2_f32_bf16 against (1, 1))
  __device__ static float sum2(uint32_t packed, float acc) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, packed), one, acc, false);
  }
};
template <> struct AIo<AttnType::F16> {
  __device__ static f32x16 mma(i32x4 a, i32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float a, float b) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    const f16x2 v = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, v);
  }
  __device__ static float sum2(uint32_t packed, float acc) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, packed), one, acc, false);
  }
};

struct AParams {
  const uint8_t* q; const uint8_t* k; const uint8_t* v; uint8_t* o;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int B, H, S;
  int qtiles;
  int heads;      // B * H
  int causal;
  float c;  // scale * log2(e)
  grxCycleSlot* probe;   // one slot per wave, or null
};

// K rows: ds_read_b128 of one logical chunk by 32 consecutive rows must hit
// distinct banks; V rows: the 8 keys x 4 chunks of one transposing read must
// spread evenly. Both are XOR swizzles of the 16-byte chunk index.
template <int D> __device__ __forceinline__ int kswz(int row) {
  if constexpr (D == 128) return row & 15;
  else return (row ^ (row >> 3)) & 7;
}
template <int D> __device__ __forceinline__ int vswz(int row) {
  if constexpr (D == 128) return 4 * (row & 3);
  else return 4 * ((row >> 1) & 1);
}

// Value from the other half of the wave (lane ^ 32): v_permlane32_swap
// exchanges the upper half of its first operand with the lower half of its
// second; with both operands = x, lane l of the two results holds x[l] and
// x[l ^ 32] in some order.
__device__ __forceinline__ float half_swap_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_swap_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// One work item = one (batch, head) and one tile of kBQ queries. Items are
// split over the 8 XCDs by head (head h on XCD h % 8, so one head's K/V stay
// in one L2). Inside an XCD, round r deals the items of the next block of
// heads (as many heads as one round has workgroups for their query tiles:
// 2 at 32 workgroups and 16 tiles), heaviest (causal: last) query tile
// first, to the XCD's workgroups in a snake order, left to right for even r
// and right to left for odd r: two rounds give every workgroup the same
// number of key tiles, and the workgroups of an XCD share few heads' K/V at
// a time (B4 H32 S4096: FETCH_SIZE 564 MB per launch, against 1420 MB when
// a round took the heaviest tiles of all 16 heads of the XCD).
struct ItemMap {
  int xcd, wg, nwg;     // this workgroup's XCD, index within it, workgroups per XCD
  int hx;               // heads on this XCD
};
__device__ __forceinline__ bool item_at(const AParams& p, const ItemMap& m, int round,
                                        int* bh, int* qt) {
  const int nloc = m.hx * p.qtiles;
  const int k = (round & 1) ? (m.nwg - 1 - m.wg) : m.wg;
  const int j = round * m.nwg + k;
  if (j >= nloc || m.hx == 0) return false;
  int hb = m.nwg / p.qtiles;          // heads per block
  if (hb < 1) hb = 1;
  if (hb > m.hx) hb = m.hx;
  const int blk_items = hb * p.qtiles;
  const int blk = j / blk_items;
  const int r2 = j - blk * blk_items;
  const int hb_here = min(hb, m.hx - blk * hb);   // the last block may hold fewer
  const int rank = r2 / hb_here;                  // weight rank: 0 = heaviest
  const int hl = blk * hb + r2 % hb_here;
  *bh = m.xcd + 8 * hl;
  *qt = p.causal ? (p.qtiles - 1 - rank) : rank;
  return true;
}

template <AttnType T, int D>
__global__ __launch_bounds__(64 * kNW, 1) void attn_fwd(AParams p) {
  using IO = AIo<T>;
  constexpr int CH = D / 8;
  constexpr int RPI = 64 / CH;
  constexpr int IPW = kBK / RPI / kNW;
  constexpr int DSTEPS = D / 16;
  constexpr int DT = D / 32;
  static_assert(IPW >= 1, "tile too small for the wave count");
  __shared__ __attribute__((aligned(1024))) i32x4 lds[kNS][2][kBK * CH];
  // Each wave's O tile (32 rows of D values) passes through here on its way
  // out, so that every global store writes whole rows (8 KB per wave at
  // D = 128; 160 KB of LDS in all).
  __shared__ __attribute__((aligned(1024))) i32x4 ost[kNW][32 * CH];

  const uint64_t t_start = cycle_now();
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  ItemMap map;
  map.xcd = blockIdx.x & 7;
  map.wg = blockIdx.x >> 3;
  map.nwg = gridDim.x >> 3;
  map.hx = p.heads / 8 + (map.xcd < (p.heads & 7) ? 1 : 0);

  const uint32_t q_rs = (uint32_t)(2 * p.q_ss), k_rs = (uint32_t)(2 * p.k_ss), v_rs = (uint32_t)(2 * p.v_ss);
  uint32_t kbase[IPW], vbase[IPW];
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int blk = IPW * wave + i;
    const int row = RPI * blk + lane / CH;
    const int pc = lane % CH;
    kbase[i] = (uint32_t)row * k_rs + (uint32_t)(16 * (pc ^ kswz<D>(row)));
    vbase[i] = (uint32_t)row * v_rs + (uint32_t)(16 * (pc ^ vswz<D>(row)));
  }

  // Per-item state: head pointers, buffer descriptors, tile count.
  struct St {
    int q0, ntiles;
    const uint8_t* qg;
    uint8_t* og;
    i32x4 rk, rv;
  };
  auto setup = [&](int bh, int qt, St& s) {
    const int b = bh / p.H, h = bh % p.H;
    s.q0 = qt * kBQ;
    s.qg = p.q + 2 * (b * p.q_sb + h * p.q_sh);
    const uint8_t* kg = p.k + 2 * (b * p.k_sb + h * p.k_sh);
    const uint8_t* vg = p.v + 2 * (b * p.v_sb + h * p.v_sh);
    s.og = p.o + 2 * (b * p.o_sb + h * p.o_sh);
    s.rk = rsrc_words(kg, (uint32_t)(p.S - 1) * k_rs + 2 * D);
    s.rv = rsrc_words(vg, (uint32_t)(p.S - 1) * v_rs + 2 * D);
    const int kv_end = p.causal ? min(p.S, s.q0 + kBQ) : p.S;
    s.ntiles = (kv_end + kBK - 1) / kBK;
  };
  auto load_q = [&](const St& s, i32x4 (&qf)[DSTEPS]) {
    const int myq = s.q0 + 32 * wave + l32;
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        (void*)s.qg, (short)0, (int)((uint32_t)(p.S - 1) * q_rs + 2 * D), kRsrcWord3);
#pragma unroll
    for (int t = 0; t < DSTEPS; ++t)
      qf[t] = __builtin_amdgcn_raw_buffer_load_b128(
          rq, (uint32_t)myq * q_rs + (uint32_t)(2 * (16 * t + 8 * hh)), 0, 0);
  };
  // DMA of tile t of item s into LDS stage st (K and V).
  auto dma_tile = [&](const St& s, int t, int st) {
    const int kv0 = t * kBK;
    if (kv0 + kBK <= p.S) {
      const uint32_t ks = (uint32_t)kv0 * k_rs, vs = (uint32_t)kv0 * v_rs;
#pragma unroll
      for (int i = 0; i < IPW; ++i) {
        const int blk = IPW * wave + i;
        dma16_so(s.rk, lds_addr(&lds[st][0][blk * 64]), kbase[i], ks);
        dma16_so(s.rv, lds_addr(&lds[st][1][blk * 64]), vbase[i], vs);
      }
    } else {
#pragma unroll
      for (int i = 0; i < IPW; ++i) {
        const int blk = IPW * wave + i;
        dma16(s.rk, lds_addr(&lds[st][0][blk * 64]), (uint32_t)kv0 * k_rs + kbase[i]);
        dma16(s.rv, lds_addr(&lds[st][1][blk * 64]), (uint32_t)kv0 * v_rs + vbase[i]);
      }
    }
  };

  int round = 0, bh = 0, qt = 0;
  if (!item_at(p, map, round, &bh, &qt)) return;
  St cur;
  setup(bh, qt, cur);
  // DMA pointer: tile pft of item pround (state pf), kNS-1 tiles ahead of
  // the tile being computed, running on into the next items.
  int pround = 0, pft = 0;
  St pf = cur;
  bool pvalid = true;
  auto advance = [&]() {
    if (++pft == pf.ntiles) {
      int b2 = 0, q2 = 0;
      if (item_at(p, map, pround + 1, &b2, &q2)) {
        ++pround;
        setup(b2, q2, pf);
        pft = 0;
      } else {
        pvalid = false;
      }
    }
  };

  i32x4 qf[DSTEPS];
  load_q(cur, qf);
#pragma unroll
  for (int s0 = 0; s0 < kNS - 1; ++s0) {
    if (pvalid) {
      dma_tile(pf, pft, s0);
      advance();
    }
  }
  wait_vmem_all();
  __syncthreads();

  f32x16 o_acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[i][r] = 0.0f;
  float m_run = -INFINITY;
  float l_run = 0.0f;

  const int tr_key = 4 * hh + ((lane & 15) >> 2);
  const int tr_d = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  int t = 0;          // tile of the current item
  bool done = false;
  // One 64-key tile of the current item from LDS stage `stage`, while the
  // tile kNS-1 ahead (of this item or the next ones) loads into the stage
  // the previous tile used. After an item's last tile its O is written and
  // the next item's Q fragments are loaded.
  auto tile = [&](auto stage) {
    constexpr int cs = decltype(stage)::value;
    const bool last = (t + 1 == cur.ntiles);
    if (pvalid) {
      dma_tile(pf, pft, (cs + kNS - 1) % kNS);
      advance();
    }
    const int kv0 = t * kBK;
    const int wq0 = cur.q0 + 32 * wave;
    const int myq = wq0 + l32;
    const i32x4* kt = &lds[cs][0][0];
    const uint8_t* vt = (const uint8_t*)&lds[cs][1][0];
    const bool wave_live = !p.causal || kv0 <= wq0 + 31;
    if (wave_live) {
      // S^T for keys 0-31 and 32-63: two independent accumulation chains,
      // issued alternately, with the K fragments read kQkAhead MFMAs ahead
      // of their use (the schedule is pinned below: left to itself the
      // compiler reads each fragment just before its MFMA and waits for it,
      // 4-5 % slower).
      f32x16 s[2];
      {
        i32x4 kf[DSTEPS][2];
#pragma unroll
        for (int d = 0; d < DSTEPS; ++d)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) {
            const int row = kb * 32 + l32;
            kf[d][kb] = kt[row * CH + ((2 * d + hh) ^ kswz<D>(row))];
          }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
#pragma unroll
        for (int d = 0; d < DSTEPS; ++d)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) s[kb] = IO::mma(kf[d][kb], qf[d], s[kb]);
      }
      // instruction groups, in order: kQkAhead LDS reads, then alternately
      // one MFMA and one read, then the last kQkAhead MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, kQkAhead, 0);
#pragma unroll
      for (int i = 0; i < 2 * DSTEPS - kQkAhead; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, kQkAhead, 0);
      const bool need_mask = (kv0 + kBK > p.S) || (p.causal && kv0 + kBK - 1 > wq0);
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kv0 + kb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
            const bool masked = key >= p.S || (p.causal && key > myq);
            s[kb][r] = masked ? -INFINITY : s[kb][r];
          }
      }
      uint32_t pk[2][8];
      {
        float mx0 = -INFINITY, mx1 = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          mx0 = fmaxf(mx0, s[0][r]);
          mx1 = fmaxf(mx1, s[1][r]);
        }
        const float mx = half_swap_max(fmaxf(mx0, mx1)) * p.c;
        const bool raise = mx > m_run + 8.0f;
        if (__builtin_amdgcn_ballot_w64(raise)) {
          const float m_new = raise ? mx : m_run;
          const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
          m_run = m_new;
          l_run *= alpha;
#pragma unroll
          for (int i = 0; i < DT; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) o_acc[i][r] *= alpha;
        }
        const float m = m_run;
        float ps0 = 0.0f, ps1 = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int r = 0; r < 16; r += 2) {
            const float p0 = __builtin_amdgcn_exp2f(fmaf(s[kb][r], p.c, -m));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(s[kb][r + 1], p.c, -m));
            pk[kb][r >> 1] = IO::pack2(p0, p1);
            if (kb == 0) ps0 = IO::sum2(pk[kb][r >> 1], ps0);
            else ps1 = IO::sum2(pk[kb][r >> 1], ps1);
          }
        l_run += ps0 + ps1;
      }
#pragma unroll
      for (int st = 0; st < kBK / 16; ++st) {
        const int kb = st >> 1, half = st & 1;
        const i32x4 pf4 = i32x4{(int)pk[kb][4 * half + 0], (int)pk[kb][4 * half + 1],
                                (int)pk[kb][4 * half + 2], (int)pk[kb][4 * half + 3]};
        const int k1 = 16 * st + tr_key, k2 = k1 + 8;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int d = 32 * dt + tr_d;
          const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4_t)(vt + k1 * (2 * D) + 16 * ((d >> 3) ^ vswz<D>(k1)) + 2 * (d & 7)));
          const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4_t)(vt + k2 * (2 * D) + 16 * ((d >> 3) ^ vswz<D>(k2)) + 2 * (d & 7)));
          const u32x2 w0 = __builtin_bit_cast(u32x2, v0), w1 = __builtin_bit_cast(u32x2, v1);
          const i32x4 vf = i32x4{(int)w0.x, (int)w0.y, (int)w1.x, (int)w1.y};
          o_acc[dt] = IO::mma(vf, pf4, o_acc[dt]);
        }
      }
    }
    if (last) {
      // O[q, d] = O^T[d, q] / l for this item; then start the next one.
      const float l_tot = half_swap_sum(l_run);
      const float inv_l = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
      // A lane holds 4-value pieces of its query's row, 16 of them spread
      // over the row; stored as they are, one instruction writes 8 bytes in
      // each of 32 rows. Instead the wave parks the rounded tile in its LDS
      // region ([row][16-byte chunk], chunk XOR row) and reads it back as
      // whole rows, RPI rows per instruction (+1.5-2.2 %; non-temporal
      // stores measured the same).
      {
        uint8_t* my = (uint8_t*)&ost[wave][0];
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int c = (4 * dt + g) ^ (l32 & (CH - 1));
            u32x2 w;
            w.x = IO::pack2(o_acc[dt][4 * g + 0] * inv_l, o_acc[dt][4 * g + 1] * inv_l);
            w.y = IO::pack2(o_acc[dt][4 * g + 2] * inv_l, o_acc[dt][4 * g + 3] * inv_l);
            *(u32x2*)(my + 16 * (l32 * CH + c) + 8 * hh) = w;
          }
        // LDS operations of one wave complete in order; the compiler only
        // must not move the reads above the writes.
        asm volatile("" ::: "memory");
        const int rr = lane / CH, cc = lane % CH;
        // Rows at or past S lie outside the descriptor's range: the buffer
        // store drops them.
        const uint32_t o_rs = (uint32_t)(2 * p.o_ss);
        const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
            (void*)cur.og, (short)0, (int)((uint32_t)(p.S - 1) * o_rs + 2 * D), kRsrcWord3);
        const uint32_t vo = (uint32_t)(cur.q0 + 32 * wave + rr) * o_rs + 16 * cc;
#pragma unroll
        for (int i = 0; i < 32 / RPI; ++i) {
          const int r = RPI * i + rr;
          const i32x4 v = *(const i32x4*)(my + 16 * (r * CH + (cc ^ (r & (CH - 1)))));
          __builtin_amdgcn_raw_buffer_store_b128(v, ro, vo + (uint32_t)(RPI * i) * o_rs, 0, 0);
        }
        asm volatile("" ::: "memory");
      }
#pragma unroll
      for (int i = 0; i < DT; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o_acc[i][r] = 0.0f;
      m_run = -INFINITY;
      l_run = 0.0f;
      int nbh = 0, nqt = 0;
      if (item_at(p, map, round + 1, &nbh, &nqt)) {
        setup(nbh, nqt, cur);
        load_q(cur, qf);   // waited for below, with the DMA
        ++round;
        t = 0;
      } else {
        done = true;
      }
    } else {
      ++t;
    }
    wait_vmem_all();
    __syncthreads();
  };
  while (true) {
    tile(Stage<0>{});
    if (done) break;
    tile(Stage<1>{});
    if (done) break;
    tile(Stage<2>{});
    if (done) break;
  }
  cycle_record(p.probe, t_start, blockIdx.x * kNW + wave, wave);
}

// One workgroup per CU, a multiple of 8 (one share per XCD), no more than
// the items need.
int64_t workgroups(int B, int H, int S) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess)
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t qtiles = (S + kBQ - 1) / kBQ;
  int64_t wgs = (cus / 8) * 8;
  const int64_t per_xcd_items = ((int64_t)B * H + 7) / 8 * qtiles;
  if (wgs / 8 > per_xcd_items) wgs = 8 * per_xcd_items;
  if (wgs < 8) wgs = 8;
  return wgs;
}

template <AttnType T, int D>
hipError_t run(const AttnDesc& d, hipStream_t s) {
  AParams p{};
  p.q = (const uint8_t*)d.q; p.k = (const uint8_t*)d.k; p.v = (const uint8_t*)d.v;
  p.o = (uint8_t*)d.o;
  p.q_sb = d.q_sb; p.q_sh = d.q_sh; p.q_ss = d.q_ss;
  p.k_sb = d.k_sb; p.k_sh = d.k_sh; p.k_ss = d.k_ss;
  p.v_sb = d.v_sb; p.v_sh = d.v_sh; p.v_ss = d.v_ss;
  p.o_sb = d.o_sb; p.o_sh = d.o_sh; p.o_ss = d.o_ss;
  p.B = d.B; p.H = d.H; p.S = d.S;
  p.qtiles = (d.S + kBQ - 1) / kBQ;
  p.heads = d.B * d.H;
  p.causal = d.causal ? 1 : 0;
  p.c = d.scale * 1.4426950408889634f;
  p.probe = d.probe;
  // Every buffer offset (Q, K and V loads, O stores) is 32-bit.
  int64_t pitch = d.q_ss > d.k_ss ? d.q_ss : d.k_ss;
  pitch = pitch > d.v_ss ? pitch : d.v_ss;
  pitch = pitch > d.o_ss ? pitch : d.o_ss;
  const int64_t span = ((int64_t)d.S + kBQ) * 2 * pitch + 2 * d.D;
  if (span >= (1ll << 31)) return hipErrorNotSupported;
  // item indices are 32-bit in the kernel
  if ((int64_t)d.B * d.H * p.qtiles > 0x7fffffff) return hipErrorInvalidValue;
  const int64_t wgs = workgroups(d.B, d.H, d.S);
  hipLaunchKernelGGL((attn_fwd<T, D>), dim3((unsigned)wgs), dim3(64 * kNW), 0, s, p);
  return hipGetLastError();
}

}  // namespace

int64_t attention_probe_slots(int B, int H, int S) { return workgroups(B, H, S) * kNW; }

hipError_t launch_attention(AttnType t, const AttnDesc& d, hipStream_t s) {
  if (t == AttnType::BF16) {
    if (d.D == 128) return run<AttnType::BF16, 128>(d, s);
    if (d.D == 64) return run<AttnType::BF16, 64>(d, s);
  } else {
    if (d.D == 128) return run<AttnType::F16, 128>(d, s);
    if (d.D == 64) return run<AttnType::F16, 64>(d, s);
  }
  return hipErrorNotSupported;
}

}  // namespace grxk
