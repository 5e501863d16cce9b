// grxDNN fused scaled-dot-product attention (forward) on gfx950.
//
// New: the reference plans attention for grxDNN but ships no code
// (ref docs/designs/grxcp_roadmap.md:864-877). Single pass, online softmax,
// O(S) memory:
//
//  * one workgroup = 8 wavefronts (two per SIMD) = 256 query rows of one
//    (batch, head); each wave owns 32 queries whose Q fragments stay in
//    VGPRs for the whole pass;
//  * K and V stream through LDS in 64-key tiles by direct-to-LDS buffer loads
//    (no staging registers; rows past the sequence read as zero), double
//    buffered, the next tile's loads in flight during the current tile;
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
//    divided by the row sum once at the end and rounded once;
//  * registers: this file is compiled with MFMA results in VGPRs
//    (-amdgpu-mfma-vgpr-form), which keeps the scores, P and O out of
//    AGPR<->VGPR copies (194 VGPRs, two waves per SIMD);
//  * causal: key tiles past the query tile are never loaded; a 32-query block
//    skips tiles entirely above its diagonal; workgroups run heaviest first,
//    and all query tiles of a head run on one XCD (K/V shared in its L2).

#include "../launch.h"
#include "device_common.h"

namespace grxk {
namespace {

constexpr int kNW = 8;          // wavefronts per workgroup (two per SIMD)
constexpr int kBQ = 32 * kNW;   // queries per workgroup, 32 per wave
constexpr int kBK = 64;   // keys per tile
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
  int causal;
  float c;  // scale * log2(e)
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

template <AttnType T, int D>
__global__ __launch_bounds__(64 * kNW, 1) void attn_fwd(AParams p) {
  using IO = AIo<T>;
  constexpr int CH = D / 8;            // 16-byte chunks per row
  constexpr int RPI = 64 / CH;         // rows per 1 KB DMA instruction
  constexpr int IPW = kBK / RPI / kNW; // DMA instructions per wave per tensor per tile
  constexpr int DSTEPS = D / 16;       // MFMA k-steps over the head dim
  constexpr int DT = D / 32;           // 32-wide output tiles over the head dim
  static_assert(IPW >= 1, "tile too small for the wave count");
  // [stage][K | V][key * CH + physical chunk]
  __shared__ __attribute__((aligned(1024))) i32x4 lds[2][2][kBK * CH];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  // Work order: each XCD gets a contiguous run of logical ids (whole heads),
  // and inside a head the longest (last) query tiles come first.
  const int nb = gridDim.x;
  int logical = blockIdx.x;
  if ((nb & 7) == 0) logical = (blockIdx.x & 7) * (nb >> 3) + (blockIdx.x >> 3);
  const int bh = logical / p.qtiles;
  const int qt = p.causal ? (p.qtiles - 1 - logical % p.qtiles) : (logical % p.qtiles);
  const int b = bh / p.H, h = bh % p.H;
  const int q0 = qt * kBQ;
  const int wq0 = q0 + 32 * wave;  // this wave's first query

  const uint8_t* qg = p.q + 2 * (b * p.q_sb + h * p.q_sh);
  const uint8_t* kg = p.k + 2 * (b * p.k_sb + h * p.k_sh);
  const uint8_t* vg = p.v + 2 * (b * p.v_sb + h * p.v_sh);
  uint8_t* og = p.o + 2 * (b * p.o_sb + h * p.o_sh);
  // Byte pitches and offsets are unsigned 32-bit: the host guarantees one
  // head's rows span < 2^31 bytes; padding rows past S wrap harmlessly into
  // range checks that read zero.
  const uint32_t q_rs = (uint32_t)(2 * p.q_ss), k_rs = (uint32_t)(2 * p.k_ss), v_rs = (uint32_t)(2 * p.v_ss);

  // Row-ranged buffer descriptors: rows past S read as zero.
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
      (void*)qg, (short)0, (int)((uint32_t)(p.S - 1) * q_rs + 2 * D), kRsrcWord3);
  const i32x4 rk = rsrc_words(kg, (uint32_t)(p.S - 1) * k_rs + 2 * D);
  const i32x4 rv = rsrc_words(vg, (uint32_t)(p.S - 1) * v_rs + 2 * D);

  // Q fragments (B operand of S^T = K Q^T): query wq0 + l32, head-dim
  // elements 16*t + 8*hh .. +7.
  const int myq = wq0 + l32;
  i32x4 qf[DSTEPS];
#pragma unroll
  for (int t = 0; t < DSTEPS; ++t) {
    qf[t] = __builtin_amdgcn_raw_buffer_load_b128(
        rq, (uint32_t)myq * q_rs + (uint32_t)(2 * (16 * t + 8 * hh)), 0, 0);
  }

  const int kv_end = p.causal ? min(p.S, q0 + kBQ) : p.S;
  const int ntiles = (kv_end + kBK - 1) / kBK;

  // DMA: instruction i of wave w fills rows RPI*(IPW*w + i) .. of K or V;
  // lane L lands in row +L/CH at physical chunk L%CH.
  // The tile-invariant part of each DMA's offset (row within the tile and
  // swizzled chunk). A tile whose rows all lie inside the sequence takes it
  // with the tile's offset in soffset: no VALU work per DMA. The last,
  // ragged tile and the prefetch past the end keep the masked form, whose
  // per-lane offsets the buffer's range check turns into zeros.
  uint32_t kbase[IPW], vbase[IPW];
#pragma unroll
  for (int i = 0; i < IPW; ++i) {
    const int blk = IPW * wave + i;
    const int row = RPI * blk + lane / CH;
    const int pc = lane % CH;
    kbase[i] = (uint32_t)row * k_rs + (uint32_t)(16 * (pc ^ kswz<D>(row)));
    vbase[i] = (uint32_t)row * v_rs + (uint32_t)(16 * (pc ^ vswz<D>(row)));
  }
  auto dma_tile = [&](int t, int st) {
    const int kv0 = t * kBK;
    if (kv0 + kBK <= p.S) {
      const uint32_t ks = (uint32_t)kv0 * k_rs, vs = (uint32_t)kv0 * v_rs;
#pragma unroll
      for (int i = 0; i < IPW; ++i) {
        const int blk = IPW * wave + i;
        dma16_so(rk, lds_addr(&lds[st][0][blk * 64]), kbase[i], ks);
        dma16_so(rv, lds_addr(&lds[st][1][blk * 64]), vbase[i], vs);
      }
    } else {
#pragma unroll
      for (int i = 0; i < IPW; ++i) {
        const int blk = IPW * wave + i;
        const bool ok = t < ntiles;
        const uint32_t ko = ok ? (uint32_t)kv0 * k_rs + kbase[i] : 0x80000000u;
        const uint32_t vo = ok ? (uint32_t)kv0 * v_rs + vbase[i] : 0x80000000u;
        dma16(rk, lds_addr(&lds[st][0][blk * 64]), ko);
        dma16(rv, lds_addr(&lds[st][1][blk * 64]), vo);
      }
    }
  };

  f32x16 o_acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[i][r] = 0.0f;
  float m_run = -INFINITY;  // running max, scaled (log2) units
  float l_run = 0.0f;       // this half-wave's share of the sum

  dma_tile(0, 0);
  wait_vmem_all();  // Q fragments and the first tile
  __syncthreads();

  // Transposed-read addressing for V^T (A operand of O^T = V^T P^T): lane l
  // supplies head-dim row d = 32*dt + l32 and keys {16st + 4hh + r} (first
  // read) and {16st + 8 + 4hh + r} (second read), r = 0..3. Source lane
  // s = l%16 of its 16-lane group points at key 16st + 4hh + s/4 (+8),
  // head-dim 32*dt + 16*((l>>4)&1) + 4*(s&3).
  const int tr_key = 4 * hh + ((lane & 15) >> 2);
  const int tr_d = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  // One 64-key tile; the LDS stage is a compile-time constant so every LDS
  // address is a loop-invariant register plus an immediate offset.
  auto tile = [&](auto stage, int t) {
    constexpr int cur = decltype(stage)::value;
    dma_tile(t + 1, cur ^ 1);
    const int kv0 = t * kBK;
    const i32x4* kt = &lds[cur][0][0];
    const uint8_t* vt = (const uint8_t*)&lds[cur][1][0];

    // A wave whose 32 queries all precede this tile skips it (causal); the
    // DMA it issued above and the barrier below are still its share.
    const bool wave_live = !p.causal || kv0 <= wq0 + 31;
    if (wave_live) {
      // S^T tiles: [key block], 32 keys x 32 queries each. The K fragments
      // of a key block are all read before its MFMAs.
      f32x16 s[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int row = kb * 32 + l32;
        i32x4 kf[DSTEPS];
#pragma unroll
        for (int d = 0; d < DSTEPS; ++d) kf[d] = kt[row * CH + ((2 * d + hh) ^ kswz<D>(row))];
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
#pragma unroll
        for (int d = 0; d < DSTEPS; ++d) s[kb] = IO::mma(kf[d], qf[d], s[kb]);
      }

      // Keys past the sequence end, and (causal) past the query, are masked
      // only on tiles that can contain such keys for this wave.
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

      // Online softmax for this lane's query.
      uint32_t pk[2][8];
      {
        float mx0 = -INFINITY, mx1 = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          mx0 = fmaxf(mx0, s[0][r]);
          mx1 = fmaxf(mx1, s[1][r]);
        }
        const float mx = half_swap_max(fmaxf(mx0, mx1)) * p.c;
        // Raise the running max only when this tile exceeds it by > 8.
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
        // The row sum adds the ROUNDED probabilities (v_dot2 over the packed
        // pairs), the same values the O update multiplies.
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

      // O^T += V^T P^T, 16 keys per MFMA step.
#pragma unroll
      for (int st = 0; st < kBK / 16; ++st) {
        const int kb = st >> 1, half = st & 1;
        const i32x4 pf = i32x4{(int)pk[kb][4 * half + 0], (int)pk[kb][4 * half + 1],
                               (int)pk[kb][4 * half + 2], (int)pk[kb][4 * half + 3]};
        const int k1 = 16 * st + tr_key, k2 = k1 + 8;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int d = 32 * dt + tr_d;  // element column; 8-byte aligned
          const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4_t)(vt + k1 * (2 * D) + 16 * ((d >> 3) ^ vswz<D>(k1)) + 2 * (d & 7)));
          const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_s16x4_t)(vt + k2 * (2 * D) + 16 * ((d >> 3) ^ vswz<D>(k2)) + 2 * (d & 7)));
          const u32x2 w0 = __builtin_bit_cast(u32x2, v0), w1 = __builtin_bit_cast(u32x2, v1);
          const i32x4 vf = i32x4{(int)w0.x, (int)w0.y, (int)w1.x, (int)w1.y};
          o_acc[dt] = IO::mma(vf, pf, o_acc[dt]);
        }
      }
    }

    wait_vmem_all();  // next tile's DMA landed
    __syncthreads();
  };
  for (int t = 0; t < ntiles; t += 2) {
    tile(Stage<0>{}, t);
    if (t + 1 < ntiles) tile(Stage<1>{}, t + 1);
  }

  // O[q, d] = O^T[d, q] / l; lane holds d = 32*dt + 8*g + 4*hh + 0..3.
  const float l_tot = half_swap_sum(l_run);
  const float inv_l = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  if (myq < p.S) {
    uint8_t* orow = og + 2 * (int64_t)myq * p.o_ss;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = dt * 32 + 8 * g + 4 * hh;
        u32x2 w;
        w.x = IO::pack2(o_acc[dt][4 * g + 0] * inv_l, o_acc[dt][4 * g + 1] * inv_l);
        w.y = IO::pack2(o_acc[dt][4 * g + 2] * inv_l, o_acc[dt][4 * g + 3] * inv_l);
        *(u32x2*)(orow + 2 * d) = w;
      }
  }
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
  p.causal = d.causal ? 1 : 0;
  p.c = d.scale * 1.4426950408889634f;
  // 32-bit buffer offsets within one head: (S-1) * row pitch + row < 2^31.
  int64_t pitch = d.q_ss > d.k_ss ? d.q_ss : d.k_ss;
  pitch = pitch > d.v_ss ? pitch : d.v_ss;
  const int64_t span = ((int64_t)d.S + kBQ) * 2 * pitch + 2 * d.D;
  if (span >= (1ll << 31)) return hipErrorNotSupported;
  const int64_t blocks = (int64_t)d.B * d.H * p.qtiles;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((attn_fwd<T, D>), dim3((unsigned)blocks), dim3(64 * kNW), 0, s, p);
  return hipGetLastError();
}

}  // namespace

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
