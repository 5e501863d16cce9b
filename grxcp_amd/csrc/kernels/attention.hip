// grxDNN fused scaled-dot-product attention (forward) on gfx950.
//
// New: the reference plans attention for grxDNN but ships no code
// (ref docs/designs/grxcp_roadmap.md:864-877). Single pass, online softmax,
// O(S) memory:
//
//  * one workgroup = 4 wavefronts = 128 query rows of one (batch, head); each
//    wave owns 32 queries whose Q fragment (32 x D bf16) stays in VGPRs;
//  * K and V stream through LDS in 64-key tiles, double-buffered with the
//    next tile's global loads in flight during the current tile's math;
//  * scores are computed TRANSPOSED, S^T = K Q^T (v_mfma_f32_32x32x16): the
//    accumulator then holds, per lane, 32 keys of ONE query, so the softmax
//    row max/sum is an in-register reduction plus one exchange with the lane
//    32 away, instead of a 32-lane shuffle tree;
//  * O^T += V^T P^T (v_mfma again): P^T is already in the B-operand layout in
//    the lanes that computed it (no LDS round trip for P); V is written to LDS
//    transposed (key-contiguous, padded rows) so the A operand is two
//    ds_read_b64 per step;
//  * softmax in the exp2 domain: p = exp2(s*scale*log2e - m), with m tracked
//    on raw scores; fp32 throughout; O is divided by the row sum once at the
//    end and rounded to bf16/fp16 (RNE) once;
//  * causal: key tiles past the query tile are never visited, only tiles that
//    cross the diagonal are masked; workgroups are ordered heaviest first and
//    all query tiles of a head run on one XCD (shared K/V in that XCD's L2).

#include "../launch.h"
#include "device_common.h"

namespace grxk {
namespace {

constexpr int kBQ = 128;          // queries per workgroup
constexpr int kBK = 64;           // keys per tile
constexpr int kVtPitch = kBK * 2 + 8;  // bytes per transposed-V row (padded)

template <AttnType T> struct AIo;
template <> struct AIo<AttnType::BF16> {
  __device__ static f32x16 mma(i32x4 a, i32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float a, float b) { return pack_bf16x2(a, b); }
};
template <> struct AIo<AttnType::F16> {
  __device__ static f32x16 mma(i32x4 a, i32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float a, float b) {
    return (uint32_t)f32_to_f16(a) | ((uint32_t)f32_to_f16(b) << 16);
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

template <AttnType T, int D>
__global__ __launch_bounds__(256, 2) void attn_fwd(AParams p) {
  using IO = AIo<T>;
  constexpr int DCH = D / 8;            // 16-byte chunks per K row
  constexpr int DSTEPS = D / 16;        // MFMA k-steps over the head dim
  constexpr int DT = D / 32;            // 32-wide output tiles over the head dim
  __shared__ __attribute__((aligned(16))) i32x4 ks[2][kBK * DCH];
  __shared__ __attribute__((aligned(16))) uint8_t vt[2][D * kVtPitch];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
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

  const uint8_t* qg = p.q + 2 * (b * p.q_sb + h * p.q_sh);
  const uint8_t* kg = p.k + 2 * (b * p.k_sb + h * p.k_sh);
  const uint8_t* vg = p.v + 2 * (b * p.v_sb + h * p.v_sh);
  uint8_t* og = p.o + 2 * (b * p.o_sb + h * p.o_sh);

  // Q fragment (B operand of S^T = K Q^T): query q0 + 32*wave + l32,
  // head-dim elements 16*t + 8*hh .. +7.
  const int myq = q0 + wave * 32 + l32;
  i32x4 qf[DSTEPS];
#pragma unroll
  for (int t = 0; t < DSTEPS; ++t) {
    qf[t] = i32x4{0, 0, 0, 0};
    if (myq < p.S) qf[t] = *(const i32x4*)(qg + 2 * ((int64_t)myq * p.q_ss + 16 * t + 8 * hh));
  }

  const int kv_end = p.causal ? min(p.S, q0 + kBQ) : p.S;
  const int ntiles = (kv_end + kBK - 1) / kBK;

  // K loader: 64 rows x DCH chunks, swizzled chunk = c ^ (row & 15).
  constexpr int KCH_PER_T = kBK * DCH / 256;
  // V loader: key pair kp (0..31) x head-dim chunk dc: reads keys 2kp, 2kp+1
  // and writes 8 packed (key, key+1) words into the transposed tile.
  constexpr int VT_PER_T = (kBK / 2) * DCH / 256;
  i32x4 kr[KCH_PER_T];
  i32x4 vr[VT_PER_T][2];

  auto load_tile = [&](int t) {
    const int kv0 = t * kBK;
#pragma unroll
    for (int i = 0; i < KCH_PER_T; ++i) {
      const int e = tid + 256 * i;
      const int row = e / DCH, c = e % DCH;
      const int key = kv0 + row;
      kr[i] = i32x4{0, 0, 0, 0};
      if (key < p.S) kr[i] = *(const i32x4*)(kg + 2 * ((int64_t)key * p.k_ss + 8 * c));
    }
#pragma unroll
    for (int i = 0; i < VT_PER_T; ++i) {
      const int e = tid + 256 * i;
      const int kp = e % (kBK / 2), dc = e / (kBK / 2);
      const int key = kv0 + 2 * kp;
      vr[i][0] = i32x4{0, 0, 0, 0};
      vr[i][1] = i32x4{0, 0, 0, 0};
      if (key < p.S) vr[i][0] = *(const i32x4*)(vg + 2 * ((int64_t)key * p.v_ss + 8 * dc));
      if (key + 1 < p.S) vr[i][1] = *(const i32x4*)(vg + 2 * ((int64_t)(key + 1) * p.v_ss + 8 * dc));
    }
  };
  auto store_tile = [&](int st) {
#pragma unroll
    for (int i = 0; i < KCH_PER_T; ++i) {
      const int e = tid + 256 * i;
      const int row = e / DCH, c = e % DCH;
      ks[st][row * DCH + (c ^ ((row & 15) % DCH))] = kr[i];
    }
#pragma unroll
    for (int i = 0; i < VT_PER_T; ++i) {
      const int e = tid + 256 * i;
      const int kp = e % (kBK / 2), dc = e / (kBK / 2);
      const u32x4 a = __builtin_bit_cast(u32x4, vr[i][0]);
      const u32x4 c = __builtin_bit_cast(u32x4, vr[i][1]);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const uint32_t lo = (a[w] & 0xffffu) | (c[w] << 16);
        const uint32_t hi = (a[w] >> 16) | (c[w] & 0xffff0000u);
        *(uint32_t*)(vt[st] + (8 * dc + 2 * w) * kVtPitch + 4 * kp) = lo;
        *(uint32_t*)(vt[st] + (8 * dc + 2 * w + 1) * kVtPitch + 4 * kp) = hi;
      }
    }
  };

  f32x16 o_acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_acc[i][r] = 0.0f;
  float m_run = -INFINITY;  // running max of raw scores for query myq
  float l_run = 0.0f;       // this half-wave's share of the running sum

  if (ntiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int cur = t & 1;
    const bool more = t + 1 < ntiles;
    if (more) load_tile(t + 1);
    const int kv0 = t * kBK;

    // S^T tile: two 32-key blocks x 32 queries.
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
      const int row = kb * 32 + l32;
#pragma unroll
      for (int d = 0; d < DSTEPS; ++d) {
        const int c = 2 * d + hh;
        const i32x4 kf = ks[cur][row * DCH + (c ^ ((row & 15) % DCH))];
        s[kb] = IO::mma(kf, qf[d], s[kb]);
      }
    }

    // Mask keys past the sequence end and (causal) past the query.
    const bool need_mask = (kv0 + kBK > p.S) || (p.causal && kv0 + kBK - 1 > q0 + wave * 32);
    if (need_mask) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kv0 + kb * 32 + 8 * (r >> 2) + 4 * hh + (r & 3);
          if (key >= p.S || (p.causal && key > myq)) s[kb][r] = -INFINITY;
        }
    }

    // Online softmax for this lane's query (other half of its keys in lane^32).
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f((m_run - m_use) * p.c);
    m_run = m_new;
    const float mc = m_use * p.c;
    float psum = 0.0f;
    uint32_t pk[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float p0 = __builtin_amdgcn_exp2f(fmaf(s[kb][r], p.c, -mc));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(s[kb][r + 1], p.c, -mc));
        psum += p0 + p1;
        pk[kb][r >> 1] = IO::pack2(p0, p1);
      }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int i = 0; i < DT; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) o_acc[i][r] *= alpha;

    // O^T += V^T P^T over the 64 keys, 16 keys per MFMA step.
#pragma unroll
    for (int st = 0; st < kBK / 16; ++st) {
      const int kb = st >> 1;
      const int half = st & 1;
      const i32x4 pf = i32x4{(int)pk[kb][4 * half + 0], (int)pk[kb][4 * half + 1],
                             (int)pk[kb][4 * half + 2], (int)pk[kb][4 * half + 3]};
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const uint8_t* vrow = vt[cur] + (dt * 32 + l32) * kVtPitch;
        const u32x2 v0 = *(const u32x2*)(vrow + 2 * (16 * st + 4 * hh));
        const u32x2 v1 = *(const u32x2*)(vrow + 2 * (16 * st + 8 + 4 * hh));
        const i32x4 vf = i32x4{(int)v0.x, (int)v0.y, (int)v1.x, (int)v1.y};
        o_acc[dt] = IO::mma(vf, pf, o_acc[dt]);
      }
    }

    if (more) store_tile(cur ^ 1);
    __syncthreads();
  }

  // O[myq, d] = O^T[d, myq] / l; lane holds d = 32*dt + 8*g + 4*hh + 0..3.
  const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
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
  const int64_t blocks = (int64_t)d.B * d.H * p.qtiles;
  if (blocks > 0x7fffffff) return hipErrorInvalidValue;
  hipLaunchKernelGGL((attn_fwd<T, D>), dim3((unsigned)blocks), dim3(256), 0, s, p);
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
