// Internal interface between the host libraries (argument validation, status
// mapping) and the gfx950 kernels (one launcher per kernel family). Nothing
// here is exported from the shared libraries.
#ifndef GRXCP_LAUNCH_H
#define GRXCP_LAUNCH_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include <grx/grx_cycles.h>

namespace grxk {

// Element types the matrix-core GEMM reads and the epilogue it ends in.
enum class MmaIn { BF16, F16, I8, F32 };   // F32: Sgemm's large problems
enum class MmaOut {
  F32,        // alpha*acc + beta*C, fp32 C
  BF16,       // same, rounded to bf16 (RNE)
  F16,        // same, rounded to fp16 (RNE)
  I32,        // integral alpha/beta in int32, wrapping
  DEQ_BF16    // bf16(f32(acc) * scale[col])
};

struct GemmDesc {
  int m, n, k;
  bool ta, tb;              // op(A) = A^T / op(B) = B^T
  const void* a; int64_t lda;
  const void* b; int64_t ldb;
  void* c;       int64_t ldc;
  float alpha, beta;        // floating epilogues
  int32_t ialpha, ibeta;    // integer epilogue
  const float* scale;       // DEQ_BF16
  grxCycleSlot* probe;      // may be null
  int batch = 1;            // grid.y; batch b offsets a, b, c by b * stride
  int64_t stride_a = 0, stride_b = 0, stride_c = 0;  // elements, signed
  void* ws = nullptr;       // device workspace for transposed operand copies
  size_t ws_bytes = 0;
  // K not a multiple of 16 bytes (or an operand the TN kernels cannot read
  // as it lies) may be served by copies of both operands with K padded with
  // zeros, and C off 16-byte boundaries through raw partials in the
  // workspace; false keeps such a problem on the general path.
  bool pad_copies = true;
};

// Picks the kernel (TN fast path, TN fast path behind transposed copies of
// the operands that are not K-contiguous, or the general path) and launches.
hipError_t launch_mma_gemm(MmaIn in, MmaOut out, const GemmDesc& d, hipStream_t s);
// Workspace bytes launch_mma_gemm would use for d (0: it needs none). With a
// smaller d.ws_bytes the call takes the general path instead.
size_t gemm_workspace_bytes(MmaIn in, MmaOut out, const GemmDesc& d);
// The current device's scratch for grxblasGemmExNoAlloc (kNoAllocScratchBytes,
// a __device__ array in its own code object, resolved once per device) for
// one launch on stream s. The constructor takes the device's lock and makes
// s wait for the array's previous user on another stream; release(true)
// records the launch behind it and drops the lock. ptr() is null if the
// array cannot be resolved. Allocates nothing after the device's first call.
constexpr size_t kNoAllocScratchBytes = size_t(64) << 20;
class NoAllocScratch {
 public:
  explicit NoAllocScratch(hipStream_t s);
  ~NoAllocScratch();
  NoAllocScratch(const NoAllocScratch&) = delete;
  NoAllocScratch& operator=(const NoAllocScratch&) = delete;
  void* ptr() const { return ptr_; }
  hipError_t release(bool launched);

 private:
  hipStream_t stream_;
  int dev_ = -1;
  void* ptr_ = nullptr;
  bool captured_ = false;
};
// fp32 problem d (MmaIn::F32 -> MmaOut::F32, no probe) that fills the GPU
// with 256x256 tiles and can run the TN kernel, directly or behind copies.
bool fp32_mma_wanted(const GemmDesc& d);
// Upper bound of probe slots any GEMM launch for an m x n output uses.
int64_t gemm_probe_slots(int m, int n);

struct SgemmDesc {
  int m, n, k, batch;
  bool ta, tb;
  const float* a; int64_t lda; int64_t stride_a;
  const float* b; int64_t ldb; int64_t stride_b;
  float* c;       int64_t ldc; int64_t stride_c;
  float alpha, beta;
  grxCycleSlot* probe;
};
hipError_t launch_sgemm(const SgemmDesc& d, hipStream_t s);

// Level 1/2, fp32 (256-thread workgroups; with a probe, 4 slots per workgroup).
int64_t l1_blocks(int n);
int64_t sgemv_blocks(bool trans, int m, int n);
hipError_t launch_saxpy(int n, float alpha, const float* x, int incx, float* y,
                        int incy, grxCycleSlot* probe, hipStream_t s);
hipError_t launch_sscal(int n, float alpha, float* x, int incx, grxCycleSlot* probe,
                        hipStream_t s);
hipError_t launch_sgemv(bool trans, int m, int n, float alpha, const float* A,
                        int lda, const float* x, int incx, float beta, float* y,
                        int incy, grxCycleSlot* probe, hipStream_t s);

// grxDNN.
enum class NormType { BF16, F16, F32 };
struct NormDesc {
  int64_t rows;
  int hidden;
  int64_t x_row_stride, y_row_stride;  // elements
  const void* x; const void* gamma; const void* beta;  // beta: LayerNorm only
  void* y;
  float eps;
};
hipError_t launch_rmsnorm(NormType t, const NormDesc& d, hipStream_t s);
hipError_t launch_layernorm(NormType t, const NormDesc& d, hipStream_t s);

// Row-wise softmax over the last dimension and element-wise GELU.
struct RowDesc {
  int64_t rows;
  int hidden;
  int64_t x_row_stride, y_row_stride;  // elements
  const void* x;
  void* y;
};
hipError_t launch_softmax(NormType t, const RowDesc& d, hipStream_t s);
hipError_t launch_gelu(NormType t, bool tanh_form, const RowDesc& d, hipStream_t s);

enum class AttnType { BF16, F16 };
struct AttnDesc {
  int B, H, S, D;
  bool causal;
  float scale;
  const void* q; int64_t q_sb, q_sh, q_ss;   // strides (elements) of b, h, s
  const void* k; int64_t k_sb, k_sh, k_ss;
  const void* v; int64_t v_sb, v_sh, v_ss;
  void* o;       int64_t o_sb, o_sh, o_ss;
  grxCycleSlot* probe = nullptr;   // one slot per wave of the launch, or null
};
hipError_t launch_attention(AttnType t, const AttnDesc& d, hipStream_t s);
// Probe slots an attention launch of this shape uses on the current device
// (workgroups x waves per workgroup; slot = blockIdx * waves + wave).
int64_t attention_probe_slots(int B, int H, int S);

}  // namespace grxk

#endif  // GRXCP_LAUNCH_H
