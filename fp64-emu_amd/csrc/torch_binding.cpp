// PyTorch-ROCm operator registration for the fp64_emu ops.  The schemas are
// the reference's (torch-ext/torch_binding.cpp:7-12) and the argument checks
// raise its TORCH_CHECK messages (fp64_emu_cuda/fp64_emu.cu:1586-1600,
// 1616-1628, 1640-1654, 1668-1682, 1692-1693).  Each op validates, takes its
// scratch from the caching allocator on the current stream and calls the C
// ABI of include/fp64emu.h; nothing here computes.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <algorithm>
#include <vector>

#include "fp64emu.h"

namespace {

constexpr int64_t kMaxKSingle = 131071;
constexpr int64_t kMaxKDeep = (int64_t)128 * 65536;   // K-segmented bound (mm, bmm)

void check_status(int st) { TORCH_CHECK(st == FP64EMU_OK, fp64emu_last_error()); }

std::vector<int32_t> primes_vec(const at::Tensor& primes_cpu) {
  const at::Tensor pc = primes_cpu.to(at::kCPU, at::kInt).contiguous();
  const int32_t* p = pc.data_ptr<int32_t>();
  return std::vector<int32_t>(p, p + pc.numel());
}

at::Tensor workspace(const at::Tensor& like, size_t bytes) {
  return at::empty({(int64_t)std::max<size_t>(bytes, 1)}, like.options().dtype(at::kByte));
}

// The full workspace when the caching allocator can provide it; otherwise
// the largest of full/2, full/4, ... down to the minimum the library accepts
// (it then runs the rows of A in as few chunks as fit).  Only batch-1 calls
// with K <= 131071 have a smaller minimum; the others need the full size.
at::Tensor workspace_fit(const at::Tensor& like, size_t full, size_t minimum) {
  size_t want = full;
  while (want > minimum) {
    try {
      return workspace(like, want);
    } catch (const c10::OutOfMemoryError&) {
      want /= 2;
    }
  }
  return workspace(like, minimum);
}

fp64emu_stream_t current_stream(const at::Tensor& t) {
  return reinterpret_cast<fp64emu_stream_t>(
      c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_common(const at::Tensor& A, const at::Tensor& B, const char* dtype_msg,
                  const at::Tensor& primes_cpu, int64_t bits) {
  TORCH_CHECK(A.is_cuda() && B.is_cuda() && A.scalar_type() == at::kDouble &&
                  B.scalar_type() == at::kDouble,
              dtype_msg);
  TORCH_CHECK(A.device() == B.device(), "A and B must be on the same device");
  TORCH_CHECK(primes_cpu.numel() <= FP64EMU_MAXP, "too many primes");
  TORCH_CHECK(primes_cpu.numel() >= 1, "nprimes must be >= 1");
  TORCH_CHECK(bits >= 16 && bits <= 53, "bits must be in [16, 53]");
}

void check_out(const at::Tensor& out, const at::Tensor& A, at::IntArrayRef sizes,
               const char* msg) {
  TORCH_CHECK(out.scalar_type() == at::kDouble && out.sizes() == sizes && out.is_contiguous(),
              msg);
  TORCH_CHECK(out.device() == A.device(), "out must be on the device of A");
}

}  // namespace

int64_t fp64_emu_maxp() { return fp64emu_maxp(); }

// out[m,n] = A[m,k] @ B[n,k]^T.   fp64_emu_cuda/fp64_emu.cu:1583-1608
void fp64_emu_mm(at::Tensor& out, const at::Tensor& A, const at::Tensor& B,
                 const at::Tensor& primes_cpu, const at::Tensor& inv_cpu,
                 const at::Tensor& mu_cpu, bool exact, int64_t bits, bool use_corr) {
  (void)inv_cpu; (void)mu_cpu;
  check_common(A, B, "A,B must be f64 CUDA", primes_cpu, bits);
  TORCH_CHECK(A.dim() == 2 && B.dim() == 2 && A.is_contiguous() && B.is_contiguous(), "2D contig");
  const int64_t M = A.size(0), K = A.size(1), N = B.size(0);
  TORCH_CHECK(B.size(1) == K, "expect B as [N, K]");
  check_out(out, A, {M, N}, "out f64 [M,N]");
  // Deeper than 131071 runs K-segmented, to 128 segments of 65536.
  TORCH_CHECK(K <= kMaxKDeep, "K bound: 128 segments of 65536");
  const c10::DeviceGuard guard(A.device());
  const std::vector<int32_t> pv = primes_vec(primes_cpu);
  const int P = (int)pv.size();
  at::Tensor ws = workspace_fit(A, fp64emu_workspace_size(1, M, N, K, P, use_corr),
                                fp64emu_workspace_size_min(1, M, N, K, P, use_corr));
  check_status(fp64emu_mm(out.data_ptr<double>(), A.data_ptr<double>(), B.data_ptr<double>(), M,
                          N, K, pv.data(), nullptr, nullptr, P, exact, bits, use_corr,
                          ws.data_ptr(), (size_t)ws.numel(), current_stream(A)));
}

// out[m,n] = A[m,k] @ Bt[k,n], Bt in its [K, N] layout.
// fp64_emu_cuda/fp64_emu.cu:1613-1632
void fp64_emu_mm_nt(at::Tensor& out, const at::Tensor& A, const at::Tensor& Bt,
                    const at::Tensor& primes_cpu, const at::Tensor& inv_cpu,
                    const at::Tensor& mu_cpu, bool exact, int64_t bits, bool use_corr) {
  (void)inv_cpu; (void)mu_cpu;
  check_common(A, Bt, "A,Bt must be f64 CUDA", primes_cpu, bits);
  TORCH_CHECK(A.dim() == 2 && Bt.dim() == 2 && A.is_contiguous() && Bt.is_contiguous(),
              "2D contig");
  const int64_t M = A.size(0), K = A.size(1), N = Bt.size(1);
  TORCH_CHECK(Bt.size(0) == K, "expect Bt as [K, N]");
  check_out(out, A, {M, N}, "out f64 [M,N]");
  TORCH_CHECK(K <= kMaxKSingle, "K bound for int32 modular GEMM");
  const c10::DeviceGuard guard(A.device());
  const std::vector<int32_t> pv = primes_vec(primes_cpu);
  const int P = (int)pv.size();
  at::Tensor ws = workspace_fit(A, fp64emu_workspace_size(1, M, N, K, P, use_corr),
                                fp64emu_workspace_size_min(1, M, N, K, P, use_corr));
  check_status(fp64emu_mm_nt(out.data_ptr<double>(), A.data_ptr<double>(), Bt.data_ptr<double>(),
                             M, N, K, pv.data(), nullptr, nullptr, P, exact, bits, use_corr,
                             ws.data_ptr(), (size_t)ws.numel(), current_stream(A)));
}

// out[b,m,n] = A[b,m,k] @ B[b,n,k]^T.   fp64_emu_cuda/fp64_emu.cu:1637-1662
void fp64_emu_bmm(at::Tensor& out, const at::Tensor& A, const at::Tensor& B,
                  const at::Tensor& primes_cpu, const at::Tensor& inv_cpu,
                  const at::Tensor& mu_cpu, bool exact, int64_t bits, bool use_corr) {
  (void)inv_cpu; (void)mu_cpu;
  check_common(A, B, "A,B must be f64 CUDA", primes_cpu, bits);
  TORCH_CHECK(A.dim() == 3 && B.dim() == 3 && A.is_contiguous() && B.is_contiguous(), "3D contig");
  const int64_t batch = A.size(0), M = A.size(1), K = A.size(2), N = B.size(1);
  TORCH_CHECK(B.size(0) == batch && B.size(2) == K, "expect B as [batch, N, K]");
  check_out(out, A, {batch, M, N}, "out f64 [batch,M,N]");
  TORCH_CHECK(K <= kMaxKDeep, "K bound: 128 segments of 65536");
  const c10::DeviceGuard guard(A.device());
  const std::vector<int32_t> pv = primes_vec(primes_cpu);
  const int P = (int)pv.size();
  at::Tensor ws = workspace(A, fp64emu_workspace_size(batch, M, N, K, P, use_corr));
  check_status(fp64emu_bmm(out.data_ptr<double>(), A.data_ptr<double>(), B.data_ptr<double>(),
                           batch, M, N, K, pv.data(), nullptr, nullptr, P, exact, bits, use_corr,
                           ws.data_ptr(), (size_t)ws.numel(), current_stream(A)));
}

// out[b,m,n] = A[b,m,k] @ Bt[b,k,n].   fp64_emu_cuda/fp64_emu.cu:1665-1686
void fp64_emu_bmm_nt(at::Tensor& out, const at::Tensor& A, const at::Tensor& Bt,
                     const at::Tensor& primes_cpu, const at::Tensor& inv_cpu,
                     const at::Tensor& mu_cpu, bool exact, int64_t bits, bool use_corr) {
  (void)inv_cpu; (void)mu_cpu;
  check_common(A, Bt, "A,Bt must be f64 CUDA", primes_cpu, bits);
  TORCH_CHECK(A.dim() == 3 && Bt.dim() == 3 && A.is_contiguous() && Bt.is_contiguous(),
              "3D contig");
  const int64_t batch = A.size(0), M = A.size(1), K = A.size(2), N = Bt.size(2);
  TORCH_CHECK(Bt.size(0) == batch && Bt.size(1) == K, "expect Bt as [batch, K, N]");
  check_out(out, A, {batch, M, N}, "out f64 [batch,M,N]");
  TORCH_CHECK(K <= kMaxKSingle, "K bound for int32 modular GEMM");
  const c10::DeviceGuard guard(A.device());
  const std::vector<int32_t> pv = primes_vec(primes_cpu);
  const int P = (int)pv.size();
  at::Tensor ws = workspace(A, fp64emu_workspace_size(batch, M, N, K, P, use_corr));
  check_status(fp64emu_bmm_nt(out.data_ptr<double>(), A.data_ptr<double>(),
                              Bt.data_ptr<double>(), batch, M, N, K, pv.data(), nullptr, nullptr,
                              P, exact, bits, use_corr, ws.data_ptr(), (size_t)ws.numel(),
                              current_stream(A)));
}

// mm with phase times [scale+extract, gemms, marker, reconstruct] in ms.
// fp64_emu_cuda/fp64_emu.cu:1688-1704 (plus the dtype/shape checks it lacks).
void fp64_emu_mm_timed(at::Tensor& out, at::Tensor& times, const at::Tensor& A,
                       const at::Tensor& B, const at::Tensor& primes_cpu,
                       const at::Tensor& inv_cpu, const at::Tensor& mu_cpu, bool exact,
                       int64_t bits, bool use_corr) {
  (void)inv_cpu; (void)mu_cpu;
  check_common(A, B, "A,B must be f64 CUDA", primes_cpu, bits);
  TORCH_CHECK(A.dim() == 2 && B.dim() == 2 && A.is_contiguous() && B.is_contiguous(), "2D contig");
  const int64_t M = A.size(0), K = A.size(1), N = B.size(0);
  TORCH_CHECK(B.size(1) == K, "expect B as [N, K]");
  check_out(out, A, {M, N}, "out f64 [M,N]");
  TORCH_CHECK(K <= kMaxKSingle, "K bound for int32 modular GEMM");
  TORCH_CHECK(times.device().is_cpu() && times.scalar_type() == at::kFloat &&
                  times.numel() >= 4 && times.is_contiguous(),
              "times must be a CPU float32 tensor of 4");
  const c10::DeviceGuard guard(A.device());
  const std::vector<int32_t> pv = primes_vec(primes_cpu);
  const int P = (int)pv.size();
  at::Tensor ws = workspace(A, fp64emu_workspace_size(1, M, N, K, P, use_corr));
  check_status(fp64emu_mm_timed(out.data_ptr<double>(), times.data_ptr<float>(),
                                A.data_ptr<double>(), B.data_ptr<double>(), M, N, K, pv.data(),
                                nullptr, nullptr, P, exact, bits, use_corr, ws.data_ptr(),
                                (size_t)ws.numel(), current_stream(A)));
}

TORCH_LIBRARY(fp64_emu, ops) {
  ops.def("fp64_emu_maxp() -> int", &fp64_emu_maxp);
  ops.def("fp64_emu_mm(Tensor! out, Tensor A, Tensor B, Tensor primes_cpu, Tensor inv_cpu, Tensor mu_cpu, bool exact, int bits=53, bool use_corr=True) -> ()");
  ops.def("fp64_emu_bmm(Tensor! out, Tensor A, Tensor B, Tensor primes_cpu, Tensor inv_cpu, Tensor mu_cpu, bool exact, int bits=53, bool use_corr=True) -> ()");
  ops.def("fp64_emu_mm_nt(Tensor! out, Tensor A, Tensor Bt, Tensor primes_cpu, Tensor inv_cpu, Tensor mu_cpu, bool exact, int bits=53, bool use_corr=True) -> ()");
  ops.def("fp64_emu_bmm_nt(Tensor! out, Tensor A, Tensor Bt, Tensor primes_cpu, Tensor inv_cpu, Tensor mu_cpu, bool exact, int bits=53, bool use_corr=True) -> ()");
  ops.def("fp64_emu_mm_timed(Tensor! out, Tensor! times, Tensor A, Tensor B, Tensor primes_cpu, Tensor inv_cpu, Tensor mu_cpu, bool exact, int bits=53, bool use_corr=True) -> ()");
}

// PyTorch-ROCm keeps the CUDA dispatch key for HIP devices.
TORCH_LIBRARY_IMPL(fp64_emu, CUDA, ops) {
  ops.impl("fp64_emu_mm", &fp64_emu_mm);
  ops.impl("fp64_emu_bmm", &fp64_emu_bmm);
  ops.impl("fp64_emu_mm_nt", &fp64_emu_mm_nt);
  ops.impl("fp64_emu_bmm_nt", &fp64_emu_bmm_nt);
  ops.impl("fp64_emu_mm_timed", &fp64_emu_mm_timed);
}
