// PyTorch operators over the C ABI of libmhcpre.so:
//   torch.ops.mhcpre.mhc_pre(x, phi, alpha, bias, gamma=None, norm_eps=1e-6, hc_eps=1e-6)
//       -> (hIn, hPost, hRes)
//   torch.ops.mhcpre.mhc_pre_with_h_pre(...) -> (hIn, hPost, hRes, hPre)
//   torch.ops.mhcpre.status_word(device) -> the device's sticky status word (int32[1])
//
// Each call is the reference caller's sequence (cloud_runner/runner.cpp:443-476) in native
// code: phase 1 (mhcPreGetWorkspaceSize[WithHPre]; the library caches the plan per shape,
// so on a repeated shape it validates and binds the tensors), the outputs and the workspace
// from PyTorch's caching allocator, phase 2 (mhcPre) on the current stream, the executor
// freed.  Arguments, defaults and validation are the reference operator's
// (code/op_host/mhc_pre.cpp:57-79,126-130,217-257,297-298); the library's status codes
// come back as errors naming the status.
//
// Only device tensors have a kernel (dispatch key CUDA, which is ROCm's device key in
// PyTorch: its device tensors report the CUDA device type, hence the "masquerading" guard
// and stream helpers); the shape-only implementation for tracing is registered from Python.
//
// Expired waits: every executor made here marks the current device's sticky status word
// (mhcPreExecutorSetStatusWord) when a bounded wait between workgroups expires, so a caller
// learns of NaN rows without a synchronization of the operator's own.
// MHCPRE_CHECK_STATUS=1 instead waits for the stream after every call and raises.
#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "mhc_pre.h"

namespace {

int32_t dtype_code(at::ScalarType t)
{
    switch (t) {
    case at::kFloat:
        return MHC_DTYPE_FLOAT;
    case at::kHalf:
        return MHC_DTYPE_FLOAT16;
    case at::kBFloat16:
        return MHC_DTYPE_BF16;
    default:
        return -1;  // the library rejects it with MHC_STATUS_INVALID_DTYPE
    }
}

mhcTensor describe(void *data, int32_t dtype, at::IntArrayRef dims)
{
    mhcTensor d;
    std::memset(&d, 0, sizeof(d));
    d.data = data;
    d.dtype = dtype;
    TORCH_CHECK(dims.size() <= MHC_MAX_DIMS, "mhcpre: tensor of rank ", dims.size());
    d.ndim = static_cast<int32_t>(dims.size());
    for (size_t i = 0; i < dims.size(); ++i) {
        d.dims[i] = dims[i];
    }
    return d;
}

mhcTensor describe(const at::Tensor &t)
{
    return describe(t.data_ptr(), dtype_code(t.scalar_type()), t.sizes());
}

[[noreturn]] void fail(const char *where, int status)
{
    TORCH_CHECK(false, where, " failed: ", mhcPreStatusString(status), " (", status, ")");
}

// One int32 word per device, zero until a launch's bounded wait expires.  Allocated on
// first use and kept for the process (never freed: a static tensor destroyed after the
// HIP runtime shuts down would free into a dead allocator).
at::Tensor &status_word_of(c10::DeviceIndex index)
{
    static std::mutex mu;
    static std::vector<at::Tensor *> words;
    std::lock_guard<std::mutex> lock(mu);
    if (static_cast<size_t>(index) >= words.size()) {
        words.resize(static_cast<size_t>(index) + 1, nullptr);
    }
    if (words[index] == nullptr) {
        words[index] = new at::Tensor(
            at::zeros({1}, at::TensorOptions().dtype(at::kInt).device(at::kCUDA, index)));
    }
    return *words[index];
}

at::Tensor status_word(int64_t device)
{
    TORCH_CHECK(device >= 0, "mhcpre.status_word: device index ", device);
    return status_word_of(static_cast<c10::DeviceIndex>(device));
}

bool check_status()
{
    const char *v = std::getenv("MHCPRE_CHECK_STATUS");
    return v != nullptr && v[0] != '\0' && std::strcmp(v, "0") != 0;
}

// Frees the executor on every way out of a call.
struct ExecutorOwner {
    mhcPreExecutor *exe = nullptr;
    ~ExecutorOwner()
    {
        if (exe != nullptr) {
            mhcPreExecutorDestroy(exe);
        }
    }
};

std::vector<at::Tensor> launch(const at::Tensor &x_, const at::Tensor &phi_, const at::Tensor &alpha_,
                               const at::Tensor &bias_, const std::optional<at::Tensor> &gamma_,
                               double normEps, double hcEps, bool withHPre)
{
    TORCH_CHECK(x_.is_cuda(), "mhcpre: x must be a device tensor");
    TORCH_CHECK(x_.dim() >= 2, "mhcpre: x must be [B, S, n, D] or [T, n, D]");
    // The library launches on the current device, which must hold x.
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(x_.device());
    const at::Tensor x = x_.contiguous(), phi = phi_.contiguous(), alpha = alpha_.contiguous(),
                     bias = bias_.contiguous();
    at::Tensor gamma;
    if (gamma_.has_value() && gamma_->defined()) {
        gamma = gamma_->contiguous();
    }
    const int64_t n = x.size(-2), D = x.size(-1);
    std::vector<int64_t> lead(x.sizes().begin(), x.sizes().end() - 2);
    auto shape = [&](std::initializer_list<int64_t> tail) {
        std::vector<int64_t> s = lead;
        s.insert(s.end(), tail);
        return s;
    };
    const auto f32 = x.options().dtype(at::kFloat);
    at::Tensor hIn = at::empty(shape({D}), x.options());
    at::Tensor hPost = at::empty(shape({n}), f32);
    at::Tensor hRes = at::empty(shape({n, n}), f32);
    at::Tensor hPre;
    if (withHPre) {
        hPre = at::empty(shape({n}), f32);
    }

    const mhcTensor dx = describe(x), dphi = describe(phi), dalpha = describe(alpha),
                    dbias = describe(bias), dhin = describe(hIn), dpost = describe(hPost),
                    dres = describe(hRes);
    mhcTensor dgamma, dpre;
    if (gamma.defined()) {
        dgamma = describe(gamma);
    }
    if (withHPre) {
        dpre = describe(hPre);
    }
    uint64_t wsBytes = 0;
    ExecutorOwner owner;
    const int st = withHPre
        ? mhcPreGetWorkspaceSizeWithHPre(&dx, &dphi, &dalpha, &dbias, gamma.defined() ? &dgamma : nullptr,
                                         static_cast<float>(normEps), static_cast<float>(hcEps), &dhin,
                                         &dpost, &dres, &dpre, &wsBytes, &owner.exe)
        : mhcPreGetWorkspaceSize(&dx, &dphi, &dalpha, &dbias, gamma.defined() ? &dgamma : nullptr,
                                 static_cast<float>(normEps), static_cast<float>(hcEps), &dhin, &dpost,
                                 &dres, &wsBytes, &owner.exe);
    if (st != MHC_STATUS_SUCCESS) {
        fail(withHPre ? "mhcPreGetWorkspaceSizeWithHPre" : "mhcPreGetWorkspaceSize", st);
    }
    // The workspace goes back to the caching allocator when this call returns, in the
    // order of the current stream, after the launch that uses it.
    const at::Tensor ws = at::empty({static_cast<int64_t>(std::max<uint64_t>(wsBytes, 256))},
                                    x.options().dtype(at::kByte));
    hipStream_t stream = c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(x.device().index()).stream();
    int rc = mhcPreExecutorSetStatusWord(
        owner.exe, static_cast<uint32_t *>(status_word_of(x.device().index()).data_ptr()));
    if (rc != MHC_STATUS_SUCCESS) {
        fail("mhcPreExecutorSetStatusWord", rc);
    }
    rc = mhcPre(ws.data_ptr(), wsBytes, owner.exe, stream);
    if (rc != MHC_STATUS_SUCCESS) {
        fail("mhcPre", rc);
    }
    if (check_status()) {
        rc = mhcPreQueryDeviceStatus(ws.data_ptr(), wsBytes, owner.exe, stream);
        if (rc != MHC_STATUS_SUCCESS) {
            fail("mhcPreQueryDeviceStatus", rc);
        }
    }
    std::vector<at::Tensor> out{hIn, hPost, hRes};
    if (withHPre) {
        out.push_back(hPre);
    }
    return out;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> mhc_pre(const at::Tensor &x, const at::Tensor &phi,
                                                       const at::Tensor &alpha, const at::Tensor &bias,
                                                       const std::optional<at::Tensor> &gamma,
                                                       double normEps, double hcEps)
{
    auto o = launch(x, phi, alpha, bias, gamma, normEps, hcEps, false);
    return {o[0], o[1], o[2]};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> mhc_pre_with_h_pre(
    const at::Tensor &x, const at::Tensor &phi, const at::Tensor &alpha, const at::Tensor &bias,
    const std::optional<at::Tensor> &gamma, double normEps, double hcEps)
{
    auto o = launch(x, phi, alpha, bias, gamma, normEps, hcEps, true);
    return {o[0], o[1], o[2], o[3]};
}

}  // namespace

TORCH_LIBRARY(mhcpre, m)
{
    m.def("mhc_pre(Tensor x, Tensor phi, Tensor alpha, Tensor bias, Tensor? gamma=None, "
          "float norm_eps=1e-06, float hc_eps=1e-06) -> (Tensor, Tensor, Tensor)");
    m.def("mhc_pre_with_h_pre(Tensor x, Tensor phi, Tensor alpha, Tensor bias, "
          "Tensor? gamma=None, float norm_eps=1e-06, float hc_eps=1e-06) "
          "-> (Tensor, Tensor, Tensor, Tensor)");
    m.def("status_word(int device) -> Tensor", &status_word);
}

TORCH_LIBRARY_IMPL(mhcpre, CUDA, m)
{
    m.impl("mhc_pre", &mhc_pre);
    m.impl("mhc_pre_with_h_pre", &mhc_pre_with_h_pre);
}
