// Native harness over the C ABI (include/mhc_pre.h), the counterpart of the
// reference's on-device runner:
//   * its case matrix (cloud_runner/runner.cpp:320-327) and inputs, glibc
//     rand() after srand(42) in its draw order (:368-382), alpha {0.5, 0.3,
//     0.2} (:369), eps 1e-6 (:446);
//   * its host wall-clock latency mode: one warm-up launch and stream sync,
//     then 20 iterations of launch + stream synchronize timed on the host
//     clock, reported as min / median / avg (:458-490);
//   * the probe's relaunch of one executor, whose second launch must give
//     identical outputs (cloud_runner/probe_e1e2.cpp:312-326).
// Every output is checked against the C oracle (test infrastructure): hPost,
// hRes and hPre within 1e-5 + 1e-4 |want|; the device's hIn equal bit for bit
// to the oracle's weighted stream reduction on the device's own hPre; and the
// harness's own acceptance rule on hIn (|a - b| / max(1, |a|, |b|) <= 5e-2 for
// all but 0.1 % of elements, cloud_runner/runner.cpp:279-301).
//
// Usage: mhc_pre_runner [--iters N] [--shape B S n D gamma(0|1) bf16(0|1)]...
// With no --shape the reference matrix runs.  Exit status 0 iff every case
// passed; one line per case and check.

#include "mhc_pre.h"
#include "mhc_pre_oracle.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

struct Case {
    int64_t B, S;
    int n;
    int64_t D;
    bool gamma;
    bool bf16;
};

// cloud_runner/runner.cpp:320-327
const Case kReferenceCases[] = {
    {1, 2048, 4, 2560, true, false}, {1, 2048, 6, 1024, true, false},
    {1, 1024, 8, 1024, true, false}, {1, 2048, 4, 2560, false, false},
    {1, 2048, 6, 1024, true, true},  {1, 1024, 8, 1024, false, true},
};

bool hip_ok(hipError_t e, const char *what)
{
    if (e != hipSuccess) {
        std::printf("  FAIL %s: %s\n", what, hipGetErrorString(e));
        return false;
    }
    return true;
}

bool mhc_ok(int st, const char *what)
{
    if (st != MHC_STATUS_SUCCESS) {
        std::printf("  FAIL %s: %s (%d)\n", what, mhcPreStatusString(st), st);
        return false;
    }
    return true;
}

mhcTensor desc(void *p, int dtype, std::vector<int64_t> dims)
{
    mhcTensor t;
    std::memset(&t, 0, sizeof t);
    t.data = p;
    t.dtype = dtype;
    t.ndim = static_cast<int32_t>(dims.size());
    for (size_t i = 0; i < dims.size(); ++i) {
        t.dims[i] = dims[i];
    }
    return t;
}

float decode16(uint16_t b, bool bf16) { return bf16 ? oracle_bf16_to_f32(b) : oracle_f16_to_f32(b); }

// Device buffers of one case, freed on scope exit.
struct DevBuf {
    void *p = nullptr;
    bool alloc(size_t bytes) { return hipMalloc(&p, std::max<size_t>(bytes, 256)) == hipSuccess; }
    ~DevBuf()
    {
        if (p != nullptr) {
            (void)hipFree(p);
        }
    }
};

bool run_case(const Case &c, int iters, hipStream_t stream)
{
    const int64_t T = c.B * c.S, n = c.n, D = c.D, K = n * D, M = n * n + 2 * n;
    std::printf("case B=%lld S=%lld n=%lld D=%lld gamma=%d dtype=%s\n", (long long)c.B,
                (long long)c.S, (long long)n, (long long)D, (int)c.gamma, c.bf16 ? "bf16" : "fp16");
    std::fflush(stdout);

    // Inputs: the reference harness's generator, then the 16-bit cast of x.
    std::vector<float> xf(T * K), phi(K * M), bias(M), gamma(K);
    oracle_reference_harness_inputs(42, T, c.n, D, xf.data(), phi.data(), bias.data(), gamma.data());
    const float alpha[3] = {0.5f, 0.3f, 0.2f};
    std::vector<uint16_t> x(T * K);
    if (c.bf16) {
        oracle_f32_to_bf16_n(xf.data(), x.data(), T * K);
    } else {
        oracle_f32_to_f16_n(xf.data(), x.data(), T * K);
    }
    const float *g = c.gamma ? gamma.data() : nullptr;

    // Oracle.
    std::vector<uint16_t> inRef(T * D);
    std::vector<float> postRef(T * n), resRef(T * n * n), preRef(T * n);
    if (oracle_mhc_pre(x.data(), c.bf16, T, c.n, D, phi.data(), alpha, bias.data(), g, 1e-6f, 1e-6f,
                       nullptr, T, inRef.data(), postRef.data(), resRef.data(), preRef.data(), nullptr,
                       nullptr, 0) != 0) {
        std::printf("  FAIL oracle\n");
        return false;
    }

    DevBuf dx, dphi, dalpha, dbias, dgamma, din, dpost, dres, dpre, dws;
    if (!dx.alloc(T * K * 2) || !dphi.alloc(K * M * 4) || !dalpha.alloc(12) || !dbias.alloc(M * 4) ||
        !dgamma.alloc(K * 4) || !din.alloc(T * D * 2) || !dpost.alloc(T * n * 4) ||
        !dres.alloc(T * n * n * 4) || !dpre.alloc(T * n * 4)) {
        std::printf("  FAIL hipMalloc\n");
        return false;
    }
    bool ok = hip_ok(hipMemcpy(dx.p, x.data(), T * K * 2, hipMemcpyHostToDevice), "copy x") &&
              hip_ok(hipMemcpy(dphi.p, phi.data(), K * M * 4, hipMemcpyHostToDevice), "copy phi") &&
              hip_ok(hipMemcpy(dalpha.p, alpha, 12, hipMemcpyHostToDevice), "copy alpha") &&
              hip_ok(hipMemcpy(dbias.p, bias.data(), M * 4, hipMemcpyHostToDevice), "copy bias") &&
              hip_ok(hipMemcpy(dgamma.p, gamma.data(), K * 4, hipMemcpyHostToDevice), "copy gamma");
    if (!ok) {
        return false;
    }
    const int xdt = c.bf16 ? MHC_DTYPE_BF16 : MHC_DTYPE_FLOAT16;
    mhcTensor tx = desc(dx.p, xdt, {c.B, c.S, n, D});
    mhcTensor tphi = desc(dphi.p, MHC_DTYPE_FLOAT, {K, M});
    mhcTensor talpha = desc(dalpha.p, MHC_DTYPE_FLOAT, {3});
    mhcTensor tbias = desc(dbias.p, MHC_DTYPE_FLOAT, {M});
    mhcTensor tgamma = desc(dgamma.p, MHC_DTYPE_FLOAT, {n, D});
    mhcTensor tin = desc(din.p, xdt, {c.B, c.S, D});
    mhcTensor tpost = desc(dpost.p, MHC_DTYPE_FLOAT, {c.B, c.S, n});
    mhcTensor tres = desc(dres.p, MHC_DTYPE_FLOAT, {c.B, c.S, n, n});
    mhcTensor tpre = desc(dpre.p, MHC_DTYPE_FLOAT, {c.B, c.S, n});

    uint64_t wsBytes = 0;
    mhcPreExecutor *ex = nullptr;
    if (!mhc_ok(mhcPreGetWorkspaceSizeWithHPre(&tx, &tphi, &talpha, &tbias, c.gamma ? &tgamma : nullptr,
                                               1e-6f, 1e-6f, &tin, &tpost, &tres, &tpre, &wsBytes, &ex),
                "phase 1")) {
        return false;
    }
    const char *path = "?";
    (void)mhcPreExecutorPath(ex, &path);
    if (!dws.alloc(wsBytes)) {
        mhcPreExecutorDestroy(ex);
        std::printf("  FAIL workspace hipMalloc\n");
        return false;
    }

    // Warm-up, then the timed iterations (launch + stream synchronize each).
    ok = mhc_ok(mhcPre(dws.p, wsBytes, ex, stream), "warm-up launch") &&
         hip_ok(hipStreamSynchronize(stream), "warm-up sync");
    std::vector<double> us;
    for (int i = 0; ok && i < iters; ++i) {
        const auto t0 = std::chrono::steady_clock::now();
        ok = mhc_ok(mhcPre(dws.p, wsBytes, ex, stream), "launch") &&
             hip_ok(hipStreamSynchronize(stream), "sync");
        const auto t1 = std::chrono::steady_clock::now();
        us.push_back(std::chrono::duration<double, std::micro>(t1 - t0).count());
    }
    ok = ok && mhc_ok(mhcPreQueryDeviceStatus(dws.p, wsBytes, ex, stream), "device status");
    if (ok && !us.empty()) {
        std::sort(us.begin(), us.end());
        double avg = 0.0;
        for (double v : us) {
            avg += v;
        }
        avg /= static_cast<double>(us.size());
        std::printf("  path=%s workspace=%llu B  latency: min=%.2f us  median=%.2f us  avg=%.2f us  "
                    "(iters=%d)\n",
                    path, (unsigned long long)wsBytes, us.front(), us[us.size() / 2], avg, iters);
    }

    std::vector<uint16_t> in(T * D);
    std::vector<float> post(T * n), res(T * n * n), pre(T * n);
    ok = ok && hip_ok(hipMemcpy(in.data(), din.p, T * D * 2, hipMemcpyDeviceToHost), "copy hIn") &&
         hip_ok(hipMemcpy(post.data(), dpost.p, T * n * 4, hipMemcpyDeviceToHost), "copy hPost") &&
         hip_ok(hipMemcpy(res.data(), dres.p, T * n * n * 4, hipMemcpyDeviceToHost), "copy hRes") &&
         hip_ok(hipMemcpy(pre.data(), dpre.p, T * n * 4, hipMemcpyDeviceToHost), "copy hPre");
    if (!ok) {
        mhcPreExecutorDestroy(ex);
        return false;
    }

    // fp32 outputs.
    auto close = [](const std::vector<float> &got, const std::vector<float> &want, const char *name) {
        int64_t bad = 0;
        for (size_t i = 0; i < got.size(); ++i) {
            const double err = std::fabs((double)got[i] - (double)want[i]);
            if (!(err <= 1e-5 + 1e-4 * std::fabs((double)want[i]))) {
                ++bad;
            }
        }
        std::printf("  %-5s %s (%lld of %zu beyond 1e-5 + 1e-4 |want|)\n", name, bad ? "FAIL" : "ok",
                    (long long)bad, got.size());
        return bad == 0;
    };
    bool pass = close(post, postRef, "hPost");
    pass = close(res, resRef, "hRes") && pass;
    pass = close(pre, preRef, "hPre") && pass;

    // hIn: the device's stream reduction, bit for bit, on its own hPre.
    std::vector<uint16_t> stage(T * D);
    oracle_weighted_stream_sum(x.data(), c.bf16, T, c.n, D, pre.data(), stage.data());
    int64_t diff = 0;
    for (int64_t i = 0; i < T * D; ++i) {
        diff += in[i] != stage[i];
    }
    std::printf("  hIn   %s (stream reduction on the device hPre: %lld of %lld differ)\n",
                diff ? "FAIL" : "ok", (long long)diff, (long long)(T * D));
    pass = pass && diff == 0;
    // The harness's acceptance rule against the oracle's hIn.
    int64_t far = 0;
    for (int64_t i = 0; i < T * D; ++i) {
        const double a = decode16(in[i], c.bf16), b = decode16(inRef[i], c.bf16);
        if (std::fabs(a - b) / std::max(1.0, std::max(std::fabs(a), std::fabs(b))) > 5e-2) {
            ++far;
        }
    }
    std::printf("  hIn   %s (harness rule: %lld of %lld beyond 5e-2 relative)\n",
                far <= T * D / 1000 ? "ok" : "FAIL", (long long)far, (long long)(T * D));
    pass = pass && far <= T * D / 1000;

    // Relaunch of the same executor after clearing the outputs: identical.
    ok = hip_ok(hipMemset(din.p, 0, T * D * 2), "clear hIn") &&
         hip_ok(hipMemset(dpost.p, 0, T * n * 4), "clear hPost") &&
         hip_ok(hipMemset(dres.p, 0, T * n * n * 4), "clear hRes") &&
         mhc_ok(mhcPre(dws.p, wsBytes, ex, stream), "relaunch") &&
         hip_ok(hipStreamSynchronize(stream), "relaunch sync");
    std::vector<uint16_t> in2(T * D);
    std::vector<float> post2(T * n), res2(T * n * n);
    ok = ok && hip_ok(hipMemcpy(in2.data(), din.p, T * D * 2, hipMemcpyDeviceToHost), "copy hIn") &&
         hip_ok(hipMemcpy(post2.data(), dpost.p, T * n * 4, hipMemcpyDeviceToHost), "copy hPost") &&
         hip_ok(hipMemcpy(res2.data(), dres.p, T * n * n * 4, hipMemcpyDeviceToHost), "copy hRes");
    const bool same = ok && in2 == in && std::memcmp(post2.data(), post.data(), post.size() * 4) == 0 &&
                      std::memcmp(res2.data(), res.data(), res.size() * 4) == 0;
    std::printf("  relaunch %s (second launch of the executor bit-identical)\n", same ? "ok" : "FAIL");
    pass = pass && same;
    mhcPreExecutorDestroy(ex);
    std::printf("  %s\n", pass ? "PASS" : "FAIL");
    std::fflush(stdout);
    return pass;
}

}  // namespace

int main(int argc, char **argv)
{
    int iters = 20;
    std::vector<Case> cases;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "--iters" && i + 1 < argc) {
            iters = std::atoi(argv[++i]);
        } else if (a == "--shape" && i + 6 < argc) {
            Case c;
            c.B = std::atoll(argv[i + 1]);
            c.S = std::atoll(argv[i + 2]);
            c.n = std::atoi(argv[i + 3]);
            c.D = std::atoll(argv[i + 4]);
            c.gamma = std::atoi(argv[i + 5]) != 0;
            c.bf16 = std::atoi(argv[i + 6]) != 0;
            cases.push_back(c);
            i += 6;
        } else {
            std::fprintf(stderr, "usage: %s [--iters N] [--shape B S n D gamma bf16]...\n", argv[0]);
            return 2;
        }
    }
    if (cases.empty()) {
        cases.assign(std::begin(kReferenceCases), std::end(kReferenceCases));
    }
    hipStream_t stream = nullptr;
    if (!hip_ok(hipSetDevice(0), "hipSetDevice") || !hip_ok(hipStreamCreate(&stream), "hipStreamCreate")) {
        return 1;
    }
    int failed = 0;
    for (const Case &c : cases) {
        failed += run_case(c, iters, stream) ? 0 : 1;
    }
    (void)hipStreamDestroy(stream);
    std::printf("%s: %zu cases, %d failed\n", failed ? "FAILED" : "All cases passed", cases.size(), failed);
    return failed ? 1 : 0;
}
