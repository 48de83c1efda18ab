// compat_driver.cpp -- runs the reference-signature C++ layer (include/helios/exl3_compat.hpp) on
// the GPU the way the reference engine's call sites do (src/engine/runner.cpp:711-959, 1411), dumps
// every input and output for the Python parity test (tests/test_gpu_compat.py), and times the host
// side of a call: the microseconds the calling thread spends per call when nothing waits for the GPU.
//
// Usage: compat_driver <outdir>
// Writes <outdir>/<name>.bin for each array and prints one JSON line of host timings.
#include "helios/exl3_compat.hpp"

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

namespace {

using helios::Stream;

struct Rng {  // xorshift64*: deterministic data without the C library's generator
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed * 2654435761u + 0x9E3779B97F4A7C15ull) {}
    uint64_t next()
    {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        return s * 2685821657736338717ull;
    }
    double uniform() { return (double)(next() >> 11) * (1.0 / 9007199254740992.0); }
    double normal()
    {
        const double u = uniform() + 1e-300, v = uniform();
        return std::sqrt(-2.0 * std::log(u)) * std::cos(6.283185307179586 * v);
    }
};

uint16_t f2h(float f)  // fp32 -> fp16, round to nearest even (finite inputs)
{
    _Float16 h = (_Float16)f;
    uint16_t u;
    std::memcpy(&u, &h, 2);
    return u;
}

void die(const char* what)
{
    std::fprintf(stderr, "compat_driver: %s\n", what);
    std::exit(1);
}

void hip_ok(hipError_t e, const char* what)
{
    if (e != hipSuccess) {
        std::fprintf(stderr, "compat_driver: %s: %s\n", what, hipGetErrorString(e));
        std::exit(1);
    }
}

std::string g_out;

void dump(const char* name, const void* host, size_t bytes)
{
    const std::string path = g_out + "/" + name + ".bin";
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(host, 1, bytes, f) != bytes) die("write failed");
    std::fclose(f);
}

template <class T>
T* upload(const std::vector<T>& v)
{
    T* d = nullptr;
    hip_ok(hipMalloc(&d, v.size() * sizeof(T) + 256), "hipMalloc");
    hip_ok(hipMemcpy(d, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy");
    return d;
}

template <class T>
std::vector<T> download(const T* d, size_t n)
{
    std::vector<T> v(n);
    hip_ok(hipMemcpy(v.data(), d, n * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy");
    return v;
}

// One EXL3 linear with seeded weights: trellis words uniform, suh = +-1, svh = +-U(0.5, 1.5).
struct Lin {
    int K, N, bits;
    std::vector<uint16_t> tr, suh, svh;
    uint16_t* dtr = nullptr;
    uint16_t* dsuh = nullptr;
    uint16_t* dsvh = nullptr;
    Lin(int K_, int N_, int bits_, Rng& r) : K(K_), N(N_), bits(bits_)
    {
        tr.resize((size_t)K * N * bits / 16);
        for (auto& w : tr) w = (uint16_t)r.next();
        suh.resize(K);
        for (auto& s : suh) s = f2h(r.uniform() < 0.5 ? -1.0f : 1.0f);
        svh.resize(N);
        for (auto& s : svh) s = f2h((float)((r.uniform() < 0.5 ? -1.0 : 1.0) * (0.5 + r.uniform())));
        dtr = upload(tr);
        dsuh = upload(suh);
        dsvh = upload(svh);
    }
    helios::exl3::GroupWords gw() const { return {dtr, dsuh, dsvh, (int)0x83DCD12Du}; }
    void dump_as(const std::string& p) const
    {
        dump((p + "_trellis").c_str(), tr.data(), tr.size() * 2);
        dump((p + "_suh").c_str(), suh.data(), suh.size() * 2);
        dump((p + "_svh").c_str(), svh.data(), svh.size() * 2);
    }
};

// Routed experts of one layer and their device pointer tables (the engine's ExpertTables).
struct Experts {
    std::vector<Lin> lin;  // expert e: lin[3e + p]
    helios::exl3::ExpertTables t{};
    Experts(int E, int hidden, int inter, int bits, Rng& r)
    {
        lin.reserve((size_t)3 * E);
        for (int e = 0; e < E; ++e) {
            lin.emplace_back(hidden, inter, bits, r);
            lin.emplace_back(hidden, inter, bits, r);
            lin.emplace_back(inter, hidden, bits, r);
        }
        std::vector<const void*> p[9];
        for (int e = 0; e < E; ++e)
            for (int q = 0; q < 3; ++q) {
                const Lin& l = lin[3 * e + q];
                p[3 * q + 0].push_back(l.dtr);
                p[3 * q + 1].push_back(l.dsuh);
                p[3 * q + 2].push_back(l.dsvh);
            }
        const void** d[9];
        for (int i = 0; i < 9; ++i) d[i] = reinterpret_cast<const void**>(upload(p[i]));
        t.gate_trellis = reinterpret_cast<const uint16_t**>(d[0]);
        t.gate_suh = d[1];
        t.gate_svh = d[2];
        t.up_trellis = reinterpret_cast<const uint16_t**>(d[3]);
        t.up_suh = d[4];
        t.up_svh = d[5];
        t.down_trellis = reinterpret_cast<const uint16_t**>(d[6]);
        t.down_suh = d[7];
        t.down_svh = d[8];
    }
};

std::vector<uint16_t> normal_f16(size_t n, Rng& r)
{
    std::vector<uint16_t> v(n);
    for (auto& x : v) x = f2h((float)r.normal());
    return v;
}

double host_us_per_call(int n, const std::function<void()>& fn)
{
    fn();
    hip_ok(hipDeviceSynchronize(), "sync");
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < n; ++i) fn();
    const auto t1 = std::chrono::steady_clock::now();
    hip_ok(hipDeviceSynchronize(), "sync");
    return std::chrono::duration<double, std::micro>(t1 - t0).count() / n;
}

}  // namespace

int main(int argc, char** argv)
{
    if (argc < 2) die("usage: compat_driver <outdir>");
    g_out = argv[1];
    Rng r(20240601);
    Stream s = nullptr;
    hip_ok(hipStreamCreate(&s), "hipStreamCreate");

    // ---- quantized linear: helios::exl3::gemm, GEMV (M = 1) and MFMA (M = 32) paths
    {
        const int K = 1024, N = 512, bits = 3;
        Lin l(K, N, bits, r);
        l.dump_as("lin");
        for (int M : {1, 32}) {
            const auto x = normal_f16((size_t)M * K, r);
            uint16_t* dx = upload(x);
            float* dy = nullptr;
            _Float16* a_had = nullptr;
            hip_ok(hipMalloc(&dy, (size_t)M * N * 4), "hipMalloc");
            hip_ok(hipMalloc(&a_had, (size_t)M * K * 2), "hipMalloc");
            const int path = helios::exl3::gemm(dy, dx, l.gw(), M, N, K, bits, true, s, a_had);
            hip_ok(hipStreamSynchronize(s), "sync");
            const auto y = download(dy, (size_t)M * N);
            const std::string tag = "gemm_m" + std::to_string(M);
            dump((tag + "_x").c_str(), x.data(), x.size() * 2);
            dump((tag + "_y").c_str(), y.data(), y.size() * 4);
            dump((tag + "_path").c_str(), &path, sizeof(path));
        }
    }

    // ---- helios::exl3::had_r_128 in the reference's form: DType, scale multiplied by 1/sqrt(128),
    //      pre and post scales exclusive
    {
        const int rows = 8, cols = 256;
        const auto x = normal_f16((size_t)rows * cols, r);
        auto sc = normal_f16(cols, r);
        uint16_t* dx = upload(x);
        uint16_t* dsc = upload(sc);
        uint16_t* dout = nullptr;
        hip_ok(hipMalloc(&dout, (size_t)rows * cols * 2), "hipMalloc");
        helios::exl3::had_r_128(dx, dout, nullptr, dsc, rows, cols, helios::exl3::DType::Half, 1.0f, s);
        hip_ok(hipStreamSynchronize(s), "sync");
        const auto o = download(dout, (size_t)rows * cols);
        dump("had_x", x.data(), x.size() * 2);
        dump("had_post", sc.data(), sc.size() * 2);
        dump("had_y", o.data(), o.size() * 2);
        int refused = 0;
        try {
            helios::exl3::had_r_128(dx, dout, dsc, dsc, rows, cols, helios::exl3::DType::Half, 1.0f, s);
        } catch (const helios::exl3::Error&) {
            refused = 1;
        }
        dump("had_refused", &refused, sizeof(refused));
    }

    // ---- the same linear on two streams at once: each (device, stream) has its own workspace
    {
        const int K = 4096, N = 2048, bits = 2;
        Lin l(K, N, bits, r);
        Stream s2 = nullptr;
        hip_ok(hipStreamCreate(&s2), "hipStreamCreate");
        uint16_t* dx = upload(normal_f16(K, r));
        float *y1 = nullptr, *y2 = nullptr;
        hip_ok(hipMalloc(&y1, (size_t)N * 4), "hipMalloc");
        hip_ok(hipMalloc(&y2, (size_t)N * 4), "hipMalloc");
        helios::exl3::gemm(y1, dx, l.gw(), 1, N, K, bits, true, s);
        hip_ok(hipDeviceSynchronize(), "sync");
        const auto ref = download(y1, N);
        int same = 1;
        for (int it = 0; it < 20; ++it) {
            helios::exl3::gemm(y1, dx, l.gw(), 1, N, K, bits, true, s);
            helios::exl3::gemm(y2, dx, l.gw(), 1, N, K, bits, true, s2);
            hip_ok(hipDeviceSynchronize(), "sync");
            const auto a = download(y1, N), b = download(y2, N);
            for (int n = 0; n < N; ++n) same &= (a[n] == ref[n]) & (b[n] == ref[n]);
        }
        dump("two_streams_same", &same, sizeof(same));
    }

    // ---- the engine's routed-MoE sequence (runner.cpp:759-764, 918-922): router, permutation,
    //      moe_grouped with sorted contributions, ordered reduction; then the dense fallback's row glue
    const int E = 16, hidden = 512, inter = 256, topk = 4, bits = 2;
    Experts ex(E, hidden, inter, bits, r);
    for (int e = 0; e < E; ++e)
        for (int q = 0; q < 3; ++q) ex.lin[3 * e + q].dump_as("ex" + std::to_string(e) + "_" + std::to_string(q));
    for (int T : {3, 20}) {
        const auto x = normal_f16((size_t)T * hidden, r);
        const auto sc = normal_f16((size_t)T * E, r);
        uint16_t* dx = upload(x);
        uint16_t* dsc = upload(sc);
        int64_t *idx, *cnt, *ts, *r2s, *pws;
        uint16_t *w, *wsr;
        float *contrib, *y;
        hip_ok(hipMalloc(&idx, (size_t)T * topk * 8), "m");
        hip_ok(hipMalloc(&w, (size_t)T * topk * 2), "m");
        hip_ok(hipMalloc(&cnt, (E + 1) * 8), "m");
        hip_ok(hipMalloc(&ts, (size_t)T * topk * 8), "m");
        hip_ok(hipMalloc(&wsr, (size_t)T * topk * 2), "m");
        hip_ok(hipMalloc(&r2s, (size_t)T * topk * 8), "m");
        hip_ok(hipMalloc(&pws, (size_t)3 * (E + 2) * 8), "m");
        hip_ok(hipMalloc(&contrib, (size_t)T * topk * hidden * 4), "m");
        hip_ok(hipMalloc(&y, (size_t)T * hidden * 4), "m");
        helios::aux::routing_ds3_nogroup(dsc, nullptr, idx, w, T, E, topk, 2.5f, true, 0, s);
        helios::glue::moe_permute(idx, w, T, topk, E, cnt, ts, wsr, pws, s, r2s);
        helios::exl3::moe_grouped(dx, y, cnt, ts, wsr, nullptr, nullptr, nullptr, nullptr, ex.t, T, hidden, inter, E,
                                  topk, T, 1, bits, bits, bits, false, true, 10.0f, 0, -1, s, contrib);
        helios::glue::moe_reduce_sorted(y, contrib, r2s, T, topk, hidden, s);
        hip_ok(hipStreamSynchronize(s), "sync");
        const std::string tag = "moe_t" + std::to_string(T);
        dump((tag + "_x").c_str(), x.data(), x.size() * 2);
        dump((tag + "_scores").c_str(), sc.data(), sc.size() * 2);
        const auto hidx = download(idx, (size_t)T * topk);
        const auto hw = download(w, (size_t)T * topk);
        const auto hy = download(y, (size_t)T * hidden);
        dump((tag + "_idx").c_str(), hidx.data(), hidx.size() * 8);
        dump((tag + "_w").c_str(), hw.data(), hw.size() * 2);
        dump((tag + "_y").c_str(), hy.data(), hy.size() * 4);

        // dense-MoE fallback glue (runner.cpp:902-907) on expert 0's rows
        const auto hcnt = download(cnt, E + 1);
        const int n0 = (int)hcnt[0];
        uint16_t* gx = nullptr;
        float* acc = nullptr;
        hip_ok(hipMalloc(&gx, (size_t)(n0 + 1) * hidden * 2), "m");
        hip_ok(hipMalloc(&acc, (size_t)T * hidden * 4), "m");
        hip_ok(hipMemset(acc, 0, (size_t)T * hidden * 4), "memset");
        helios::glue::gather_rows(dx, ts, gx, n0, hidden, s);
        helios::glue::scatter_add_rows(acc, contrib, ts, wsr, n0, hidden, s);
        hip_ok(hipStreamSynchronize(s), "sync");
        const auto hg = download(gx, (size_t)n0 * hidden);
        const auto ha = download(acc, (size_t)T * hidden);
        const auto hts = download(ts, (size_t)T * topk);
        const auto hwsr = download(wsr, (size_t)T * topk);
        const auto hc = download(contrib, (size_t)T * topk * hidden);
        dump((tag + "_gather").c_str(), hg.data(), hg.size() * 2);
        dump((tag + "_scatter").c_str(), ha.data(), ha.size() * 4);
        dump((tag + "_ts").c_str(), hts.data(), hts.size() * 8);
        dump((tag + "_wsorted").c_str(), hwsr.data(), hwsr.size() * 2);
        dump((tag + "_contrib").c_str(), hc.data(), hc.size() * 4);
        dump((tag + "_n0").c_str(), &n0, sizeof(n0));
    }

    // ---- the whole layer through helios::exl3::moe_layer, with a shared expert, 1 token
    {
        Lin sg(hidden, inter, bits, r), su(hidden, inter, bits, r), sd(inter, hidden, bits, r);
        sg.dump_as("sh0");
        su.dump_as("sh1");
        sd.dump_as("sh2");
        const helios::exl3::GroupWords shw[3] = {sg.gw(), su.gw(), sd.gw()};
        const int shb[3] = {bits, bits, bits};
        const auto x = normal_f16(hidden, r);
        const auto sc = normal_f16(E, r);
        uint16_t* dx = upload(x);
        uint16_t* dsc = upload(sc);
        uint16_t* dy = nullptr;
        float* dyr = nullptr;
        hip_ok(hipMalloc(&dy, hidden * 2), "m");
        hip_ok(hipMalloc(&dyr, hidden * 4), "m");
        helios::exl3::moe_layer(dy, dyr, dx, dsc, nullptr, ex.t, shw, shb, 1, hidden, inter, E, topk, bits, bits, bits,
                                2.5f, 10.0f, false, true, s);
        hip_ok(hipStreamSynchronize(s), "sync");
        dump("layer_x", x.data(), x.size() * 2);
        dump("layer_scores", sc.data(), sc.size() * 2);
        const auto hy = download(dy, hidden);
        const auto hyr = download(dyr, hidden);
        dump("layer_y", hy.data(), hy.size() * 2);
        dump("layer_yr", hyr.data(), hyr.size() * 4);
    }

    // ---- host cost per call at the decode shapes (config 3 layer, config 1 linear): the calling
    //      thread's time per call in a loop of asynchronous calls (the synchronous status check,
    //      a debug option the parity tests turn on, is off here)
    unsetenv("HX_MOE_SYNC_CHECK");
    {
        const int E3 = 288, H3 = 4096, I3 = 2048;
        Rng r3(7);
        Experts ex3(E3, H3, I3, 2, r3);
        Lin g3(H3, I3, 2, r3), u3(H3, I3, 2, r3), d3(I3, H3, 2, r3), l1(4096, 2048, 2, r3);
        const helios::exl3::GroupWords shw[3] = {g3.gw(), u3.gw(), d3.gw()};
        const int shb[3] = {2, 2, 2};
        uint16_t* dx = upload(normal_f16(H3, r3));
        uint16_t* dsc = upload(normal_f16(E3, r3));
        uint16_t* dy = nullptr;
        float* dy1 = nullptr;
        hip_ok(hipMalloc(&dy, H3 * 2), "m");
        hip_ok(hipMalloc(&dy1, 2048 * 4), "m");
        const double layer_us = host_us_per_call(256, [&]() {
            helios::exl3::moe_layer(dy, nullptr, dx, dsc, nullptr, ex3.t, shw, shb, 1, H3, I3, E3, 8, 2, 2, 2, 2.5f,
                                    10.0f, false, true, s);
        });
        const double gemm_us = host_us_per_call(256, [&]() {
            helios::exl3::gemm(dy1, dx, l1.gw(), 1, 2048, 4096, 2, true, s);
        });
        std::printf("{\"host_us_per_call\": {\"moe_layer_config3\": %.2f, \"gemm_config1\": %.2f}, \"calls\": 256}\n",
                    layer_us, gemm_us);
    }
    return 0;
}
