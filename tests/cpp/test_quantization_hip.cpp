// DeviceType::HIP tests through the VeloMind API: graphs built with
// g.build(DeviceType::HIP) against the oracle (the reference's CPU
// algorithm).  Mirrors the reference's tests/test_quantization.cpp
// (:140-207 numerics, :310-374 cross-backend, :376-411 storage sizes,
// :448-469 half-precision sources) and the concurrent build/execute stress
// of tests/test_coverage_matrix.cpp:690-738.
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <span>
#include <stdexcept>
#include <thread>

#include "internal/registry/kernel.h"
#include "internal/registry/storage.h"
#include "test_helpers.h"

using namespace velomind;
using namespace vmtest;

namespace {

struct QmmCase {
    std::size_t m, k, n;
    QuantType qt;
    int block;
};

// Runs one QMM graph on `device`; weights given as packed codes + scales.
std::vector<float> run_graph(DeviceType device, const QmmCase& c, const std::vector<float>& a,
                             const std::vector<std::int8_t>& q, const std::vector<float>& s) {
    Graph g;
    const dim_t qrows = c.qt == QuantType::Int4 ? (dim_t)((c.k + 1) / 2) : (dim_t)c.k;
    auto ta = g.input({(dim_t)c.m, (dim_t)c.k}, DataType::Float32);
    auto tw = g.input({qrows, (dim_t)c.n}, DataType::Int8);
    auto ts = c.block > 0 ? g.input({(dim_t)(s.size() / c.n), (dim_t)c.n}, DataType::Float32)
                          : g.input({(dim_t)c.n}, DataType::Float32);
    auto tc = g.op(OpDescriptor{Op::QuantizedMatMul, QuantizedMatMulAttrs{.quant_type = c.qt, .block_size = c.block}},
                   ta, tw, ts);
    auto exec = g.build(device);
    ta.copy_from_host(as_bytes(a));
    tw.copy_from_host(as_bytes(q));
    ts.copy_from_host(as_bytes(s));
    exec->execute();
    std::vector<float> out(c.m * c.n);
    tc.copy_to_host(as_writeable_bytes(out));
    return out;
}

}  // namespace

TEST_CASE("QuantizedMatMul HIP vs CPU oracle on the reference test matrix", "[gpu][quantization]") {
    REQUIRE_HIP();
    for (std::size_t m : {1, 4, 16}) {
        for (auto [k, n] : std::vector<std::pair<std::size_t, std::size_t>>{{64, 64}, {128, 256}, {576, 576}, {576, 1536}}) {
            const auto w = generate_random_weights(k, n);
            const auto a = generate_activations(m, k);
            std::vector<std::int8_t> q(k * n);
            std::vector<float> s(n);
            quantize_weights_int8_per_channel(w.data(), q.data(), s.data(), k, n);  // GPU packer
            std::vector<std::int8_t> q_ref(k * n);
            std::vector<float> s_ref(n);
            vmo_quantize_int8_per_channel(w.data(), q_ref.data(), s_ref.data(), k, n);
            REQUIRE(q == q_ref);
            REQUIRE(s == s_ref);
            const QmmCase c{m, k, n, QuantType::Int8, 0};
            const auto hip = run_graph(DeviceType::HIP, c, a, q, s);
            const auto cpu = run_graph(DeviceType::CPU, c, a, q, s);
            require_all_finite(hip);
            // GEMV path (m <= 4): fp32 end to end, the reference's 1e-4 bound;
            // MFMA path: fp16 activations, 1e-3 * max|ref|.
            const float bound = m <= 4 ? 1e-4f : 1e-3f * max_abs(cpu);
            REQUIRE(max_abs_diff(hip, cpu) < bound);
        }
    }
}

TEST_CASE("INT4 graph: quantize_storage_int4 on HIP, block 32, TinyLlama q shape", "[gpu][quantization]") {
    REQUIRE_HIP();
    const std::size_t k = 2048, n = 2048;
    const auto w = normal(k * n, 7, 0.02f);
    TensorStorage src;
    src.shape = {(dim_t)k, (dim_t)n};
    src.dtype = DataType::Float32;
    src.data = const_cast<float*>(w.data());
    src.size_bytes = src.capacity_bytes = w.size() * 4;
    auto [q, s] = quantize_storage_int4(src, 32, DeviceType::HIP);
    REQUIRE(q->device == DeviceType::HIP && q->shape == shape_t({1024, 2048}) && q->dtype == DataType::Int8);
    REQUIRE(s->shape == shape_t({64, 2048}) && s->dtype == DataType::Float32);
    REQUIRE(q->size_bytes == ((k + 1) / 2) * n);  // tests/test_quantization.cpp:376-390

    std::vector<std::uint8_t> q_host(q->size_bytes), q_ref(q->size_bytes);
    std::vector<float> s_host(s->size_bytes / 4), s_ref(s->size_bytes / 4);
    REQUIRE(vm_hip_memcpy_d2h(q_host.data(), q->data, q->size_bytes, nullptr) == 0);
    REQUIRE(vm_hip_memcpy_d2h(s_host.data(), s->data, s->size_bytes, nullptr) == 0);
    vmo_quantize_int4_block(w.data(), q_ref.data(), s_ref.data(), k, n, 32);
    REQUIRE(q_host == q_ref);
    REQUIRE(s_host == s_ref);

    Graph g;
    auto x = g.input({1, (dim_t)k}, DataType::Float32);
    auto tw = g.input(q);
    auto ts = g.input(s);
    auto y = g.op(OpDescriptor{Op::QuantizedMatMul, QuantizedMatMulAttrs{.quant_type = QuantType::Int4, .block_size = 32}},
                  x, tw, ts);
    auto exec = g.build(DeviceType::HIP);
    const auto xv = normal(k, 8);
    x.copy_from_host(as_bytes(xv));
    exec->execute();
    std::vector<float> out(n), ref(n);
    y.copy_to_host(as_writeable_bytes(out));
    vmo_qmm_2d_f32(xv.data(), reinterpret_cast<const std::int8_t*>(q_ref.data()), s_ref.data(), ref.data(), 1, k, n, 2, 32);
    REQUIRE(max_abs_diff(out, ref) <= 1e-5f * max_abs(ref));
}

TEST_CASE("batched activation [2,16,64] folds into the row count", "[gpu][quantization]") {
    REQUIRE_HIP();
    const std::size_t k = 64, n = 128;
    const auto w = generate_random_weights(k, n);
    std::vector<std::int8_t> q(k * n);
    std::vector<float> s(n);
    vmo_quantize_int8_per_channel(w.data(), q.data(), s.data(), k, n);
    const auto a = generate_activations(32, k);
    Graph g;
    auto ta = g.input({2, 16, (dim_t)k}, DataType::Float32);
    auto tw = g.input({(dim_t)k, (dim_t)n}, DataType::Int8);
    auto ts = g.input({(dim_t)n}, DataType::Float32);
    auto tc = g.op(Op::QuantizedMatMul, ta, tw, ts);
    REQUIRE(tc.shape() == shape_t({2, 16, (dim_t)n}));
    auto exec = g.build(DeviceType::HIP);
    ta.copy_from_host(as_bytes(a));
    tw.copy_from_host(as_bytes(q));
    ts.copy_from_host(as_bytes(s));
    exec->execute();
    std::vector<float> out(32 * n), ref(32 * n);
    tc.copy_to_host(as_writeable_bytes(out));
    vmo_qmm_2d_f32(a.data(), q.data(), s.data(), ref.data(), 32, k, n, 1, 0);
    REQUIRE(max_abs_diff(out, ref) <= 1e-3f * max_abs(ref));
}

TEST_CASE("Float16 and BFloat16 dtype keys on HIP", "[gpu][quantization][dtype]") {
    REQUIRE_HIP();
    const std::size_t m = 2, k = 64, n = 64;
    const auto w = generate_random_weights(k, n);
    const auto a32 = generate_activations(m, k);
    std::vector<std::int8_t> q(k * n);
    std::vector<float> s32(n);
    vmo_quantize_int8_per_channel(w.data(), q.data(), s32.data(), k, n);
    for (DataType dt : {DataType::Float16, DataType::BFloat16}) {
        for (bool f32_scale : {false, true}) {
            std::vector<std::uint16_t> a16(m * k), s16(n);
            for (std::size_t i = 0; i < a16.size(); ++i)
                a16[i] = dt == DataType::Float16 ? vmo_f32_to_f16(a32[i]) : vmo_f32_to_bf16(a32[i]);
            for (std::size_t j = 0; j < n; ++j)
                s16[j] = dt == DataType::Float16 ? vmo_f32_to_f16(s32[j]) : vmo_f32_to_bf16(s32[j]);
            Graph g;
            auto ta = g.input({(dim_t)m, (dim_t)k}, dt);
            auto tw = g.input({(dim_t)k, (dim_t)n}, DataType::Int8);
            auto ts = g.input({(dim_t)n}, f32_scale ? DataType::Float32 : dt);
            auto tc = g.op(Op::QuantizedMatMul, ta, tw, ts);
            REQUIRE(tc.dtype() == dt);
            auto exec = g.build(DeviceType::HIP);
            ta.copy_from_host(as_bytes(a16));
            tw.copy_from_host(as_bytes(q));
            if (f32_scale) ts.copy_from_host(as_bytes(s32)); else ts.copy_from_host(as_bytes(s16));
            exec->execute();
            std::vector<std::uint16_t> out(m * n), ref(m * n);
            tc.copy_to_host(as_writeable_bytes(out));
            const int code = dt == DataType::Float16 ? VMO_F16 : VMO_BF16;
            vmo_qmm_scalar_mixed(a16.data(), code, q.data(), f32_scale ? (const void*)s32.data() : (const void*)s16.data(),
                                 f32_scale ? VMO_F32 : code, ref.data(), code, m, k, n, 1, 0);
            for (std::size_t i = 0; i < out.size(); ++i) {
                const float o = dt == DataType::Float16 ? vmo_f16_to_f32(out[i]) : vmo_bf16_to_f32(out[i]);
                const float r = dt == DataType::Float16 ? vmo_f16_to_f32(ref[i]) : vmo_bf16_to_f32(ref[i]);
                REQUIRE(std::isfinite(o));
                // at most one half-precision ulp apart (summation order)
                const float ulp = dt == DataType::Float16 ? 1.0f / 1024 : 1.0f / 128;
                REQUIRE(std::abs(o - r) <= ulp * std::max(std::abs(r), 1e-3f) * 2.0f);
            }
        }
    }
}

TEST_CASE("quantize_storage_int8 from a Float16 host source", "[gpu][quantization]") {
    REQUIRE_HIP();
    const std::size_t rows = 4, cols = 8;
    std::vector<float16_t> f16(rows * cols);
    for (std::size_t i = 0; i < f16.size(); ++i) f16[i] = float16_t(static_cast<float>(i + 1) * 0.1f);
    TensorStorage st;
    st.shape = {(dim_t)rows, (dim_t)cols};
    st.dtype = DataType::Float16;
    st.data = f16.data();
    st.size_bytes = st.capacity_bytes = f16.size() * 2;
    auto [q, s] = quantize_storage_int8(st, DeviceType::CPU);
    REQUIRE(q && s && q->dtype == DataType::Int8 && s->dtype == DataType::Float32);
    REQUIRE(q->device == DeviceType::CPU);
    REQUIRE(q->shape == shape_t({(dim_t)rows, (dim_t)cols}) && s->shape == shape_t({(dim_t)cols}));
    std::vector<float> w32(f16.size());
    for (std::size_t i = 0; i < f16.size(); ++i) w32[i] = static_cast<float>(f16[i]);
    std::vector<std::int8_t> q_ref(rows * cols);
    std::vector<float> s_ref(cols);
    vmo_quantize_int8_per_channel(w32.data(), q_ref.data(), s_ref.data(), rows, cols);
    REQUIRE(std::memcmp(q->data, q_ref.data(), q_ref.size()) == 0);
    REQUIRE(std::memcmp(s->data, s_ref.data(), s_ref.size() * 4) == 0);
}

TEST_CASE("HIP graph memory plan uses one device arena", "[gpu][memory]") {
    REQUIRE_HIP();
    Graph g;
    auto x = g.input({1, 256}, DataType::Float32);
    Tensor h = x;
    std::vector<std::pair<Tensor, Tensor>> ws;
    for (int i = 0; i < 5; ++i) {
        auto w = g.input({256, 256}, DataType::Int8);
        auto s = g.input({256}, DataType::Float32);
        ws.push_back({w, s});
        h = g.op(Op::QuantizedMatMul, h, w, s);
    }
    g.mark_output(h);
    auto exec = g.build(DeviceType::HIP);
    const auto& st = exec->memory_plan_stats();
    REQUIRE(st.intermediate_tensor_count == 4);
    REQUIRE(st.allocation_count == 1 + 1 + 10 + 1);  // arena + x + weights/scales + output
    // run it: identity-like weights (code 127 on the diagonal, scale 1/127)
    std::vector<std::int8_t> eye(256 * 256, 0);
    for (int i = 0; i < 256; ++i) eye[i * 256 + i] = 127;
    std::vector<float> sc(256, 1.0f / 127.0f);
    for (auto& [w, s] : ws) {
        w.copy_from_host(as_bytes(eye));
        s.copy_from_host(as_bytes(sc));
    }
    const auto xv = normal(256, 9);
    x.copy_from_host(as_bytes(xv));
    exec->execute();
    std::vector<float> out(256);
    h.copy_to_host(as_writeable_bytes(out));
    REQUIRE(max_abs_diff(out, xv) <= 1e-5f * max_abs(xv));
}

TEST_CASE("HIP storages of a rebuilt graph come from the block cache", "[gpu][memory]") {
    REQUIRE_HIP();
    // The reference engine rebuilds its graph per call: the second build
    // of the same graph allocates from the blocks the first one freed and
    // gives identical results.
    const std::size_t k = 256;
    const auto w = normal(k * k, 31, 0.02f);
    std::vector<std::int8_t> q(k * k);
    std::vector<float> s(k);
    vmo_quantize_int8_per_channel(w.data(), q.data(), s.data(), k, k);
    const auto a = normal(k, 32);
    auto run = [&]() {
        Graph g;
        auto x = g.input({1, (dim_t)k}, DataType::Float32);
        auto tw = g.input({(dim_t)k, (dim_t)k}, DataType::Int8);
        auto ts = g.input({(dim_t)k}, DataType::Float32);
        auto h = g.op(Op::QuantizedMatMul, x, tw, ts);
        auto y = g.op(Op::QuantizedMatMul, h, tw, ts);
        g.mark_output(y);
        auto exec = g.build(DeviceType::HIP);
        x.copy_from_host(as_bytes(a));
        tw.copy_from_host(as_bytes(q));
        ts.copy_from_host(as_bytes(s));
        exec->execute();
        REQUIRE(y.capacity_bytes() >= y.nbytes());
        std::vector<float> out(k);
        y.copy_to_host(as_writeable_bytes(out));
        return out;
    };
    const auto o1 = run();
    const auto o2 = run();
    REQUIRE(std::memcmp(o1.data(), o2.data(), k * 4) == 0);
    std::vector<float> h(k), ref(k);
    vmo_qmm_2d_f32(a.data(), q.data(), s.data(), h.data(), 1, k, k, 1, 0);
    vmo_qmm_2d_f32(h.data(), q.data(), s.data(), ref.data(), 1, k, k, 1, 0);
    REQUIRE(max_abs_diff(o1, ref) <= 1e-5f * max_abs(ref));

    // A freed block returns for the next request of its size class (a
    // size no other test uses, so the class holds only this block), also
    // for a request one K/V row larger; its contents survive the round trip.
    const std::size_t bytes = 7654321;
    auto st = internal::create_tensor_storage(bytes, DeviceType::HIP);
    REQUIRE(st->capacity_bytes >= bytes);
    const void* p = st->data;
    std::vector<std::uint8_t> pattern(bytes), back(bytes);
    for (std::size_t i = 0; i < bytes; ++i) pattern[i] = static_cast<std::uint8_t>(i * 7 + 3);
    REQUIRE(vm_hip_memcpy_h2d(st->data, pattern.data(), bytes, nullptr) == 0);
    st.reset();
    auto again = internal::create_tensor_storage(bytes + 256, DeviceType::HIP);
    REQUIRE(again->data == p);
    REQUIRE(again->size_bytes == bytes + 256);
    REQUIRE(vm_hip_memcpy_d2h(back.data(), again->data, bytes, nullptr) == 0);
    REQUIRE(back == pattern);
    auto other = internal::create_tensor_storage(bytes, DeviceType::HIP);   // the class is empty again
    REQUIRE(other->data != p);
}

TEST_CASE("byte-preserving Reshape and Transpose steps view their input", "[gpu][memory]") {
    REQUIRE_HIP();
    // x + y -> Transpose moving a unit axis -> Reshape -> (+ itself), and a
    // Transpose that does reorder bytes; results equal with the views on
    // and off (VELOMIND_GRAPH_ALIAS=0), and an intermediate's bytes stay
    // valid while a view of them is read later in the plan.
    const auto a = normal(6 * 4, 41);
    const auto b = normal(6 * 4, 42);
    auto run = [&]() {
        Graph g;
        auto x = g.input({1, 6, 4}, DataType::Float32);
        auto y = g.input({1, 6, 4}, DataType::Float32);
        auto t1 = g.op(Op::Add, x, y);
        auto t2 = g.op(OpDescriptor{Op::Transpose, TransposeAttrs{{1, 0, 2}}}, t1);    // [6, 1, 4], same bytes
        auto t3 = g.op(OpDescriptor{Op::Reshape, ReshapeAttrs{shape_t{24}}}, t2);
        auto t4 = g.op(OpDescriptor{Op::Transpose, TransposeAttrs{{0, 2, 1}}}, t1);    // [1, 4, 6], reordered
        auto t5 = g.op(OpDescriptor{Op::Reshape, ReshapeAttrs{shape_t{24}}}, t4);
        auto u = g.op(Op::Mul, x, y);   // more intermediates in flight
        auto u2 = g.op(OpDescriptor{Op::Reshape, ReshapeAttrs{shape_t{24}}}, u);
        auto o1 = g.op(Op::Add, t3, u2);
        auto o2 = g.op(Op::Add, t5, t3);
        g.mark_output(o1);
        g.mark_output(o2);
        auto exec = g.build(DeviceType::HIP);
        x.copy_from_host(as_bytes(a));
        y.copy_from_host(as_bytes(b));
        exec->execute();
        std::vector<float> r1(24), r2(24);
        o1.copy_to_host(as_writeable_bytes(r1));
        o2.copy_to_host(as_writeable_bytes(r2));
        return std::make_pair(r1, r2);
    };
    const auto on = run();
    ::setenv("VELOMIND_GRAPH_ALIAS", "0", 1);
    const auto off = run();
    ::unsetenv("VELOMIND_GRAPH_ALIAS");
    REQUIRE(std::memcmp(on.first.data(), off.first.data(), 24 * 4) == 0);
    REQUIRE(std::memcmp(on.second.data(), off.second.data(), 24 * 4) == 0);
    for (int e = 0; e < 24; ++e) {
        volatile float sum = a[e] + b[e], prod = a[e] * b[e];   // rounded as the device rounds them
        REQUIRE(on.first[e] == sum + prod);
    }
    for (int j = 0; j < 4; ++j)
        for (int i = 0; i < 6; ++i) {
            const float t4 = a[i * 4 + j] + b[i * 4 + j];          // t1[i][j] at t4[j][i]
            const float t3 = a[j * 6 + i] + b[j * 6 + i];          // t3 flat index j * 6 + i
            REQUIRE(on.second[j * 6 + i] == t4 + t3);
        }
}

TEST_CASE("bind_input uses an external device buffer", "[gpu][api]") {
    REQUIRE_HIP();
    const std::size_t k = 128, n = 64;
    const auto w = generate_random_weights(k, n);
    std::vector<std::int8_t> q(k * n);
    std::vector<float> s(n);
    vmo_quantize_int8_per_channel(w.data(), q.data(), s.data(), k, n);
    Graph g;
    auto ta = g.input({1, (dim_t)k}, DataType::Float32);
    auto tw = g.input({(dim_t)k, (dim_t)n}, DataType::Int8);
    auto ts = g.input({(dim_t)n}, DataType::Float32);
    auto tc = g.op(Op::QuantizedMatMul, ta, tw, ts);
    auto exec = g.build(DeviceType::HIP);
    void* dev = nullptr;
    REQUIRE(vm_hip_malloc(&dev, k * 4) == 0);
    std::shared_ptr<void> owner(dev, [](void* p) { vm_hip_free(p); });
    const auto a = generate_activations(1, k);
    REQUIRE(vm_hip_memcpy_h2d(dev, a.data(), k * 4, nullptr) == 0);
    exec->bind_input(ta, ExternalBuffer{dev, k * 4, DeviceType::HIP, owner});
    REQUIRE(ta.data() == dev);
    tw.copy_from_host(as_bytes(q));
    ts.copy_from_host(as_bytes(s));
    exec->execute();
    std::vector<float> out(n), ref(n);
    tc.copy_to_host(as_writeable_bytes(out));
    vmo_qmm_2d_f32(a.data(), q.data(), s.data(), ref.data(), 1, k, n, 1, 0);
    REQUIRE(max_abs_diff(out, ref) < 1e-4f);
    REQUIRE_THROWS_AS(exec->bind_input(ta, ExternalBuffer{dev, 4, DeviceType::HIP, owner}), std::invalid_argument);
    REQUIRE_THROWS_AS(exec->bind_input(tc, ExternalBuffer{dev, k * 4, DeviceType::HIP, owner}), std::invalid_argument);
}

TEST_CASE("injected backend failures carry the reference's message format", "[gpu][failure]") {
    REQUIRE_HIP();
    Graph g;
    auto ta = g.input({1, 64}, DataType::Float32);
    auto tw = g.input({64, 32}, DataType::Int8);
    auto ts = g.input({32}, DataType::Float32);
    g.op(Op::QuantizedMatMul, ta, tw, ts);
    auto exec = g.build(DeviceType::HIP);
    for (const char* stage : {"launch", "sync"}) {
        const std::string spec = std::string("HIP:QuantizedMatMul:") + stage;
        ScopedEnv env("VELOMIND_FAIL_BACKEND", spec.c_str());
        bool thrown = false;
        try {
            exec->execute();
        } catch (const std::runtime_error& e) {
            const std::string msg = e.what();
            thrown = msg.find("QuantizedMatMul on HIP output shape=[1,32] at ") != std::string::npos &&
                     msg.find("injected failure") != std::string::npos;
        }
        REQUIRE(thrown);
    }
    REQUIRE_NOTHROW(exec->execute());  // recovers once the injection is gone
}

TEST_CASE("concurrent build and execute on per-thread HIP streams", "[gpu][threads]") {
    REQUIRE_HIP();
    const std::size_t k = 512, n = 1024;
    const auto w = normal(k * n, 21, 0.02f);
    std::vector<std::int8_t> q(k * n);
    std::vector<float> s(n);
    vmo_quantize_int8_per_channel(w.data(), q.data(), s.data(), k, n);
    std::atomic<int> ok{0};
    std::vector<std::thread> threads;
    for (int t = 0; t < 6; ++t) {
        threads.emplace_back([&, t] {
            try {
                for (int it = 0; it < 5; ++it) {
                    const std::size_t m = 1 + (t + it) % 4;
                    const auto a = normal(m * k, 100 + t * 10 + it);
                    const auto out = run_graph(DeviceType::HIP, QmmCase{m, k, n, QuantType::Int8, 0}, a, q, s);
                    std::vector<float> ref(m * n);
                    vmo_qmm_2d_f32(a.data(), q.data(), s.data(), ref.data(), m, k, n, 1, 0);
                    if (max_abs_diff(out, ref) > 1e-5f * max_abs(ref)) return;
                }
                ++ok;
            } catch (...) {
            }
        });
    }
    for (auto& th : threads) th.join();
    REQUIRE(ok == 6);
}

TEST_CASE("sibling QuantizedMatMuls sharing A run as one grouped step", "[gpu][quantization][group]") {
    // q | v read x with INT4 block-32 weights and no other input pending:
    // one grouped step.  k's scales come from an Add that follows q in the
    // order, so k is not ready at q's step and runs on its own; gate | up
    // (INT8 per column) read x too but quantise differently: their own
    // group.  Eight rows of A: no grouping at all.
    REQUIRE_HIP();
    const std::size_t k = 256, nq = 256, nkv = 64, ni = 192;
    auto int4 = [&](std::size_t n, std::uint64_t seed) {
        const auto w = normal(k * n, seed, 0.02f);
        std::vector<std::int8_t> q((k / 2) * n);
        std::vector<float> s((k / 32) * n);
        vmo_quantize_int4_block(w.data(), reinterpret_cast<std::uint8_t*>(q.data()), s.data(), k, n, 32);
        return std::pair{q, s};
    };
    auto int8 = [&](std::size_t n, std::uint64_t seed) {
        const auto w = normal(k * n, seed, 0.02f);
        std::vector<std::int8_t> q(k * n);
        std::vector<float> s(n);
        vmo_quantize_int8_per_channel(w.data(), q.data(), s.data(), k, n);
        return std::pair{q, s};
    };
    const auto [wq, sq] = int4(nq, 1);
    const auto [wk, sk] = int4(nkv, 2);
    const auto [wv, sv] = int4(nkv, 3);
    const auto [wg, sg] = int8(ni, 4);
    const auto [wu, su] = int8(ni, 5);
    const QuantizedMatMulAttrs a4{.quant_type = QuantType::Int4, .block_size = 32};
    const QuantizedMatMulAttrs a8{.quant_type = QuantType::Int8, .block_size = 0};
    const std::vector<float> zeros(sk.size(), 0.0f);

    for (std::size_t m : {1, 4, 8}) {
        const auto xv = normal(m * k, 10 + m);
        auto run = [&](bool grouped, std::size_t* steps) {
            ScopedEnv env("VELOMIND_GROUP_QMM", grouped ? "1" : "0");
            Graph g;
            auto x = g.input({(dim_t)m, (dim_t)k}, DataType::Float32);
            auto in = [&](const auto& v, shape_t shape, DataType dt) {
                auto t = g.input(shape, dt);
                return std::pair{t, &v};
            };
            auto [tq, pq] = in(wq, {(dim_t)k / 2, (dim_t)nq}, DataType::Int8);
            auto [tsq, psq] = in(sq, {(dim_t)k / 32, (dim_t)nq}, DataType::Float32);
            auto [tk, pk] = in(wk, {(dim_t)k / 2, (dim_t)nkv}, DataType::Int8);
            auto [tsk, psk] = in(sk, {(dim_t)k / 32, (dim_t)nkv}, DataType::Float32);
            auto [tz, pz] = in(zeros, {(dim_t)k / 32, (dim_t)nkv}, DataType::Float32);
            auto [tv, pv] = in(wv, {(dim_t)k / 2, (dim_t)nkv}, DataType::Int8);
            auto [tsv, psv] = in(sv, {(dim_t)k / 32, (dim_t)nkv}, DataType::Float32);
            auto [tg, pg] = in(wg, {(dim_t)k, (dim_t)ni}, DataType::Int8);
            auto [tsg, psg] = in(sg, {(dim_t)ni}, DataType::Float32);
            auto [tu, pu] = in(wu, {(dim_t)k, (dim_t)ni}, DataType::Int8);
            auto [tsu, psu] = in(su, {(dim_t)ni}, DataType::Float32);
            auto yq = g.op(OpDescriptor{Op::QuantizedMatMul, a4}, x, tq, tsq);
            // tz holds zeros: tz + sk is sk exactly, produced by a node
            // that follows q in the order
            auto sk2 = g.op(Op::Add, tz, tsk);
            auto yk = g.op(OpDescriptor{Op::QuantizedMatMul, a4}, x, tk, sk2);
            auto yv = g.op(OpDescriptor{Op::QuantizedMatMul, a4}, x, tv, tsv);
            auto yg = g.op(OpDescriptor{Op::QuantizedMatMul, a8}, x, tg, tsg);
            auto yu = g.op(OpDescriptor{Op::QuantizedMatMul, a8}, x, tu, tsu);
            g.mark_output(yq);
            g.mark_output(yk);
            g.mark_output(yv);
            g.mark_output(yg);
            g.mark_output(yu);
            auto exec = g.build(DeviceType::HIP);
            REQUIRE(exec->num_nodes() == 6);
            *steps = exec->num_steps();
            x.copy_from_host(as_bytes(xv));
            tq.copy_from_host(as_bytes(*pq));
            tsq.copy_from_host(as_bytes(*psq));
            tk.copy_from_host(as_bytes(*pk));
            tsk.copy_from_host(as_bytes(*psk));
            tz.copy_from_host(as_bytes(*pz));
            tv.copy_from_host(as_bytes(*pv));
            tsv.copy_from_host(as_bytes(*psv));
            tg.copy_from_host(as_bytes(*pg));
            tsg.copy_from_host(as_bytes(*psg));
            tu.copy_from_host(as_bytes(*pu));
            tsu.copy_from_host(as_bytes(*psu));
            exec->execute();
            std::vector<std::vector<float>> out;
            for (auto [t, n] : std::vector<std::pair<Tensor, std::size_t>>{{yq, nq}, {yk, nkv}, {yv, nkv}, {yg, ni}, {yu, ni}}) {
                std::vector<float> o(m * n);
                t.copy_to_host(as_writeable_bytes(o));
                out.push_back(std::move(o));
            }
            return out;
        };
        std::size_t steps_grouped = 0, steps_single = 0;
        const auto grouped = run(true, &steps_grouped);
        const auto single = run(false, &steps_single);
        REQUIRE(steps_single == 6);
        // m <= 4: {q, v}, add, {gate, up}, k; m = 8: nothing grouped
        REQUIRE(steps_grouped == (m <= 4 ? 4 : 6));
        const std::vector<std::tuple<const std::vector<std::int8_t>*, const std::vector<float>*, std::size_t, int>>
            mats{{&wq, &sq, nq, 2}, {&wk, &sk, nkv, 2}, {&wv, &sv, nkv, 2}, {&wg, &sg, ni, 1}, {&wu, &su, ni, 1}};
        for (std::size_t i = 0; i < mats.size(); ++i) {
            const auto& [w, s, n, qt] = mats[i];
            std::vector<float> ref(m * n);
            vmo_qmm_2d_f32(xv.data(), w->data(), s->data(), ref.data(), m, k, n, qt, qt == 2 ? 32 : 0);
            const float bound = (m <= 4 ? 1e-5f : 1e-3f) * max_abs(ref);
            REQUIRE(max_abs_diff(grouped[i], ref) <= bound);
            REQUIRE(max_abs_diff(grouped[i], single[i]) <= 1e-6f * max_abs(single[i]));
        }
    }
}

namespace {

// A device copy of `v` with `pad_bytes` of zeros after it.
std::shared_ptr<TensorStorage> device_copy(std::span<const std::byte> v, std::size_t pad_bytes = 0) {
    auto s = TensorStorage::allocate(v.size() + pad_bytes, DeviceType::HIP);
    REQUIRE(s);
    std::vector<std::byte> host(v.begin(), v.end());
    host.resize(v.size() + pad_bytes, std::byte{0});
    REQUIRE(vm_hip_memcpy_h2d(s->data, host.data(), host.size(), nullptr) == 0);
    return s;
}

// A strided view of `base` starting `offset` bytes in.
std::shared_ptr<TensorStorage> view_of(const std::shared_ptr<TensorStorage>& base, shape_t shape, stride_t strides,
                                       DataType dt, std::size_t offset = 0) {
    auto v = std::make_shared<TensorStorage>();
    v->shape = std::move(shape);
    v->strides = std::move(strides);
    v->dtype = dt;
    v->device = DeviceType::HIP;
    v->offset_bytes = base->offset_bytes + offset;
    v->capacity_bytes = base->capacity_bytes ? base->capacity_bytes : base->size_bytes;
    v->data = static_cast<std::byte*>(base->data) + offset;
    v->size_bytes = storage_nbytes(*v);
    v->external_owner = base;
    return v;
}

template <typename T>
std::vector<T> to_host(const TensorStorage& s, std::size_t count) {
    std::vector<T> out(count);
    REQUIRE(vm_hip_device_synchronize() == 0);
    REQUIRE(vm_hip_memcpy_d2h(out.data(), s.data, count * sizeof(T), nullptr) == 0);
    return out;
}

}  // namespace

TEST_CASE("strided A, B and C on HIP match the contiguous operands bit for bit", "[gpu][quantization][strided]") {
    // The reference's CPU kernel reads A and B through their strides and
    // writes C through its strides (quantized_matmul.cpp:306-315); here
    // the adapter gathers and scatters around the contiguous kernels.
    REQUIRE_HIP();
    const std::vector<DataType> key{DataType::Float32, DataType::Int8, DataType::Float32};
    const auto fn = internal::resolve_op_kernel(Op::QuantizedMatMul, key, DataType::Float32, DeviceType::HIP);
    REQUIRE(fn != nullptr);
    const std::size_t k = 256, n = 192, pad = 16;
    for (const int qt : {1, 2}) {
        const int block = qt == 2 ? 32 : 0;
        const OpDescriptor desc{Op::QuantizedMatMul,
                                QuantizedMatMulAttrs{.quant_type = qt == 2 ? QuantType::Int4 : QuantType::Int8,
                                                     .block_size = block}};
        const std::size_t qrows = qt == 2 ? k / 2 : k;
        const auto w = normal(k * n, 90 + qt, 0.05f);
        std::vector<std::int8_t> q(qrows * n);
        std::vector<float> s(qt == 2 ? (k / 32) * n : n);
        if (qt == 2)
            vmo_quantize_int4_block(w.data(), reinterpret_cast<std::uint8_t*>(q.data()), s.data(), k, n, 32);
        else
            vmo_quantize_int8_per_channel(w.data(), q.data(), s.data(), k, n);
        // B padded to n + pad columns
        std::vector<std::int8_t> q_pitched(qrows * (n + pad), 0);
        for (std::size_t r = 0; r < qrows; ++r)
            std::memcpy(q_pitched.data() + r * (n + pad), q.data() + r * n, n);
        const auto dq = device_copy(as_bytes(q));
        const auto dq_pitched = device_copy(as_bytes(q_pitched));
        const auto ds = device_copy(as_bytes(s));
        const auto wq_dense = view_of(dq, {(dim_t)qrows, (dim_t)n}, {}, DataType::Int8);
        const auto wq_strided = view_of(dq_pitched, {(dim_t)qrows, (dim_t)n}, {(dim_t)(n + pad), 1}, DataType::Int8);
        const auto sc = view_of(ds, {(dim_t)(s.size() / n), (dim_t)n}, {}, DataType::Float32);

        for (std::size_t m : {1, 3, 16}) {
            const auto a = normal(m * k, 100 + m);
            auto call = [&](const std::shared_ptr<TensorStorage>& ta, const std::shared_ptr<TensorStorage>& tw,
                            const std::shared_ptr<TensorStorage>& tc) {
                const pConstTensorStorage ins[3] = {ta.get(), tw.get(), sc.get()};
                const pTensorStorage outs[1] = {tc.get()};
                fn(ins, outs, &desc);
            };
            // contiguous operands: the baseline, checked against the oracle
            const auto da = device_copy(as_bytes(a));
            const auto a_dense = view_of(da, {(dim_t)m, (dim_t)k}, {}, DataType::Float32);
            auto dc = TensorStorage::allocate(m * n * 4, DeviceType::HIP);
            const auto c_dense = view_of(dc, {(dim_t)m, (dim_t)n}, {}, DataType::Float32);
            call(a_dense, wq_dense, c_dense);
            const auto base = to_host<float>(*c_dense, m * n);
            std::vector<float> ref(m * n);
            vmo_qmm_2d_f32(a.data(), q.data(), s.data(), ref.data(), m, k, n, qt, block);
            REQUIRE(max_abs_diff(base, ref) <= (m <= 4 ? 1e-5f : 1e-3f) * max_abs(ref));

            auto same = [&](const std::vector<float>& got) {
                REQUIRE(got.size() == base.size());
                REQUIRE(std::memcmp(got.data(), base.data(), base.size() * 4) == 0);
            };
            // A with a row pitch of k + 8, 4 floats into its allocation
            {
                std::vector<float> a_pitched(4 + m * (k + 8), 9.0f);
                for (std::size_t r = 0; r < m; ++r)
                    std::memcpy(a_pitched.data() + 4 + r * (k + 8), a.data() + r * k, k * 4);
                const auto d = device_copy(as_bytes(a_pitched));
                const auto av = view_of(d, {(dim_t)m, (dim_t)k}, {(dim_t)(k + 8), 1}, DataType::Float32, 16);
                REQUIRE(m == 1 || !av->is_contiguous());   // one row: any pitch is dense
                auto dc2 = TensorStorage::allocate(m * n * 4, DeviceType::HIP);
                const auto c2 = view_of(dc2, {(dim_t)m, (dim_t)n}, {}, DataType::Float32);
                call(av, wq_dense, c2);
                same(to_host<float>(*c2, m * n));
            }
            // A transposed: the [k, m] array read as [m, k] with strides {1, m}
            if (m > 1) {
                std::vector<float> at(k * m);
                for (std::size_t r = 0; r < m; ++r)
                    for (std::size_t j = 0; j < k; ++j) at[j * m + r] = a[r * k + j];
                const auto d = device_copy(as_bytes(at));
                const auto av = view_of(d, {(dim_t)m, (dim_t)k}, {1, (dim_t)m}, DataType::Float32);
                auto dc2 = TensorStorage::allocate(m * n * 4, DeviceType::HIP);
                const auto c2 = view_of(dc2, {(dim_t)m, (dim_t)n}, {}, DataType::Float32);
                call(av, wq_dense, c2);
                same(to_host<float>(*c2, m * n));
            }
            // B with a row pitch of n + pad
            {
                auto dc2 = TensorStorage::allocate(m * n * 4, DeviceType::HIP);
                const auto c2 = view_of(dc2, {(dim_t)m, (dim_t)n}, {}, DataType::Float32);
                call(a_dense, wq_strided, c2);
                same(to_host<float>(*c2, m * n));
            }
            // C written into columns [0, n) of an [m, n + pad] array: the
            // pad columns keep their values
            {
                const std::vector<float> sentinel(m * (n + pad), 7.0f);
                const auto d = device_copy(as_bytes(sentinel));
                const auto cv = view_of(d, {(dim_t)m, (dim_t)n}, {(dim_t)(n + pad), 1}, DataType::Float32);
                call(a_dense, wq_dense, cv);
                const auto all = to_host<float>(*d, m * (n + pad));
                std::vector<float> got(m * n);
                for (std::size_t r = 0; r < m; ++r) {
                    std::memcpy(got.data() + r * n, all.data() + r * (n + pad), n * 4);
                    for (std::size_t j = n; j < n + pad; ++j) REQUIRE(all[r * (n + pad) + j] == 7.0f);
                }
                same(got);
            }
            // A as [2, m, k] batches with a gap of one row between them
            // (rows 0..m-1 then m+1..2m): C [2, m, n] against the dense call
            // on the gathered rows
            {
                const auto a2 = normal(2 * m * k, 200 + m);
                std::vector<float> a_gap((2 * m + 1) * k, 5.0f);
                for (std::size_t b = 0; b < 2; ++b)
                    std::memcpy(a_gap.data() + b * (m + 1) * k, a2.data() + b * m * k, m * k * 4);
                const auto dg = device_copy(as_bytes(a_gap));
                const auto av = view_of(dg, {2, (dim_t)m, (dim_t)k}, {(dim_t)((m + 1) * k), (dim_t)k, 1},
                                        DataType::Float32);
                const auto dd = device_copy(as_bytes(a2));
                const auto ad = view_of(dd, {2, (dim_t)m, (dim_t)k}, {}, DataType::Float32);
                auto c_gap = TensorStorage::allocate(2 * m * n * 4, DeviceType::HIP);
                auto c_ref = TensorStorage::allocate(2 * m * n * 4, DeviceType::HIP);
                const auto cg = view_of(c_gap, {2, (dim_t)m, (dim_t)n}, {}, DataType::Float32);
                const auto cr = view_of(c_ref, {2, (dim_t)m, (dim_t)n}, {}, DataType::Float32);
                call(ad, wq_dense, cr);
                call(av, wq_dense, cg);
                const auto want = to_host<float>(*cr, 2 * m * n);
                const auto got = to_host<float>(*cg, 2 * m * n);
                REQUIRE(std::memcmp(got.data(), want.data(), want.size() * 4) == 0);
            }
        }
    }
}

TEST_CASE("strided operands that overlap or overrun are refused before any launch", "[gpu][quantization][strided]") {
    REQUIRE_HIP();
    const std::vector<DataType> key{DataType::Float32, DataType::Int8, DataType::Float32};
    const auto fn = internal::resolve_op_kernel(Op::QuantizedMatMul, key, DataType::Float32, DeviceType::HIP);
    REQUIRE(fn != nullptr);
    const std::size_t m = 2, k = 64, n = 32;
    const OpDescriptor desc{Op::QuantizedMatMul, QuantizedMatMulAttrs{.quant_type = QuantType::Int8, .block_size = 0}};
    const auto da = device_copy(as_bytes(normal(m * k, 1)));
    const auto dw = device_copy(as_bytes(std::vector<std::int8_t>(k * n, 1)));
    const auto ds = device_copy(as_bytes(std::vector<float>(n, 0.5f)));
    const auto dc = device_copy(as_bytes(std::vector<float>(m * n, 0.0f)));
    const auto a = view_of(da, {(dim_t)m, (dim_t)k}, {}, DataType::Float32);
    const auto w = view_of(dw, {(dim_t)k, (dim_t)n}, {}, DataType::Int8);
    const auto s = view_of(ds, {(dim_t)n}, {}, DataType::Float32);
    auto call = [&](const std::shared_ptr<TensorStorage>& ta, const std::shared_ptr<TensorStorage>& tc) {
        const pConstTensorStorage ins[3] = {ta.get(), w.get(), s.get()};
        const pTensorStorage outs[1] = {tc.get()};
        fn(ins, outs, &desc);
    };
    // both rows of C on the same addresses
    REQUIRE_THROWS_AS(call(a, view_of(dc, {(dim_t)m, (dim_t)n}, {0, 1}, DataType::Float32)), std::invalid_argument);
    // rows half a row apart: row 1 overlaps row 0
    REQUIRE_THROWS_AS(call(a, view_of(dc, {(dim_t)m, (dim_t)n}, {(dim_t)(n / 2), 1}, DataType::Float32)),
                      std::invalid_argument);
    // A's row pitch reaching past its allocation (declared as exactly m * k floats)
    auto overrun = view_of(da, {(dim_t)m, (dim_t)k}, {(dim_t)(k + 1), 1}, DataType::Float32);
    overrun->capacity_bytes = m * k * 4;
    REQUIRE_THROWS_AS(call(overrun, view_of(dc, {(dim_t)m, (dim_t)n}, {}, DataType::Float32)), std::invalid_argument);
    // a repeated A row (stride 0) is a legal read
    call(view_of(da, {(dim_t)m, (dim_t)k}, {0, 1}, DataType::Float32),
         view_of(dc, {(dim_t)m, (dim_t)n}, {}, DataType::Float32));
    const auto c = to_host<float>(*dc, m * n);
    REQUIRE(std::memcmp(c.data(), c.data() + n, n * 4) == 0);
}

TEST_CASE("a graph on a strided input view keeps its QuantizedMatMul + Add unfused", "[gpu][quantization][strided]") {
    // x is every other row of a device array: the residual Add stays out
    // of the second product's launch (the fused kernel takes dense operands
    // only), and both outputs equal the dense graph's bit for bit.
    REQUIRE_HIP();
    const std::size_t m = 2, k = 128, n = 128;
    const auto xv = normal(m * k, 301), hv = normal(m * n, 302);
    const auto w1 = normal(k * n, 303, 0.05f), w2 = normal(k * n, 304, 0.05f);
    std::vector<std::int8_t> q1(k * n), q2(k * n);
    std::vector<float> s1(n), s2(n);
    vmo_quantize_int8_per_channel(w1.data(), q1.data(), s1.data(), k, n);
    vmo_quantize_int8_per_channel(w2.data(), q2.data(), s2.data(), k, n);
    std::vector<float> x_gapped(2 * m * k, 3.0f);
    for (std::size_t r = 0; r < m; ++r) std::memcpy(x_gapped.data() + 2 * r * k, xv.data() + r * k, k * 4);
    const auto dx = device_copy(as_bytes(x_gapped));
    auto run = [&](bool strided, std::size_t* steps) {
        ScopedEnv env("VELOMIND_GROUP_QMM", "0");
        Graph g;
        auto x = strided ? g.input(view_of(dx, {(dim_t)m, (dim_t)k}, {(dim_t)(2 * k), 1}, DataType::Float32))
                         : g.input({(dim_t)m, (dim_t)k}, DataType::Float32);
        auto h = g.input({(dim_t)m, (dim_t)n}, DataType::Float32);
        auto t1 = g.input({(dim_t)k, (dim_t)n}, DataType::Int8), ts1 = g.input({(dim_t)n}, DataType::Float32);
        auto t2 = g.input({(dim_t)k, (dim_t)n}, DataType::Int8), ts2 = g.input({(dim_t)n}, DataType::Float32);
        auto y1 = g.op(Op::QuantizedMatMul, x, t1, ts1);
        auto y2 = g.op(Op::Add, h, g.op(Op::QuantizedMatMul, x, t2, ts2));
        g.mark_output(y1);
        g.mark_output(y2);
        auto exec = g.build(DeviceType::HIP);
        *steps = exec->num_steps();
        if (!strided) x.copy_from_host(as_bytes(xv));
        h.copy_from_host(as_bytes(hv));
        t1.copy_from_host(as_bytes(q1));
        ts1.copy_from_host(as_bytes(s1));
        t2.copy_from_host(as_bytes(q2));
        ts2.copy_from_host(as_bytes(s2));
        exec->execute();
        std::vector<float> o1(m * n), o2(m * n);
        y1.copy_to_host(as_writeable_bytes(o1));
        y2.copy_to_host(as_writeable_bytes(o2));
        return std::pair{o1, o2};
    };
    std::size_t dense_steps = 0, strided_steps = 0;
    const auto dense = run(false, &dense_steps);
    const auto strided = run(true, &strided_steps);
    REQUIRE(dense_steps == 2);     // product, product + Add fused
    REQUIRE(strided_steps == 3);   // product, product, Add
    REQUIRE(std::memcmp(dense.first.data(), strided.first.data(), m * n * 4) == 0);
    REQUIRE(std::memcmp(dense.second.data(), strided.second.data(), m * n * 4) == 0);
    std::vector<float> ref(m * n);
    vmo_qmm_2d_f32(xv.data(), q1.data(), s1.data(), ref.data(), m, k, n, 1, 0);
    REQUIRE(max_abs_diff(strided.first, ref) <= 1e-5f * max_abs(ref));
}
