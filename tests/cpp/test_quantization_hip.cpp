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
#include <stdexcept>
#include <thread>

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
