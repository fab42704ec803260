// Quantization API of the reference's src/quant.cpp, served by the GPU
// packers of libvmhip (bit-exact with the reference's host loops).  Host
// pointers are staged through device buffers; TensorStorage sources may
// live on the host or on HIP.  compute_quantization_metrics is plain host
// arithmetic (double accumulation, quant.cpp:26-72).
#include <cmath>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "backend_hip/hip_runtime.h"
#include "internal/registry/memory_transfer.h"
#include "velomind/quant.h"
#include "vm_hip.h"

namespace velomind {

namespace {

// Device allocation owned by a scope.
class DeviceBuffer {
public:
    explicit DeviceBuffer(std::size_t bytes) {
        backend::hip::check_status(vm_hip_malloc(&_p, bytes), "quantize: device allocation");
    }
    ~DeviceBuffer() {
        if (_p) (void)vm_hip_free(_p);
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    template <typename T = void>
    T* get() const { return static_cast<T*>(_p); }

private:
    void* _p = nullptr;
};

void require_hip(const char* what) {
    int n = 0;
    if (vm_hip_device_count(&n) != VM_HIP_OK || n < 1)
        throw std::runtime_error(std::string(what) + ": no HIP (gfx950) device available; this build packs on the GPU");
}

void h2d(void* dst, const void* src, std::size_t bytes) {
    backend::hip::check_status(vm_hip_memcpy_h2d(dst, src, bytes, backend::hip::current_stream()), "quantize: H2D");
}

void d2h(void* dst, const void* src, std::size_t bytes) {
    backend::hip::check_status(vm_hip_memcpy_d2h(dst, src, bytes, backend::hip::current_stream()), "quantize: D2H");
}

void sync() { backend::hip::check_status(vm_hip_stream_synchronize(backend::hip::current_stream()), "quantize: sync"); }

// fp32 copy of a 2-D source storage on the device; returns the pointer
// (either the source itself or `holder`'s buffer).
const float* device_f32_source(const TensorStorage& src, std::size_t numel, std::unique_ptr<DeviceBuffer>& holder) {
    if (src.device == DeviceType::HIP) {
        if (src.dtype == DataType::Float32) return static_cast<const float*>(src.data);
        if (src.dtype != DataType::Float16 && src.dtype != DataType::BFloat16)
            throw std::invalid_argument("quantize_storage: HIP source must be Float32, Float16 or BFloat16");
        holder = std::make_unique<DeviceBuffer>(numel * sizeof(float));
        backend::hip::check_status(
            vm_hip_half_to_f32(static_cast<const std::uint16_t*>(src.data),
                               src.dtype == DataType::Float16 ? VM_HIP_DTYPE_F16 : VM_HIP_DTYPE_BF16,
                               holder->get<float>(), static_cast<std::int64_t>(numel), backend::hip::current_stream()),
            "quantize_storage: widen source");
        return holder->get<float>();
    }
    if (src.device != DeviceType::CPU) throw std::invalid_argument("quantize_storage: source must be on CPU or HIP");
    std::vector<float> host(numel);
    if (src.dtype == DataType::Float32)
        std::memcpy(host.data(), src.data, numel * sizeof(float));
    else
        convert_dtype(src.data, src.dtype, host.data(), DataType::Float32, numel);
    holder = std::make_unique<DeviceBuffer>(numel * sizeof(float));
    h2d(holder->get(), host.data(), numel * sizeof(float));
    return holder->get<float>();
}

std::shared_ptr<TensorStorage> make_result(std::size_t bytes, DeviceType device, shape_t shape, DataType dtype) {
    auto s = TensorStorage::allocate(bytes, device);
    if (!s) throw std::runtime_error(std::string("quantize_storage: no allocator for device ") + device_type_name(device));
    s->shape = std::move(shape);
    s->strides = default_strides(s->shape);
    s->dtype = dtype;
    s->size_bytes = bytes;
    s->capacity_bytes = bytes;
    s->device = device;
    return s;
}

// Packs into device buffers `q_dev` / `s_dev`, then places them on `device`.
template <typename PackFn>
auto pack_storage(const TensorStorage& src, DeviceType device, std::size_t q_bytes, shape_t q_shape,
                  std::size_t s_bytes, shape_t s_shape, PackFn&& pack)
    -> std::pair<std::shared_ptr<TensorStorage>, std::shared_ptr<TensorStorage>> {
    require_hip("quantize_storage");
    const std::size_t numel = static_cast<std::size_t>(src.shape[0]) * static_cast<std::size_t>(src.shape[1]);
    if (numel > 0 && !src.data) throw std::invalid_argument("quantize_storage: source has no data");
    auto q = make_result(q_bytes, device, std::move(q_shape), DataType::Int8);
    auto s = make_result(s_bytes, device, std::move(s_shape), DataType::Float32);
    if (numel == 0) return {q, s};
    std::unique_ptr<DeviceBuffer> f32_holder;
    const float* w = device_f32_source(src, numel, f32_holder);
    if (device == DeviceType::HIP) {
        pack(w, q->data, static_cast<float*>(s->data));
        sync();
    } else {
        DeviceBuffer dq(q_bytes), ds(s_bytes);
        pack(w, dq.get(), ds.get<float>());
        d2h(q->data, dq.get(), q_bytes);
        d2h(s->data, ds.get(), s_bytes);
    }
    return {q, s};
}

}  // namespace

auto compute_quantization_metrics(const float* original, const float* reconstructed, std::size_t count)
    -> QuantizationMetrics {
    QuantizationMetrics m;
    if (count == 0 || !original || !reconstructed) return m;
    float max_diff = 0.0f;
    double sdd = 0.0, soo = 0.0, srr = 0.0, sor = 0.0;
    for (std::size_t i = 0; i < count; ++i) {
        const double o = original[i], r = reconstructed[i];
        const double d = std::abs(o - r);
        if (d > max_diff) max_diff = static_cast<float>(d);
        sdd += d * d;
        soo += o * o;
        srr += r * r;
        sor += o * r;
    }
    m.max_diff = max_diff;
    m.rmse = static_cast<float>(std::sqrt(sdd / static_cast<double>(count)));
    m.snr_db = sdd > 1e-15 ? static_cast<float>(10.0 * std::log10(soo / sdd)) : 100.0f;
    const double den = std::sqrt(soo) * std::sqrt(srr);
    m.cosine_sim = den > 1e-15 ? static_cast<float>(sor / den) : 1.0f;
    return m;
}

void quantize_weights_int8_per_channel(const float* src, std::int8_t* dst_q, float* dst_scale, std::size_t rows,
                                       std::size_t cols) {
    if (!src || !dst_q || !dst_scale || rows == 0 || cols == 0) return;  // quant.cpp:81-83
    require_hip("quantize_weights_int8_per_channel");
    DeviceBuffer w(rows * cols * 4), q(rows * cols), s(cols * 4);
    h2d(w.get(), src, rows * cols * 4);
    backend::hip::check_status(vm_hip_pack_int8(w.get<float>(), q.get<std::int8_t>(), s.get<float>(),
                                                 static_cast<std::int64_t>(rows), static_cast<std::int64_t>(cols),
                                                 backend::hip::current_stream()),
                               "quantize_weights_int8_per_channel");
    d2h(dst_q, q.get(), rows * cols);
    d2h(dst_scale, s.get(), cols * 4);
}

void dequantize_weights_int8_per_channel(const std::int8_t* src_q, const float* scale, float* dst, std::size_t rows,
                                         std::size_t cols) {
    if (!src_q || !scale || !dst || rows == 0 || cols == 0) return;
    require_hip("dequantize_weights_int8_per_channel");
    DeviceBuffer q(rows * cols), s(cols * 4), w(rows * cols * 4);
    h2d(q.get(), src_q, rows * cols);
    h2d(s.get(), scale, cols * 4);
    backend::hip::check_status(vm_hip_dequant_int8(q.get<std::int8_t>(), s.get<float>(), w.get<float>(),
                                                   static_cast<std::int64_t>(rows), static_cast<std::int64_t>(cols),
                                                   backend::hip::current_stream()),
                               "dequantize_weights_int8_per_channel");
    d2h(dst, w.get(), rows * cols * 4);
}

void quantize_weights_int4_block(const float* src, std::uint8_t* dst_packed, float* dst_scale, std::size_t rows,
                                 std::size_t cols, std::size_t block_size) {
    if (!src || !dst_packed || !dst_scale || rows == 0 || cols == 0 || block_size == 0) return;
    require_hip("quantize_weights_int4_block");
    const std::size_t prow = (rows + 1) / 2, nb = (rows + block_size - 1) / block_size;
    DeviceBuffer w(rows * cols * 4), q(prow * cols), s(nb * cols * 4);
    h2d(w.get(), src, rows * cols * 4);
    backend::hip::check_status(
        vm_hip_pack_int4(w.get<float>(), q.get<std::uint8_t>(), s.get<float>(), static_cast<std::int64_t>(rows),
                         static_cast<std::int64_t>(cols), static_cast<std::int64_t>(block_size),
                         backend::hip::current_stream()),
        "quantize_weights_int4_block");
    d2h(dst_packed, q.get(), prow * cols);
    d2h(dst_scale, s.get(), nb * cols * 4);
}

void dequantize_weights_int4_block(const std::uint8_t* src_packed, const float* scale, float* dst, std::size_t rows,
                                   std::size_t cols, std::size_t block_size) {
    if (!src_packed || !scale || !dst || rows == 0 || cols == 0 || block_size == 0) return;
    require_hip("dequantize_weights_int4_block");
    const std::size_t prow = (rows + 1) / 2, nb = (rows + block_size - 1) / block_size;
    DeviceBuffer q(prow * cols), s(nb * cols * 4), w(rows * cols * 4);
    h2d(q.get(), src_packed, prow * cols);
    h2d(s.get(), scale, nb * cols * 4);
    backend::hip::check_status(
        vm_hip_dequant_int4(q.get<std::uint8_t>(), s.get<float>(), w.get<float>(), static_cast<std::int64_t>(rows),
                            static_cast<std::int64_t>(cols), static_cast<std::int64_t>(block_size),
                            backend::hip::current_stream()),
        "dequantize_weights_int4_block");
    d2h(dst, w.get(), rows * cols * 4);
}

auto quantize_storage_int8(const TensorStorage& src, DeviceType device)
    -> std::pair<std::shared_ptr<TensorStorage>, std::shared_ptr<TensorStorage>> {
    if (src.shape.size() != 2) throw std::invalid_argument("quantize_storage_int8: only 2D weight matrices are supported");
    const auto rows = static_cast<std::size_t>(src.shape[0]);
    const auto cols = static_cast<std::size_t>(src.shape[1]);
    return pack_storage(src, device, rows * cols, {src.shape[0], src.shape[1]}, cols * 4, {src.shape[1]},
                        [&](const float* w, void* q, float* s) {
                            backend::hip::check_status(
                                vm_hip_pack_int8(w, static_cast<std::int8_t*>(q), s, static_cast<std::int64_t>(rows),
                                                 static_cast<std::int64_t>(cols), backend::hip::current_stream()),
                                "quantize_storage_int8");
                        });
}

auto quantize_storage_int4(const TensorStorage& src, std::size_t block_size, DeviceType device)
    -> std::pair<std::shared_ptr<TensorStorage>, std::shared_ptr<TensorStorage>> {
    if (src.shape.size() != 2) throw std::invalid_argument("quantize_storage_int4: only 2D weight matrices are supported");
    if (block_size == 0) throw std::invalid_argument("quantize_storage_int4: block_size must be positive");
    if (block_size % 2 != 0)
        throw std::invalid_argument("quantize_storage_int4: block_size must be even (odd blocks share packed bytes)");
    const auto rows = static_cast<std::size_t>(src.shape[0]);
    const auto cols = static_cast<std::size_t>(src.shape[1]);
    const std::size_t prow = (rows + 1) / 2, nb = (rows + block_size - 1) / block_size;
    return pack_storage(src, device, prow * cols, {static_cast<dim_t>(prow), src.shape[1]}, nb * cols * 4,
                        {static_cast<dim_t>(nb), src.shape[1]}, [&](const float* w, void* q, float* s) {
                            backend::hip::check_status(
                                vm_hip_pack_int4(w, static_cast<std::uint8_t*>(q), s, static_cast<std::int64_t>(rows),
                                                 static_cast<std::int64_t>(cols),
                                                 static_cast<std::int64_t>(block_size),
                                                 backend::hip::current_stream()),
                                "quantize_storage_int4");
                        });
}

}  // namespace velomind
