// Op::QuantizedMatMul on DeviceType::HIP: the KernelFn adapter between the
// VeloMind operator ABI and libvmhip's vm_hip_qmm.  Behaviour follows the
// reference's adapters (src/cpu/ops/quantized_matmul.cpp:271-360,
// src/cuda/ops/quantized_matmul.cu:203-266): m and k from A's last two
// dimensions, n from B, leading batch dimensions of A/C folded into the row
// count, one launch on the executing thread's stream.  Strided A, B and C
// are honoured as the reference's CPU kernel honours them
// (quantized_matmul.cpp:306-315): they are gathered into contiguous
// temporaries (and C scattered back) around the contiguous kernels; the
// scales are read as the contiguous array the reference reads.  The fused
// adapters below take contiguous operands only (the graph compiler leaves
// chains with strided operands unfused).
#include <algorithm>
#include <cstdint>
#include <memory>
#include <string>
#include <type_traits>
#include <variant>
#include <vector>

#include "backend_hip/hip_runtime.h"
#include "internal/registry/kernel.h"

namespace velomind::backend::hip {

namespace {

template <typename T>
constexpr int dtype_code() {
    if constexpr (std::is_same_v<T, float>) return VM_HIP_DTYPE_F32;
    if constexpr (std::is_same_v<T, float16_t>) return VM_HIP_DTYPE_F16;
    if constexpr (std::is_same_v<T, bfloat16_t>) return VM_HIP_DTYPE_BF16;
}

// A strided operand's layout for vm_hip_copy_strided, after checking that
// every element it addresses lies inside its allocation (a device read or
// write outside it could fault the GPU, where the reference's CPU loop
// would merely be undefined).
struct StridedView {
    std::vector<std::int64_t> shape, strides;
};

StridedView strided_view(const TensorStorage& t, const std::string& ctx, bool written) {
    const auto st = t.effective_strides();
    if (t.shape.size() > VM_HIP_COPY_MAX_RANK)
        throw std::invalid_argument(ctx + ": strided operands above rank " + std::to_string(VM_HIP_COPY_MAX_RANK) +
                                    " are not supported on HIP");
    StridedView v;
    std::uint64_t last = 0;   // largest element offset addressed
    for (std::size_t d = 0; d < t.shape.size(); ++d) {
        if (st[d] < 0) throw std::invalid_argument(ctx + ": negative strides are not supported on HIP");
        v.shape.push_back(t.shape[d]);
        v.strides.push_back(st[d]);
        std::uint64_t span = 0;
        if (t.shape[d] > 0 &&
            (__builtin_mul_overflow(static_cast<std::uint64_t>(t.shape[d] - 1), static_cast<std::uint64_t>(st[d]),
                                    &span) ||
             __builtin_add_overflow(last, span, &last)))
            throw std::invalid_argument(ctx + ": strided extent overflows");
    }
    if (written && storage_numel(t) > 0) {
        // every element written once: taken from the smallest stride up,
        // each axis must step past everything the smaller ones reach
        std::vector<std::pair<std::int64_t, std::int64_t>> axes;   // (stride, extent) of axes longer than 1
        for (std::size_t d = 0; d < t.shape.size(); ++d)
            if (t.shape[d] > 1) axes.emplace_back(st[d], t.shape[d]);
        std::sort(axes.begin(), axes.end());
        std::uint64_t reach = 0;
        for (const auto& [stride, extent] : axes) {
            if (static_cast<std::uint64_t>(stride) <= reach)
                throw std::invalid_argument(ctx + ": the output's strides overlap its elements");
            reach += static_cast<std::uint64_t>(extent - 1) * static_cast<std::uint64_t>(stride);
        }
    }
    const std::size_t width = data_type_size(t.dtype);
    // bytes from the first element to the end of the allocation
    std::size_t avail = t.size_bytes;
    if (t.capacity_bytes > 0) avail = t.capacity_bytes > t.offset_bytes ? t.capacity_bytes - t.offset_bytes : 0;
    if (storage_numel(t) > 0 && (last >= avail / width || (last + 1) * width > avail))
        throw std::invalid_argument(ctx + ": strided extent exceeds the operand's allocation");
    return v;
}

std::vector<std::int64_t> row_major_strides(const std::vector<std::int64_t>& shape) {
    std::vector<std::int64_t> s(shape.size(), 1);
    for (std::size_t d = shape.size(); d-- > 1;) s[d - 1] = s[d] * shape[d];
    return s;
}

// Copies `t` into a new contiguous device buffer (or back from one).
std::shared_ptr<TensorStorage> gather(const TensorStorage& t, const std::string& ctx) {
    const auto v = strided_view(t, ctx, false);
    auto buf = TensorStorage::allocate(storage_nbytes(t), DeviceType::HIP);
    if (!buf) throw std::runtime_error(ctx + ": no HIP allocator for a contiguous copy");
    const auto dst = row_major_strides(v.shape);
    const int status = vm_hip_copy_strided(buf->data, dst.data(), t.data, v.strides.data(), v.shape.data(),
                                           static_cast<int>(v.shape.size()), static_cast<int>(data_type_size(t.dtype)),
                                           current_stream());
    if (status != VM_HIP_OK) throw_status(status, ctx);
    return buf;
}

void scatter(const TensorStorage& from, TensorStorage& t, const std::string& ctx) {
    const auto v = strided_view(t, ctx, true);
    const auto src = row_major_strides(v.shape);
    const int status = vm_hip_copy_strided(t.data, v.strides.data(), from.data, src.data(), v.shape.data(),
                                           static_cast<int>(v.shape.size()), static_cast<int>(data_type_size(t.dtype)),
                                           current_stream());
    if (status != VM_HIP_OK) throw_status(status, ctx);
}

template <typename TAct, typename TScale, typename TOut>
void quantized_matmul_hip_impl(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    const auto* a = in[0];
    const auto* w = in[1];
    const auto* s = in[2];
    auto* c = out[0];
    if (!a || !w || !s || !c) throw std::runtime_error("quantized_matmul hip: null storage");
    const auto& desc = *static_cast<const OpDescriptor*>(attrs);
    const auto& qa = std::get<QuantizedMatMulAttrs>(desc.attrs);

    const std::size_t rank = a->shape.size();
    const std::int64_t k = a->shape[rank - 1];
    const std::int64_t n = w->shape[1];
    std::int64_t rows = 1;
    for (std::size_t i = 0; i + 1 < c->shape.size(); ++i) rows *= c->shape[i];

    const int qt = qa.quant_type == QuantType::Int4 ? VM_HIP_QUANT_INT4 : VM_HIP_QUANT_INT8;
    // The kernels read ceil(k / bs) * n scales, with bs = 32 for INT4 when
    // block_size <= 0 (quantized_matmul.cpp:67).  The operator contract lets
    // such an INT4 node through with per-column scales [n]
    // (shape_helpers.h:318-330); on the device that would read past the
    // allocation, so it is refused here instead.
    const std::int64_t bs = (qt == VM_HIP_QUANT_INT4 && qa.block_size <= 0) ? 32 : qa.block_size;
    const std::int64_t nblk = bs > 0 ? (k + bs - 1) / bs : 1;
    const std::uint64_t need_scales = static_cast<std::uint64_t>(k > 0 ? nblk : 0) * static_cast<std::uint64_t>(n);
    if (storage_numel(*s) < need_scales)
        throw std::invalid_argument(error_context(Op::QuantizedMatMul, *c, "launch") + ": scales hold " +
                                    std::to_string(storage_numel(*s)) + " values, the kernel reads " +
                                    std::to_string(need_scales) + " (" + std::to_string(nblk) + " blocks of " +
                                    std::to_string(bs > 0 ? bs : k) + " rows x " + std::to_string(n) + " columns)");
    // Strided operands: contiguous temporaries around the kernel.  They go
    // back to the block cache when this returns, and a block is reused only
    // after a device-wide synchronization that began after that, so the
    // copies queued on the stream still see them.
    const std::string ctx = error_context(Op::QuantizedMatMul, *c, "launch");
    std::shared_ptr<TensorStorage> a_tmp, w_tmp, c_tmp;
    const void* a_data = a->data;
    const void* w_data = w->data;
    void* c_data = c->data;
    if (!a->is_contiguous()) {
        a_tmp = gather(*a, ctx);
        a_data = a_tmp->data;
    }
    if (!w->is_contiguous()) {
        w_tmp = gather(*w, ctx);
        w_data = w_tmp->data;
    }
    if (!c->is_contiguous()) {
        (void)strided_view(*c, ctx, true);
        c_tmp = TensorStorage::allocate(storage_nbytes(*c), DeviceType::HIP);
        if (!c_tmp) throw std::runtime_error(ctx + ": no HIP allocator for a contiguous copy");
        c_data = c_tmp->data;
    }
    const int status = vm_hip_qmm(a_data, dtype_code<TAct>(), static_cast<const std::int8_t*>(w_data), s->data,
                                  dtype_code<TScale>(), c_data, dtype_code<TOut>(), rows, k, n, qt, qa.block_size,
                                  current_stream());
    if (status != VM_HIP_OK) {
        const std::string last = vm_hip_last_error();
        const char* stage = last.find(" at sync") != std::string::npos ? "sync" : "launch";
        throw_status(status, error_context(Op::QuantizedMatMul, *c, stage));
    }
    if (c_tmp) scatter(*c_tmp, *c, ctx);
}

// QuantizedMatMul then the Add that takes its result (fp32, fused by the
// graph compiler): inputs [A, B, scales, addend], outputs [C]; attrs the
// QuantizedMatMul's descriptor.  Checked as a single node is.
void quantized_matmul_add_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    const auto* a = in[0];
    const auto* w = in[1];
    const auto* s = in[2];
    const auto* h = in[3];
    auto* c = out[0];
    if (!a || !w || !s || !h || !c) throw std::runtime_error("quantized_matmul+add hip: null storage");
    const auto& qa = std::get<QuantizedMatMulAttrs>(static_cast<const OpDescriptor*>(attrs)->attrs);
    if (!a->is_contiguous() || !w->is_contiguous() || !s->is_contiguous() || !h->is_contiguous() ||
        !c->is_contiguous())
        throw std::invalid_argument(error_context(Op::QuantizedMatMul, *c, "launch") +
                                    ": strided operands are not supported on HIP");
    const std::int64_t k = a->shape.back();
    const std::int64_t n = w->shape[1];
    std::int64_t rows = 1;
    for (std::size_t i = 0; i + 1 < c->shape.size(); ++i) rows *= c->shape[i];
    const int qt = qa.quant_type == QuantType::Int4 ? VM_HIP_QUANT_INT4 : VM_HIP_QUANT_INT8;
    const std::int64_t bs = (qt == VM_HIP_QUANT_INT4 && qa.block_size <= 0) ? 32 : qa.block_size;
    const std::int64_t nblk = bs > 0 ? (k + bs - 1) / bs : 1;
    const std::uint64_t need_scales = static_cast<std::uint64_t>(k > 0 ? nblk : 0) * static_cast<std::uint64_t>(n);
    if (storage_numel(*s) < need_scales)
        throw std::invalid_argument(error_context(Op::QuantizedMatMul, *c, "launch") + ": scales hold " +
                                    std::to_string(storage_numel(*s)) + " values, the kernel reads " +
                                    std::to_string(need_scales));
    const int status = vm_hip_qmm_add_f32(static_cast<const float*>(a->data), static_cast<const std::int8_t*>(w->data),
                                          static_cast<const float*>(s->data), static_cast<const float*>(h->data),
                                          static_cast<float*>(c->data), rows, k, n, qt, qa.block_size,
                                          current_stream());
    if (status != VM_HIP_OK) {
        const std::string last = vm_hip_last_error();
        const char* stage = last.find(" at sync") != std::string::npos ? "sync" : "launch";
        throw_status(status, error_context(Op::QuantizedMatMul, *c, stage));
    }
}

// Add(h, QuantizedMatMul(SiluMul(g, u))) fused by the graph compiler:
// inputs [gate, up, B, scales, addend], outputs [C]; attrs the
// QuantizedMatMul's descriptor.
void quantized_matmul_swiglu_add_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    const auto* g = in[0];
    const auto* u = in[1];
    const auto* w = in[2];
    const auto* s = in[3];
    const auto* h = in[4];
    auto* c = out[0];
    if (!g || !u || !w || !s || !h || !c) throw std::runtime_error("quantized_matmul swiglu hip: null storage");
    const auto& qa = std::get<QuantizedMatMulAttrs>(static_cast<const OpDescriptor*>(attrs)->attrs);
    if (!g->is_contiguous() || !u->is_contiguous() || !w->is_contiguous() || !s->is_contiguous() ||
        !h->is_contiguous() || !c->is_contiguous())
        throw std::invalid_argument(error_context(Op::QuantizedMatMul, *c, "launch") +
                                    ": strided operands are not supported on HIP");
    const std::int64_t k = g->shape.back();
    const std::int64_t n = w->shape[1];
    std::int64_t rows = 1;
    for (std::size_t i = 0; i + 1 < c->shape.size(); ++i) rows *= c->shape[i];
    const int qt = qa.quant_type == QuantType::Int4 ? VM_HIP_QUANT_INT4 : VM_HIP_QUANT_INT8;
    const std::int64_t bs = (qt == VM_HIP_QUANT_INT4 && qa.block_size <= 0) ? 32 : qa.block_size;
    const std::int64_t nblk = bs > 0 ? (k + bs - 1) / bs : 1;
    const std::uint64_t need_scales = static_cast<std::uint64_t>(k > 0 ? nblk : 0) * static_cast<std::uint64_t>(n);
    if (storage_numel(*s) < need_scales)
        throw std::invalid_argument(error_context(Op::QuantizedMatMul, *c, "launch") + ": scales hold " +
                                    std::to_string(storage_numel(*s)) + " values, the kernel reads " +
                                    std::to_string(need_scales));
    const int status = vm_hip_qmm_swiglu_add_f32(
        static_cast<const float*>(g->data), static_cast<const float*>(u->data), static_cast<const std::int8_t*>(w->data),
        static_cast<const float*>(s->data), static_cast<const float*>(h->data), static_cast<float*>(c->data), rows, k, n,
        qt, qa.block_size, current_stream());
    if (status != VM_HIP_OK) {
        const std::string last = vm_hip_last_error();
        const char* stage = last.find(" at sync") != std::string::npos ? "sync" : "launch";
        throw_status(status, error_context(Op::QuantizedMatMul, *c, stage));
    }
}

// Sibling fp32 QuantizedMatMul nodes sharing A, compiled into one step by
// the graph compiler: inputs [A, B_1, S_1, .., B_g, S_g], outputs
// [C_1, .., C_g].  Each member is checked as a single node is; then one
// vm_hip_qmm_group_f32 call (one GEMV launch for rows <= 4).
void quantized_matmul_group_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    const auto& grp = *static_cast<const internal::QmmGroupAttrs*>(attrs);
    const auto& qa = std::get<QuantizedMatMulAttrs>(grp.desc.attrs);
    const auto* a = in[0];
    if (!a || grp.members < 1 || grp.members > VM_HIP_QMM_GROUP_MAX)
        throw std::runtime_error("quantized_matmul group hip: bad group");
    if (!a->is_contiguous())
        throw std::invalid_argument(error_context(Op::QuantizedMatMul, *out[0], "launch") +
                                    ": strided operands are not supported on HIP");
    const std::size_t rank = a->shape.size();
    const std::int64_t k = a->shape[rank - 1];
    std::int64_t rows = 1;
    for (std::size_t i = 0; i + 1 < rank; ++i) rows *= a->shape[i];
    const int qt = qa.quant_type == QuantType::Int4 ? VM_HIP_QUANT_INT4 : VM_HIP_QUANT_INT8;
    const std::int64_t bs = (qt == VM_HIP_QUANT_INT4 && qa.block_size <= 0) ? 32 : qa.block_size;
    const std::int64_t nblk = bs > 0 ? (k + bs - 1) / bs : 1;
    vm_hip_qmm_member members[VM_HIP_QMM_GROUP_MAX];
    for (std::size_t g = 0; g < grp.members; ++g) {
        const auto* w = in[1 + 2 * g];
        const auto* s = in[2 + 2 * g];
        auto* c = out[g];
        if (!w || !s || !c) throw std::runtime_error("quantized_matmul group hip: null storage");
        if (!w->is_contiguous() || !s->is_contiguous() || !c->is_contiguous())
            throw std::invalid_argument(error_context(Op::QuantizedMatMul, *c, "launch") +
                                        ": strided operands are not supported on HIP");
        const std::int64_t n = w->shape[1];
        const std::uint64_t need_scales = static_cast<std::uint64_t>(k > 0 ? nblk : 0) * static_cast<std::uint64_t>(n);
        if (storage_numel(*s) < need_scales)
            throw std::invalid_argument(error_context(Op::QuantizedMatMul, *c, "launch") + ": scales hold " +
                                        std::to_string(storage_numel(*s)) + " values, the kernel reads " +
                                        std::to_string(need_scales));
        members[g] = vm_hip_qmm_member{static_cast<const std::int8_t*>(w->data), static_cast<const float*>(s->data),
                                       static_cast<float*>(c->data), n};
    }
    const int status = vm_hip_qmm_group_f32(static_cast<const float*>(a->data), rows, k, members,
                                            static_cast<int>(grp.members), qt, qa.block_size, current_stream());
    if (status != VM_HIP_OK) {
        const std::string last = vm_hip_last_error();
        const char* stage = last.find(" at sync") != std::string::npos ? "sync" : "launch";
        throw_status(status, error_context(Op::QuantizedMatMul, *out[0], stage));
    }
}

// RMSNorm feeding QuantizedMatMul(s), fused by the graph compiler: inputs
// [x, w, B_1, S_1, .., B_g, S_g], outputs [C_1, .., C_g], attrs a
// NormQmmAttrs.  Each member is checked as a single node is.
void quantized_matmul_norm_group_hip(const pConstTensorStorage* in, const pTensorStorage* out, const void* attrs) {
    const auto& na = *static_cast<const internal::NormQmmAttrs*>(attrs);
    const auto& qa = std::get<QuantizedMatMulAttrs>(na.desc.attrs);
    const auto* x = in[0];
    const auto* nw = in[1];
    if (!x || !nw || na.members < 1 || na.members > VM_HIP_QMM_GROUP_MAX)
        throw std::runtime_error("quantized_matmul norm group hip: bad group");
    if (!x->is_contiguous() || !nw->is_contiguous())
        throw std::invalid_argument(error_context(Op::RMSNorm, *out[0], "launch") +
                                    ": strided operands are not supported on HIP");
    const std::int64_t k = x->shape.back();
    std::int64_t rows = 1;
    for (std::size_t i = 0; i + 1 < x->shape.size(); ++i) rows *= x->shape[i];
    const int qt = qa.quant_type == QuantType::Int4 ? VM_HIP_QUANT_INT4 : VM_HIP_QUANT_INT8;
    const std::int64_t bs = (qt == VM_HIP_QUANT_INT4 && qa.block_size <= 0) ? 32 : qa.block_size;
    const std::int64_t nblk = bs > 0 ? (k + bs - 1) / bs : 1;
    vm_hip_qmm_member members[VM_HIP_QMM_GROUP_MAX];
    for (std::size_t g = 0; g < na.members; ++g) {
        const auto* w = in[2 + 2 * g];
        const auto* s = in[3 + 2 * g];
        auto* c = out[g];
        if (!w || !s || !c) throw std::runtime_error("quantized_matmul norm group hip: null storage");
        if (!w->is_contiguous() || !s->is_contiguous() || !c->is_contiguous())
            throw std::invalid_argument(error_context(Op::QuantizedMatMul, *c, "launch") +
                                        ": strided operands are not supported on HIP");
        const std::int64_t n = w->shape[1];
        const std::uint64_t need_scales = static_cast<std::uint64_t>(k > 0 ? nblk : 0) * static_cast<std::uint64_t>(n);
        if (storage_numel(*s) < need_scales)
            throw std::invalid_argument(error_context(Op::QuantizedMatMul, *c, "launch") + ": scales hold " +
                                        std::to_string(storage_numel(*s)) + " values, the kernel reads " +
                                        std::to_string(need_scales));
        members[g] = vm_hip_qmm_member{static_cast<const std::int8_t*>(w->data), static_cast<const float*>(s->data),
                                       static_cast<float*>(c->data), n};
    }
    const int status = vm_hip_qmm_norm_group_f32(static_cast<const float*>(x->data), static_cast<const float*>(nw->data),
                                                 na.epsilon, rows, k, members, static_cast<int>(na.members), qt,
                                                 qa.block_size, current_stream());
    if (status != VM_HIP_OK) {
        const std::string last = vm_hip_last_error();
        const char* stage = last.find(" at sync") != std::string::npos ? "sync" : "launch";
        throw_status(status, error_context(Op::QuantizedMatMul, *out[0], stage));
    }
}

}  // namespace

VELOMIND_REGISTER_QMM_GROUP(::velomind::DeviceType::HIP, quantized_matmul_group_hip)
VELOMIND_REGISTER_FUSED(::velomind::DeviceType::HIP, ::velomind::internal::FusedKind::NormQmm,
                        &quantized_matmul_norm_group_hip)
VELOMIND_REGISTER_FUSED(::velomind::DeviceType::HIP, ::velomind::internal::FusedKind::SwigluQmmAdd,
                        &quantized_matmul_swiglu_add_hip)
VELOMIND_REGISTER_FUSED(::velomind::DeviceType::HIP, ::velomind::internal::FusedKind::QmmAdd,
                        &quantized_matmul_add_hip)

VELOMIND_REGISTER_QUANTIZED_MATMUL(::velomind::DeviceType::HIP, ::velomind::DataType::Float32,
                                   ::velomind::DataType::Float32, ::velomind::DataType::Float32,
                                   quantized_matmul_hip_impl)
VELOMIND_REGISTER_QUANTIZED_MATMUL(::velomind::DeviceType::HIP, ::velomind::DataType::Float16,
                                   ::velomind::DataType::Float16, ::velomind::DataType::Float16,
                                   quantized_matmul_hip_impl)
VELOMIND_REGISTER_QUANTIZED_MATMUL(::velomind::DeviceType::HIP, ::velomind::DataType::Float16,
                                   ::velomind::DataType::Float32, ::velomind::DataType::Float16,
                                   quantized_matmul_hip_impl)
VELOMIND_REGISTER_QUANTIZED_MATMUL(::velomind::DeviceType::HIP, ::velomind::DataType::BFloat16,
                                   ::velomind::DataType::BFloat16, ::velomind::DataType::BFloat16,
                                   quantized_matmul_hip_impl)
VELOMIND_REGISTER_QUANTIZED_MATMUL(::velomind::DeviceType::HIP, ::velomind::DataType::BFloat16,
                                   ::velomind::DataType::Float32, ::velomind::DataType::BFloat16,
                                   quantized_matmul_hip_impl)

}  // namespace velomind::backend::hip
