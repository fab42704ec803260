// Registers the oracle as the CPU QuantizedMatMul kernel of the test binary.
#include "test_helpers.h"

#include <cstring>
#include <variant>

#include "internal/registry/kernel.h"

namespace {

void oracle_qmm_cpu(const velomind::pConstTensorStorage* in, const velomind::pTensorStorage* out, const void* attrs) {
    const auto& desc = *static_cast<const velomind::OpDescriptor*>(attrs);
    const auto& qa = std::get<velomind::QuantizedMatMulAttrs>(desc.attrs);
    const auto& a = *in[0];
    const std::size_t k = static_cast<std::size_t>(a.shape.back());
    const std::size_t n = static_cast<std::size_t>(in[1]->shape[1]);
    std::size_t rows = 1;
    for (std::size_t i = 0; i + 1 < a.shape.size(); ++i) rows *= static_cast<std::size_t>(a.shape[i]);
    vmo_qmm_2d_f32(static_cast<const float*>(a.data), static_cast<const std::int8_t*>(in[1]->data),
                   static_cast<const float*>(in[2]->data), static_cast<float*>(out[0]->data), rows, k, n,
                   static_cast<int>(qa.quant_type), qa.block_size);
}

// Reshape on the host: a byte copy into the output's shape.
void copy_reshape_cpu(const velomind::pConstTensorStorage* in, const velomind::pTensorStorage* out, const void*) {
    std::memcpy(out[0]->data, in[0]->data, in[0]->size_bytes);
}

}  // namespace

VELOMIND_REGISTER_OP_KERNEL(::velomind::DeviceType::CPU, ::velomind::Op::Reshape,
                            (::velomind::internal::KernelDtypeKey{{::velomind::DataType::Float32}, 1,
                                                                  ::velomind::DataType::Float32}),
                            &copy_reshape_cpu)

VELOMIND_REGISTER_OP_KERNEL(::velomind::DeviceType::CPU, ::velomind::Op::QuantizedMatMul,
                            (::velomind::internal::KernelDtypeKey{
                                {::velomind::DataType::Float32, ::velomind::DataType::Int8, ::velomind::DataType::Float32},
                                3, ::velomind::DataType::Float32}),
                            &oracle_qmm_cpu)

VMT_MAIN()
