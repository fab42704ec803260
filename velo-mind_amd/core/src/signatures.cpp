// Signature registrations of the LLaMA-graph operators (device
// independent; the reference registers each next to its CPU kernel, e.g.
// src/cpu/ops/rmsnorm.cpp:82).  QuantizedMatMul's is in kernel.cpp.
#include "internal/registry/shape.h"
#include "internal/shape_helpers.h"

namespace vi = ::velomind::internal;

VELOMIND_REGISTER_SIGNATURE(::velomind::Op::Add, vi::signature_elementwise)
VELOMIND_REGISTER_SIGNATURE(::velomind::Op::Mul, vi::signature_elementwise)
VELOMIND_REGISTER_SIGNATURE(::velomind::Op::Sigmoid, vi::signature_elementwise)
VELOMIND_REGISTER_SIGNATURE(::velomind::Op::Softmax, vi::signature_softmax)
VELOMIND_REGISTER_SIGNATURE(::velomind::Op::MatMul, vi::signature_matmul)
VELOMIND_REGISTER_SIGNATURE(::velomind::Op::RMSNorm, vi::signature_same_as_input)
VELOMIND_REGISTER_SIGNATURE(::velomind::Op::RotaryEmbedding, vi::signature_same_as_input)
VELOMIND_REGISTER_SIGNATURE(::velomind::Op::Embedding, vi::signature_embedding)
VELOMIND_REGISTER_SIGNATURE(::velomind::Op::Reshape, vi::signature_reshape)
VELOMIND_REGISTER_SIGNATURE(::velomind::Op::Transpose, vi::signature_transpose)
VELOMIND_REGISTER_SIGNATURE(::velomind::Op::Concat, vi::signature_concat)
VELOMIND_REGISTER_SIGNATURE(::velomind::Op::RepeatKV, vi::signature_repeat_kv)
VELOMIND_REGISTER_SIGNATURE(::velomind::Op::Slice, vi::signature_slice)
VELOMIND_REGISTER_SIGNATURE(::velomind::Op::FusedAttention, vi::signature_fused_attention)
