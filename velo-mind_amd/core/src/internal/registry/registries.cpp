// Storage of all static registries.  Function-local statics make them
// available to registrations that run during static initialisation of any
// translation unit.
#include <cstdio>
#include <stdexcept>
#include <string>

#include "internal/log.h"
#include "internal/registry/device_context.h"
#include "internal/registry/kernel.h"
#include "internal/registry/memory_transfer.h"
#include "internal/registry/shape.h"
#include "internal/registry/storage.h"

namespace velomind::internal {

// ---- kernels --------------------------------------------------------------

auto operator==(const KernelDtypeKey& a, const KernelDtypeKey& b) noexcept -> bool {
    if (a.num_inputs != b.num_inputs || a.output_dtype != b.output_dtype) return false;
    for (std::size_t i = 0; i < a.num_inputs; ++i)
        if (a.input_dtypes[i] != b.input_dtypes[i]) return false;
    return true;
}

auto op_kernels(DeviceType device) -> std::array<std::vector<KernelEntry>, MAX_OPS>& {
    static std::array<std::vector<KernelEntry>, MAX_OPS> tables[MAX_DEVICE_TYPES];
    const auto idx = static_cast<std::size_t>(device);
    if (idx >= MAX_DEVICE_TYPES)
        throw std::out_of_range("op_kernels: device index exceeds MAX_DEVICE_TYPES");
    return tables[idx];
}

auto register_op_kernel(DeviceType device, Op op, KernelDtypeKey key, Executable::KernelFn fn) -> void {
    op_kernels(device)[static_cast<std::size_t>(op)].push_back({key, fn});
}

auto resolve_op_kernel(Op op, std::span<const DataType> input_dtypes, DataType output_dtype, DeviceType device)
    -> Executable::KernelFn {
    if (input_dtypes.size() > 4 || static_cast<std::size_t>(op) >= MAX_OPS) return nullptr;
    if (static_cast<std::size_t>(device) >= MAX_DEVICE_TYPES) return nullptr;
    KernelDtypeKey key;
    key.num_inputs = input_dtypes.size();
    key.output_dtype = output_dtype;
    for (std::size_t i = 0; i < input_dtypes.size(); ++i) key.input_dtypes[i] = input_dtypes[i];
    for (const auto& e : op_kernels(device)[static_cast<std::size_t>(op)])
        if (e.key == key) return e.fn;
    return nullptr;
}

namespace {
auto qmm_group_table() -> std::array<Executable::KernelFn, MAX_DEVICE_TYPES>& {
    static std::array<Executable::KernelFn, MAX_DEVICE_TYPES> table{};
    return table;
}
}  // namespace

auto register_qmm_group_kernel(DeviceType device, Executable::KernelFn fn) -> void {
    const auto idx = static_cast<std::size_t>(device);
    if (idx >= MAX_DEVICE_TYPES) throw std::out_of_range("register_qmm_group_kernel: device index out of range");
    qmm_group_table()[idx] = fn;
}

auto qmm_group_kernel(DeviceType device) -> Executable::KernelFn {
    const auto idx = static_cast<std::size_t>(device);
    return idx < MAX_DEVICE_TYPES ? qmm_group_table()[idx] : nullptr;
}

namespace {
auto fused_table() -> std::array<std::array<Executable::KernelFn, kFusedKinds>, MAX_DEVICE_TYPES>& {
    static std::array<std::array<Executable::KernelFn, kFusedKinds>, MAX_DEVICE_TYPES> table{};
    return table;
}
}  // namespace

auto register_fused_kernel(DeviceType device, FusedKind kind, Executable::KernelFn fn) -> void {
    const auto idx = static_cast<std::size_t>(device);
    const auto k = static_cast<std::size_t>(kind);
    if (idx >= MAX_DEVICE_TYPES || k >= kFusedKinds)
        throw std::out_of_range("register_fused_kernel: device or kind out of range");
    fused_table()[idx][k] = fn;
}

auto fused_kernel(DeviceType device, FusedKind kind) -> Executable::KernelFn {
    const auto idx = static_cast<std::size_t>(device);
    const auto k = static_cast<std::size_t>(kind);
    return (idx < MAX_DEVICE_TYPES && k < kFusedKinds) ? fused_table()[idx][k] : nullptr;
}

// ---- signatures and default attributes -----------------------------------

auto signatures() -> std::array<OpSignatureFn, MAX_OPS>& {
    static std::array<OpSignatureFn, MAX_OPS> table{};
    return table;
}

void register_op_signature(Op op, OpSignatureFn fn) { signatures()[static_cast<std::size_t>(op)] = fn; }

auto get_op_signature(Op op) -> OpSignatureFn {
    const auto idx = static_cast<std::size_t>(op);
    return idx < MAX_OPS ? signatures()[idx] : nullptr;
}

auto default_attrs_table() -> std::array<OpAttrs, MAX_OPS>& {
    static std::array<OpAttrs, MAX_OPS> table = [] {
        std::array<OpAttrs, MAX_OPS> t{};  // NoAttrs everywhere by default
        t[static_cast<std::size_t>(Op::Softmax)] = SoftmaxAttrs{};
        t[static_cast<std::size_t>(Op::MatMul)] = MatMulAttrs{};
        t[static_cast<std::size_t>(Op::ReduceSum)] = ReduceAttrs{};
        t[static_cast<std::size_t>(Op::ReduceMean)] = ReduceAttrs{};
        t[static_cast<std::size_t>(Op::Conv2D)] = Conv2DAttrs{};
        t[static_cast<std::size_t>(Op::Reshape)] = ReshapeAttrs{};
        t[static_cast<std::size_t>(Op::Transpose)] = TransposeAttrs{};
        t[static_cast<std::size_t>(Op::Concat)] = ConcatAttrs{};
        t[static_cast<std::size_t>(Op::Slice)] = SliceAttrs{};
        t[static_cast<std::size_t>(Op::RMSNorm)] = RMSNormAttrs{};
        t[static_cast<std::size_t>(Op::RepeatKV)] = RepeatKVAttrs{};
        t[static_cast<std::size_t>(Op::FusedAttention)] = FusedAttentionAttrs{};
        t[static_cast<std::size_t>(Op::QuantizedMatMul)] = QuantizedMatMulAttrs{};
        return t;
    }();
    return table;
}

void register_default_op_attrs(Op op, OpAttrs attrs) {
    const auto idx = static_cast<std::size_t>(op);
    if (idx < MAX_OPS) default_attrs_table()[idx] = std::move(attrs);
}

// ---- storage ----------------------------------------------------------------

auto storage_creaters() -> std::array<StorageCreatorFn, MAX_DEVICE_TYPES>& {
    static std::array<StorageCreatorFn, MAX_DEVICE_TYPES> table{};
    return table;
}

namespace {
auto availability_table() -> std::array<DeviceAvailabilityFn, MAX_DEVICE_TYPES>& {
    static std::array<DeviceAvailabilityFn, MAX_DEVICE_TYPES> table{};
    return table;
}
}  // namespace

auto register_storage_creator(DeviceType device, StorageCreatorFn fn) -> void {
    const auto idx = static_cast<std::size_t>(device);
    if (idx >= MAX_DEVICE_TYPES) return;
    if (storage_creaters()[idx] != nullptr)
        VELOMIND_LOG(Warn, std::string("storage allocator for device ") + device_type_name(device) + " replaced");
    storage_creaters()[idx] = fn;
}

auto get_storage_creator(DeviceType device) -> StorageCreatorFn {
    const auto idx = static_cast<std::size_t>(device);
    return idx < MAX_DEVICE_TYPES ? storage_creaters()[idx] : nullptr;
}

auto register_device_availability(DeviceType device, DeviceAvailabilityFn fn) -> void {
    const auto idx = static_cast<std::size_t>(device);
    if (idx < MAX_DEVICE_TYPES) availability_table()[idx] = fn;
}

auto is_device_available(DeviceType device) noexcept -> bool {
    const auto idx = static_cast<std::size_t>(device);
    if (idx >= MAX_DEVICE_TYPES) return false;
    if (auto fn = availability_table()[idx]) return fn();
    return storage_creaters()[idx] != nullptr;
}

auto create_tensor_storage(std::size_t bytes, DeviceType device) -> std::shared_ptr<TensorStorage> {
    auto fn = get_storage_creator(device);
    return fn ? fn(bytes) : nullptr;
}

// ---- memory transfer -------------------------------------------------------

auto memory_transfers() -> std::array<MemoryTransfer, MAX_DEVICE_TYPES>& {
    static std::array<MemoryTransfer, MAX_DEVICE_TYPES> table{};
    return table;
}

void register_memory_transfer(DeviceType device, MemoryTransfer t) {
    const auto idx = static_cast<std::size_t>(device);
    if (idx >= MAX_DEVICE_TYPES) return;
    if (memory_transfers()[idx].copy_h2d && t.copy_h2d)
        VELOMIND_LOG(Warn, std::string("memory transfer for device ") + device_type_name(device) + " replaced");
    memory_transfers()[idx] = t;
}

auto get_memory_transfer(DeviceType device) -> MemoryTransfer {
    const auto idx = static_cast<std::size_t>(device);
    return idx < MAX_DEVICE_TYPES ? memory_transfers()[idx] : MemoryTransfer{};
}

// ---- device contexts ---------------------------------------------------------

namespace {
auto context_table() -> std::array<DeviceContextHooks, MAX_DEVICE_TYPES>& {
    static std::array<DeviceContextHooks, MAX_DEVICE_TYPES> table{};
    return table;
}
}  // namespace

void register_device_context_hooks(DeviceType device, DeviceContextHooks hooks) {
    const auto idx = static_cast<std::size_t>(device);
    if (idx < MAX_DEVICE_TYPES) context_table()[idx] = hooks;
}

auto get_device_context_hooks(DeviceType device) -> DeviceContextHooks {
    const auto idx = static_cast<std::size_t>(device);
    return idx < MAX_DEVICE_TYPES ? context_table()[idx] : DeviceContextHooks{};
}

ScopedDeviceContext::ScopedDeviceContext(DeviceType device, void* ctx) : _hooks(get_device_context_hooks(device)) {
    if (ctx && _hooks.activate) {
        _previous = _hooks.activate(ctx);
        _active = true;
    }
}

ScopedDeviceContext::~ScopedDeviceContext() {
    if (_active && _hooks.deactivate) _hooks.deactivate(_previous);
}

// ---- logging -----------------------------------------------------------------

namespace {
void default_log_handler(LogLevel level, const std::string& message) {
    static const char* names[] = {"debug", "info", "warn", "error"};
    std::fprintf(stderr, "[velomind %s] %s\n", names[static_cast<int>(level)], message.c_str());
}
LogHandler g_log_handler = &default_log_handler;
}  // namespace

void set_log_handler(LogHandler handler) { g_log_handler = handler ? handler : &default_log_handler; }
void log_message(LogLevel level, const std::string& message) { g_log_handler(level, message); }

}  // namespace velomind::internal

namespace velomind {

auto default_op_attrs(Op op) -> OpAttrs {
    const auto idx = static_cast<std::size_t>(op);
    return idx < MAX_OPS ? internal::default_attrs_table()[idx] : OpAttrs{NoAttrs{}};
}

}  // namespace velomind
