// One operator node of a Graph: its descriptor and the storages it reads
// and writes.
#pragma once

#include <span>
#include <vector>

#include "velomind/inline_list.h"
#include "velomind/ops.h"
#include "velomind/tensor_storage.h"
#include "velomind_core_export.h"

namespace velomind {

class Graph;
namespace internal {
class GraphCompiler;
}

class VELOMIND_CORE_EXPORT Node {
public:
    Node() = default;
    auto op() const -> const OpDescriptor& { return _op; }
    auto inputs() const -> std::span<const pConstTensorStorage> { return {_inputs.data(), _inputs.size()}; }
    auto outputs() const -> std::span<const pTensorStorage> { return {_outputs.data(), _outputs.size()}; }

private:
    friend class Graph;
    friend struct GraphTestAccess;
    friend class internal::GraphCompiler;

    OpDescriptor _op;
    InlineList<pConstTensorStorage, 4> _inputs;
    InlineList<pTensorStorage, 1> _outputs;
};

VELOMIND_EXPORT_PTR(Node);

}  // namespace velomind
