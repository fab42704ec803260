// Graph -> Executable compilation (memory planning, allocation, kernel
// resolution).
#pragma once

#include <memory>

#include "velomind/executable.h"
#include "velomind/graph.h"

namespace velomind::internal {

class GraphCompiler {
public:
    // Validates, orders, plans one arena for intermediates, allocates on
    // `device` and resolves kernels.  On failure the graph is unchanged and
    // may be built again.
    static auto compile(Graph& graph, DeviceType device) -> std::unique_ptr<Executable>;
};

// Bytes between arena slots (the reference's graph_compiler.cpp:97).
inline constexpr std::size_t kArenaAlignment = 256;

}  // namespace velomind::internal
