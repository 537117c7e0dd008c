// Backend factory (reference include/runtherder/attention/factory.h:9-16).
#pragma once

#include <memory>

#include <runtherder/attention/backend.h>

namespace runtherder::attention {

enum class BackendKind {
    Naive,
    Adaptive,
};

[[nodiscard]] std::unique_ptr<AttentionBackend> make_attention_backend(
    BackendKind kind, const AttnConfig& config);

}  // namespace runtherder::attention
