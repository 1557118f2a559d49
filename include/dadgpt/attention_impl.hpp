// The reference's attention implementation choice (src/model.hpp:81), for callers that do not
// include the reference's model.hpp (which defines the same enum: include one or the other).
// The enumerators and their order are the reference's; use_fused_attention in
// <dadgpt/gpu_ops_attention.hpp> takes it.
#pragma once

enum class AttentionImpl { Auto, Fused, Materialized };
