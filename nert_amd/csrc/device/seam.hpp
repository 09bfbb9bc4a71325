#pragma once
// Shared pieces of the gfx950 HipDevice rows.
//
// Each row validates its node and views on the host exactly as the reference
// CPU row does (same checks, same order, same "<Op> (node '<name>'): ..."
// messages), then queues its kernels on the layer stream and returns without
// synchronising. Rows whose behaviour depends on small int64/float control
// operands (shapes, axes, K, scales) read them from the transfer's host
// shadow when the bytes were uploaded through the seam, and fall back to a
// blocking device-to-host read otherwise.

#include "nert/device.hpp"
#include "nert/graph.hpp"
#include "../../../include/nert_hip.h"

#include <cstdint>
#include <string>
#include <vector>

namespace nert_hip {
namespace seam {

using nert::Attribute;
using nert::DataType;
using nert::InferenceException;
using nert::Node;
using nert::TensorView;
using Views = std::vector<TensorView>;

// The reference's per-row ElementCount: every dim must be positive.
inline int64_t ElementCount(const std::vector<int64_t>& dims, const std::string& context) {
    int64_t count = 1;
    for (int64_t dim : dims) {
        if (dim <= 0) {
            throw InferenceException(context + ": non-positive dimension");
        }
        count *= dim;
    }
    return count;
}

// The other per-row ElementCount of the reference: zero dims allowed,
// negative ones rejected.
inline int64_t CountNonNeg(const std::vector<int64_t>& dims, const std::string& context) {
    int64_t count = 1;
    for (int64_t dim : dims) {
        if (dim < 0) {
            throw InferenceException(context + ": negative dimension");
        }
        count *= dim;
    }
    return count;
}

// Element count without validation (zero dims allowed).
inline int64_t Count(const std::vector<int64_t>& dims) {
    int64_t count = 1;
    for (int64_t dim : dims) {
        count *= dim;
    }
    return count;
}

inline int64_t ElementSize(DataType dtype) {
    switch (dtype) {
    case DataType::Float32:
        return 4;
    case DataType::Int64:
        return 8;
    case DataType::Bool:
        return 1;
    default:
        return 0;
    }
}

inline int DtypeCode(DataType dtype) {
    switch (dtype) {
    case DataType::Float32:
        return NERT_F32;
    case DataType::Int64:
        return NERT_I64;
    case DataType::Bool:
        return NERT_BOOL;
    default:
        return NERT_UNKNOWN;
    }
}

inline std::vector<int64_t> Strides(const std::vector<int64_t>& dims) {
    std::vector<int64_t> strides(dims.size(), 1);
    for (size_t i = dims.size(); i-- > 1;) {
        strides[i - 1] = strides[i] * dims[i];
    }
    return strides;
}

inline const Attribute* FindAttr(const Node& node, const std::string& name) {
    for (const Attribute& attr : node.attributes) {
        if (attr.name == name) {
            return &attr;
        }
    }
    return nullptr;
}

// Attribute readers. `op` names the row in the message, matching the
// reference's "<Op>: attribute '<name>' must be ... (node '<n>')" form.
int64_t IntAttr(const Node& node, const std::string& name, int64_t fallback, const char* op);
float FloatAttr(const Node& node, const std::string& name, float fallback, const char* op);
std::string StringAttr(const Node& node, const std::string& name, const std::string& fallback, const char* op);
std::vector<int64_t> IntsAttr(const Node& node, const std::string& name, const char* op);
// Same readers with the other message form the reference rows use:
// "<context>: attribute '<name>' must be an integer".
int64_t IntAttrC(const Node& node, const std::string& name, int64_t fallback, const std::string& context);
float FloatAttrC(const Node& node, const std::string& name, float fallback, const std::string& context);

// Throws when the layer reported a HIP failure.
void CheckStatus(int status, const std::string& context);

// Host copies of small control tensors (see file comment).
std::vector<int64_t> ReadInt64(const TensorView& view, int64_t count, const std::string& context);
std::vector<float> ReadFloat(const TensorView& view, int64_t count, const std::string& context);

// Host shadow only (no device read): true and `out` filled when the
// view's bytes are shadowed.
bool HostShadowInt64(const TensorView& view, int64_t count, std::vector<int64_t>& out);
// Records `bytes` at `device_ptr` as the host view of a value a queued kernel
// writes there (rows whose outputs are known on the host, e.g. Shape).
void PutHostShadow(void* device_ptr, const void* host, int64_t bytes);

// Must be called by every row after queuing writes to `outputs`: drops host
// shadows the writes made stale and, in the debug mode (NERT_HIP_SYNC=1),
// synchronises so a device fault is attributed to this row.
void AfterRow(const Views& outputs, const std::string& context);

// Synchronises and throws `message` when the row's kernels raised a device
// error flag (data-dependent failures the host could not check first).
void ThrowOnDeviceFlag(const std::string& context, const std::string& message);

// The layer stream every row launches on.
void* Stream();

} // namespace seam

// Row lookup by op type (null when the op has no row): the reference's 73
// op types, what the seam's KernelTable::find answers.
nert::KernelFn FindRow(const std::string& op_type);
// FindRow plus the runner's fused rows (FusedConv, FusedMatMul,
// FusedAddLayerNorm, FusedAttention), for the node-level C entry points.
nert::KernelFn FindRunnerRow(const std::string& op_type);

} // namespace nert_hip
