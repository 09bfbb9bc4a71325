// Movement rows: Transpose, Concat, Split, Slice, Expand, Tile, Squeeze,
// Unsqueeze, Pad. Validation mirrors src/kernels/{transpose,concat,split,
// slice,expand,tile,squeeze,unsqueeze,pad}.cpp; the data moves through
// nert_hip_copy_strided (one kernel, per-axis strides) or nert_hip_pad.

#include "rows.hpp"

#include "axes_form.hpp"

#include <algorithm>

namespace nert_hip {
namespace rows {

using namespace seam;

namespace {

bool MovableDtype(DataType d) { return d == DataType::Float32 || d == DataType::Int64 || d == DataType::Bool; }

// Copies a [dims] box: src element (c) at src + sum c_d * ss_d, dst likewise.
void CopyBox(const TensorView& like, const void* src, void* dst, const std::vector<int64_t>& dims,
             const std::vector<int64_t>& ss, const std::vector<int64_t>& ds, const std::string& context,
             const std::vector<int64_t>* mods = nullptr) {
    CheckStatus(nert_hip_copy_strided(static_cast<int>(ElementSize(like.dtype)), src, dst, static_cast<int>(dims.size()),
                                      dims.data(), ss.data(), ds.data(), mods != nullptr ? mods->data() : nullptr,
                                      Stream()),
                context);
}

void CopyAll(const TensorView& in, const TensorView& out, const std::string& context) {
    const int64_t bytes = Count(in.dims) * ElementSize(in.dtype);
    if (bytes > 0 && in.data != out.data) {
        CheckStatus(nert_hip_memcpy_d2d(out.data, in.data, bytes, Stream()), context);
    }
}

const uint8_t* Bytes(const void* p) { return static_cast<const uint8_t*>(p); }
uint8_t* Bytes(void* p) { return static_cast<uint8_t*>(p); }

} // namespace

// src/kernels/transpose.cpp:54-126
NERT_HIP_ROW(Transpose) {
    const std::string context = "Transpose (node '" + node.name + "')";
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (!MovableDtype(in.dtype)) {
        throw InferenceException(context + ": tensors must be float32, int64, or bool");
    }
    if (out.dtype != in.dtype) {
        throw InferenceException(context + ": output dtype must match the input dtype");
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    std::vector<int64_t> perm;
    bool have_perm = false;
    for (const Attribute& attr : node.attributes) {
        if (attr.name == "perm") {
            const std::vector<int64_t>* value = std::get_if<std::vector<int64_t>>(&attr.value);
            if (value == nullptr) {
                throw InferenceException(context + ": attribute 'perm' must be an int list");
            }
            perm = *value;
            have_perm = true;
        }
    }
    if (!have_perm) {
        for (int64_t i = 0; i < rank; ++i) {
            perm.push_back(rank - 1 - i);
        }
    }
    if (static_cast<int64_t>(perm.size()) != rank) {
        throw InferenceException(context + ": Transpose perm rank must match the input rank");
    }
    std::vector<int64_t> sorted = perm;
    std::sort(sorted.begin(), sorted.end());
    for (int64_t i = 0; i < rank; ++i) {
        if (sorted[static_cast<size_t>(i)] != i) {
            throw InferenceException(context + ": Transpose perm must be a permutation");
        }
    }
    std::vector<int64_t> expected(static_cast<size_t>(rank), 0);
    for (int64_t i = 0; i < rank; ++i) {
        expected[static_cast<size_t>(i)] = in.dims[static_cast<size_t>(perm[static_cast<size_t>(i)])];
    }
    if (out.dims != expected) {
        throw InferenceException(context + ": output shape does not match the transposed input");
    }
    const int64_t count = CountNonNeg(out.dims, context);
    (void)CountNonNeg(in.dims, context);
    if (count > 0 && (in.data == nullptr || out.data == nullptr)) {
        throw InferenceException(context + ": null buffer");
    }
    const std::vector<int64_t> in_strides = Strides(in.dims);
    std::vector<int64_t> ss(static_cast<size_t>(rank));
    for (int64_t i = 0; i < rank; ++i) {
        ss[static_cast<size_t>(i)] = in_strides[static_cast<size_t>(perm[static_cast<size_t>(i)])];
    }
    CopyBox(in, in.data, out.data, out.dims, ss, Strides(out.dims), context);
    AfterRow(outputs, context);
}

// src/kernels/concat.cpp:64-143
NERT_HIP_ROW(Concat) {
    const std::string context = "Concat (node '" + node.name + "')";
    if (inputs.empty() || outputs.size() != 1) {
        throw InferenceException(context + ": expected at least one input and one output");
    }
    const TensorView& first = inputs[0];
    if (!MovableDtype(first.dtype)) {
        throw InferenceException(context + ": tensors must be float32, int64, or bool");
    }
    const TensorView& out = outputs[0];
    if (out.dtype != first.dtype) {
        throw InferenceException(context + ": output dtype must match the input dtype");
    }
    const int64_t rank = static_cast<int64_t>(first.dims.size());
    if (rank == 0) {
        throw InferenceException(context + ": Concat axis is out of range");
    }
    int64_t axis = IntAttrC(node, "axis", 1, context);
    if (axis < -rank || axis >= rank) {
        throw InferenceException(context + ": Concat axis is out of range");
    }
    if (axis < 0) {
        axis += rank;
    }
    std::vector<int64_t> expected = first.dims;
    for (const TensorView& view : inputs) {
        if (view.dtype != first.dtype) {
            throw InferenceException(context + ": all inputs must share the element type");
        }
        if (static_cast<int64_t>(view.dims.size()) != rank) {
            throw InferenceException(context + ": Concat inputs must share rank");
        }
        for (int64_t j = 0; j < rank; ++j) {
            if (j != axis && view.dims[static_cast<size_t>(j)] != expected[static_cast<size_t>(j)]) {
                throw InferenceException(context + ": Concat inputs differ off the concat axis");
            }
        }
        expected[static_cast<size_t>(axis)] += view.dims[static_cast<size_t>(axis)];
    }
    expected[static_cast<size_t>(axis)] -= first.dims[static_cast<size_t>(axis)];
    if (out.dims != expected) {
        throw InferenceException(context + ": output shape does not match the concatenated inputs");
    }
    for (const TensorView& view : inputs) {
        if (CountNonNeg(view.dims, context) > 0 && view.data == nullptr) {
            throw InferenceException(context + ": null input buffer");
        }
    }
    const int64_t out_count = CountNonNeg(out.dims, context);
    if (out_count > 0 && out.data == nullptr) {
        throw InferenceException(context + ": null output buffer");
    }
    int64_t outer = 1;
    for (int64_t i = 0; i < axis; ++i) {
        outer *= expected[static_cast<size_t>(i)];
    }
    int64_t inner = 1;
    for (int64_t i = axis + 1; i < rank; ++i) {
        inner *= expected[static_cast<size_t>(i)];
    }
    const int64_t out_extent = expected[static_cast<size_t>(axis)];
    const int64_t esize = ElementSize(first.dtype);
    if (inputs.size() <= 8) {
        // One launch: output row r (of `outer`) is the inputs' rows r in order.
        std::vector<const void*> srcs;
        std::vector<int64_t> row_bytes;
        for (const TensorView& view : inputs) {
            srcs.push_back(view.data);
            row_bytes.push_back(view.dims[static_cast<size_t>(axis)] * inner * esize);
        }
        CheckStatus(nert_hip_concat_rows(static_cast<int>(inputs.size()), srcs.data(), row_bytes.data(), out.data,
                                         outer, Stream()),
                    context);
        AfterRow(outputs, context);
        return;
    }
    int64_t offset = 0;
    for (const TensorView& view : inputs) {
        const int64_t d = view.dims[static_cast<size_t>(axis)];
        CopyBox(first, view.data, Bytes(out.data) + offset * inner * esize, {outer, d * inner}, {d * inner, 1},
                {out_extent * inner, 1}, context);
        offset += d;
    }
    AfterRow(outputs, context);
}

// src/kernels/split.cpp:63-164 (sizes via src/axes_form.hpp)
NERT_HIP_ROW(Split) {
    const std::string context = "Split (node '" + node.name + "')";
    if (inputs.empty() || inputs.size() > 2 || outputs.empty()) {
        throw InferenceException(context + ": expected one or two inputs and at least one output");
    }
    const TensorView& in = inputs[0];
    if (in.dtype != DataType::Float32 && in.dtype != DataType::Int64) {
        throw InferenceException(context + ": tensors must be float32 or int64");
    }
    for (const TensorView& view : outputs) {
        if (view.dtype != in.dtype) {
            throw InferenceException(context + ": output dtype must match the input dtype");
        }
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    if (rank == 0) {
        throw InferenceException(context + ": Split axis is out of range");
    }
    int64_t axis = IntAttrC(node, "axis", 0, context);
    if (axis < -rank || axis >= rank) {
        throw InferenceException(context + ": Split axis is out of range");
    }
    if (axis < 0) {
        axis += rank;
    }
    const int64_t dim = in.dims[static_cast<size_t>(axis)];
    std::vector<int64_t> parts;
    bool parts_supplied = false;
    const nert::SplitForm form = nert::ResolveSplitForm(node);
    if (form.source == nert::AxesSource::Attribute) {
        if (form.split_attribute != nullptr) {
            const std::vector<int64_t>* values = nert::NodeAttributeIntList(form.split_attribute);
            if (values == nullptr) {
                throw InferenceException(context + ": attribute 'split' must be an integer list");
            }
            parts = *values;
            parts_supplied = true;
        }
    } else if (inputs.size() == 2 && inputs[1].dtype != DataType::Unknown) {
        const TensorView& sizes = inputs[1];
        if (sizes.dtype != DataType::Int64) {
            throw InferenceException(context + ": split sizes must be int64");
        }
        const int64_t count = CountNonNeg(sizes.dims, context);
        if (count > 0 && sizes.data == nullptr) {
            throw InferenceException(context + ": null split-sizes buffer");
        }
        parts = ReadInt64(sizes, count, context);
        parts_supplied = true;
    }
    const auto default_parts = nert::DefaultSplitParts(node, dim, outputs.size(), parts_supplied, context);
    if (parts_supplied) {
        if (parts.size() != outputs.size()) {
            throw InferenceException(context + ": Split split sizes must match the output count");
        }
        int64_t sum = 0;
        for (const int64_t v : parts) {
            if (v < 0) {
                throw InferenceException(context + ": Split split sizes must be non-negative");
            }
            sum += v;
        }
        if (sum != dim) {
            throw InferenceException(context + ": Split split sizes must sum to the axis dim");
        }
    } else {
        parts = default_parts;
    }
    for (size_t i = 0; i < outputs.size(); ++i) {
        std::vector<int64_t> want = in.dims;
        want[static_cast<size_t>(axis)] = parts[i];
        if (outputs[i].dims != want) {
            throw InferenceException(context + ": output shape does not match the split sizes");
        }
        if (CountNonNeg(outputs[i].dims, context) > 0 && outputs[i].data == nullptr) {
            throw InferenceException(context + ": null output buffer");
        }
    }
    if (CountNonNeg(in.dims, context) > 0 && in.data == nullptr) {
        throw InferenceException(context + ": null input buffer");
    }
    int64_t outer = 1;
    for (int64_t i = 0; i < axis; ++i) {
        outer *= in.dims[static_cast<size_t>(i)];
    }
    int64_t inner = 1;
    for (int64_t i = axis + 1; i < rank; ++i) {
        inner *= in.dims[static_cast<size_t>(i)];
    }
    const int64_t esize = ElementSize(in.dtype);
    int64_t offset = 0;
    for (size_t i = 0; i < outputs.size(); ++i) {
        const int64_t d = parts[i];
        CopyBox(in, Bytes(in.data) + offset * inner * esize, outputs[i].data, {outer, d * inner}, {dim * inner, 1},
                {d * inner, 1}, context);
        offset += d;
    }
    AfterRow(outputs, context);
}

// src/kernels/slice.cpp:72-176
NERT_HIP_ROW(Slice) {
    const std::string context = "Slice (node '" + node.name + "')";
    if (inputs.size() < 3 || inputs.size() > 5 || outputs.size() != 1) {
        throw InferenceException(context + ": expected data, starts, ends, and optional axes/steps inputs");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (!MovableDtype(in.dtype)) {
        throw InferenceException(context + ": tensors must be float32, int64, or bool");
    }
    if (out.dtype != in.dtype) {
        throw InferenceException(context + ": output dtype must match the input dtype");
    }
    auto read = [&](const TensorView& view, const char* what) {
        if (view.dtype != DataType::Int64) {
            throw InferenceException(context + ": Slice " + what + " must be int64");
        }
        int64_t count = 1;
        for (int64_t d : view.dims) {
            if (d < 0) {
                throw InferenceException(context + ": negative dimension");
            }
            count *= d;
        }
        if (count > 0 && view.data == nullptr) {
            throw InferenceException(context + ": null " + std::string(what) + " buffer");
        }
        return ReadInt64(view, count, context);
    };
    const std::vector<int64_t> starts = read(inputs[1], "starts");
    const std::vector<int64_t> ends = read(inputs[2], "ends");
    if (starts.size() != ends.size()) {
        throw InferenceException(context + ": Slice starts and ends must have the same length");
    }
    const size_t count = starts.size();
    std::vector<int64_t> axes(count, 0);
    for (size_t i = 0; i < count; ++i) {
        axes[i] = static_cast<int64_t>(i);
    }
    if (inputs.size() > 3 && inputs[3].dtype != DataType::Unknown) {
        axes = read(inputs[3], "axes");
        if (axes.size() != count) {
            throw InferenceException(context + ": Slice axes must match starts in length");
        }
    }
    std::vector<int64_t> steps(count, 1);
    if (inputs.size() > 4 && inputs[4].dtype != DataType::Unknown) {
        steps = read(inputs[4], "steps");
        if (steps.size() != count) {
            throw InferenceException(context + ": Slice steps must match starts in length");
        }
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    std::vector<int64_t> begins(static_cast<size_t>(rank), 0);
    std::vector<int64_t> step_of(static_cast<size_t>(rank), 1);
    std::vector<int64_t> expected = in.dims;
    for (size_t i = 0; i < count; ++i) {
        const int64_t step = steps[i];
        if (step == 0) {
            throw InferenceException(context + ": Slice steps must be non-zero");
        }
        int64_t axis = axes[i];
        if (axis < -rank || axis >= rank) {
            throw InferenceException(context + ": Slice axis is out of range");
        }
        if (axis < 0) {
            axis += rank;
        }
        const size_t ua = static_cast<size_t>(axis);
        const int64_t dim = in.dims[ua];
        int64_t begin = starts[i];
        int64_t end = ends[i];
        if (begin < 0) {
            begin += dim;
        }
        if (end < 0) {
            end += dim;
        }
        if (step > 0) {
            begin = std::max<int64_t>(0, std::min(begin, dim));
            end = std::max<int64_t>(0, std::min(end, dim));
            expected[ua] = end > begin ? (end - begin + step - 1) / step : 0;
        } else {
            begin = std::max<int64_t>(0, std::min(begin, dim - 1));
            end = std::max<int64_t>(-1, std::min(end, dim - 1));
            expected[ua] = dim > 0 && begin > end ? (begin - end - step - 1) / -step : 0;
        }
        begins[ua] = begin;
        step_of[ua] = step;
    }
    if (out.dims != expected) {
        throw InferenceException(context + ": output shape does not match the sliced ranges");
    }
    int64_t out_count = 1;
    for (const int64_t d : out.dims) {
        if (d < 0) {
            throw InferenceException(context + ": non-positive dimension");
        }
        out_count *= d;
    }
    (void)CountNonNeg(in.dims, context);
    if (out_count > 0 && (in.data == nullptr || out.data == nullptr)) {
        throw InferenceException(context + ": null buffer");
    }
    if (out_count > 0) {
        const std::vector<int64_t> in_strides = Strides(in.dims);
        int64_t base = 0;
        std::vector<int64_t> ss(static_cast<size_t>(rank));
        for (int64_t j = 0; j < rank; ++j) {
            const size_t u = static_cast<size_t>(j);
            base += begins[u] * in_strides[u];
            ss[u] = step_of[u] * in_strides[u];
        }
        CopyBox(in, Bytes(in.data) + base * ElementSize(in.dtype), out.data, out.dims, ss, Strides(out.dims), context);
    }
    AfterRow(outputs, context);
}

// src/kernels/expand.cpp:54-118
NERT_HIP_ROW(Expand) {
    const std::string context = "Expand (node '" + node.name + "')";
    if (inputs.size() != 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected a data input, a shape input, and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& shape_view = inputs[1];
    const TensorView& out = outputs[0];
    if (!MovableDtype(in.dtype)) {
        throw InferenceException(context + ": tensors must be float32, int64, or bool");
    }
    if (out.dtype != in.dtype) {
        throw InferenceException(context + ": output dtype must match the input dtype");
    }
    if (shape_view.dtype != DataType::Int64) {
        throw InferenceException(context + ": Expand requires a shape input");
    }
    auto count_nonneg = [&](const std::vector<int64_t>& dims) {
        int64_t c = 1;
        for (int64_t d : dims) {
            if (d < 0) {
                throw InferenceException(context + ": negative dimension");
            }
            c *= d;
        }
        return c;
    };
    const int64_t target_count = count_nonneg(shape_view.dims);
    if (target_count > 0 && shape_view.data == nullptr) {
        throw InferenceException(context + ": null shape buffer");
    }
    const std::vector<int64_t> target = ReadInt64(shape_view, target_count, context);
    const size_t rank = std::max(in.dims.size(), target.size());
    std::vector<int64_t> expected(rank, 1);
    for (size_t i = 0; i < rank; ++i) {
        const int64_t di = static_cast<int64_t>(in.dims.size()) - static_cast<int64_t>(rank) + static_cast<int64_t>(i);
        const int64_t si = static_cast<int64_t>(target.size()) - static_cast<int64_t>(rank) + static_cast<int64_t>(i);
        const int64_t d = di < 0 ? 1 : in.dims[static_cast<size_t>(di)];
        if (si < 0) {
            expected[i] = d;
            continue;
        }
        const int64_t s = target[static_cast<size_t>(si)];
        if (s < 1) {
            throw InferenceException(context + ": Expand target shape must be positive");
        }
        if (d == s || d == 1 || di < 0) {
            expected[i] = s;
        } else if (s == 1) {
            expected[i] = d;
        } else {
            throw InferenceException(context + ": Expand input is not broadcastable to the target shape");
        }
    }
    if (out.dims != expected) {
        throw InferenceException(context + ": output shape does not match the expanded shape");
    }
    const int64_t out_count = count_nonneg(out.dims);
    (void)count_nonneg(in.dims);
    if (out_count > 0 && (in.data == nullptr || out.data == nullptr)) {
        throw InferenceException(context + ": null buffer");
    }
    const std::vector<int64_t> in_strides = Strides(in.dims);
    std::vector<int64_t> ss(rank, 0);
    for (size_t i = 0; i < rank; ++i) {
        const int64_t di = static_cast<int64_t>(in.dims.size()) - static_cast<int64_t>(rank) + static_cast<int64_t>(i);
        if (di >= 0 && in.dims[static_cast<size_t>(di)] != 1) {
            ss[i] = in_strides[static_cast<size_t>(di)];
        }
    }
    if (out_count > 0) {
        CopyBox(in, in.data, out.data, out.dims, ss, Strides(out.dims), context);
    }
    AfterRow(outputs, context);
}

// src/kernels/tile.cpp:54-96
NERT_HIP_ROW(Tile) {
    const std::string context = "Tile (node '" + node.name + "')";
    if (inputs.size() != 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected a data input, a repeats input, and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& repeats = inputs[1];
    const TensorView& out = outputs[0];
    if (in.dtype != out.dtype || !MovableDtype(in.dtype)) {
        throw InferenceException(context + ": data must share one float32, int64, or bool dtype");
    }
    if (repeats.dtype != DataType::Int64 || repeats.dims.size() != 1 ||
        repeats.dims[0] != static_cast<int64_t>(in.dims.size())) {
        throw InferenceException(context + ": repeats must be a rank-1 int64 tensor with one entry per input axis");
    }
    (void)ElementCount(in.dims, context);
    (void)ElementCount(out.dims, context);
    if (in.data == nullptr || repeats.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    const std::vector<int64_t> reps = ReadInt64(repeats, static_cast<int64_t>(in.dims.size()), context);
    if (out.dims.size() != in.dims.size()) {
        throw InferenceException(context + ": output rank does not match the input rank");
    }
    for (size_t j = 0; j < in.dims.size(); ++j) {
        if (reps[j] <= 0 || out.dims[j] != in.dims[j] * reps[j]) {
            throw InferenceException(context + ": output shape does not match input dims times repeats");
        }
    }
    std::vector<int64_t> mods = in.dims;
    CopyBox(in, in.data, out.data, out.dims, Strides(in.dims), Strides(out.dims), context, &mods);
    AfterRow(outputs, context);
}

// src/kernels/squeeze.cpp:40-66: validation is the element count only.
NERT_HIP_ROW(Squeeze) {
    const std::string context = "Squeeze (node '" + node.name + "')";
    if (inputs.empty() || inputs.size() > 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected a data input, an optional axes input, and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != out.dtype) {
        throw InferenceException(context + ": input and output dtypes differ");
    }
    if (!MovableDtype(in.dtype)) {
        throw InferenceException(context + ": tensors must be float32, int64, or bool");
    }
    const int64_t count = ElementCount(out.dims, context);
    if (ElementCount(in.dims, context) != count) {
        throw InferenceException(context + ": element-count mismatch");
    }
    if (in.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    CopyAll(in, out, context);
    AfterRow(outputs, context);
}

// src/kernels/unsqueeze.cpp:30-118 (axes via src/axes_form.hpp)
NERT_HIP_ROW(Unsqueeze) {
    const std::string context = "Unsqueeze (node '" + node.name + "')";
    if (inputs.empty() || outputs.size() != 1) {
        throw InferenceException(context + ": expected a data input and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (!MovableDtype(in.dtype)) {
        throw InferenceException(context + ": tensors must be float32, int64, or bool");
    }
    if (out.dtype != in.dtype) {
        throw InferenceException(context + ": output dtype must match the input dtype");
    }
    auto count_nonneg = [&](const std::vector<int64_t>& dims) {
        int64_t c = 1;
        for (int64_t d : dims) {
            if (d < 0) {
                throw InferenceException(context + ": negative dimension");
            }
            c *= d;
        }
        return c;
    };
    const nert::AxesForm form = nert::ResolveAxesForm(node);
    std::vector<int64_t> axes;
    if (form.source == nert::AxesSource::Attribute) {
        if (inputs.size() != 1) {
            throw InferenceException(context + ": expected one data input for the attribute axes form");
        }
        const std::vector<int64_t>* values = nert::NodeAttributeIntList(form.axes_attribute);
        if (values == nullptr) {
            throw InferenceException(context + ": Unsqueeze requires an axes attribute");
        }
        axes = *values;
    } else {
        if (inputs.size() != 2) {
            throw InferenceException(context + ": expected a data input, an axes input, and one output");
        }
        const TensorView& av = inputs[1];
        if (av.dtype != DataType::Int64) {
            throw InferenceException(context + ": Unsqueeze requires an axes input");
        }
        const int64_t n = count_nonneg(av.dims);
        if (n > 0) {
            if (av.data == nullptr) {
                throw InferenceException(context + ": null axes buffer");
            }
            axes = ReadInt64(av, n, context);
        }
    }
    if (axes.empty()) {
        throw InferenceException(context + ": Unsqueeze axes must not be empty");
    }
    const int64_t rank_out = static_cast<int64_t>(in.dims.size()) + static_cast<int64_t>(axes.size());
    std::vector<bool> seen(static_cast<size_t>(rank_out), false);
    for (int64_t& axis : axes) {
        if (axis < -rank_out || axis >= rank_out) {
            throw InferenceException(context + ": Unsqueeze axis is out of range");
        }
        if (axis < 0) {
            axis += rank_out;
        }
        if (seen[static_cast<size_t>(axis)]) {
            throw InferenceException(context + ": Unsqueeze axes must be unique");
        }
        seen[static_cast<size_t>(axis)] = true;
    }
    std::vector<int64_t> expected(static_cast<size_t>(rank_out), 0);
    size_t data_pos = 0;
    for (int64_t i = 0; i < rank_out; ++i) {
        expected[static_cast<size_t>(i)] = seen[static_cast<size_t>(i)] ? 1 : in.dims[data_pos++];
    }
    if (out.dims != expected) {
        throw InferenceException(context + ": output shape does not match the unsqueezed input");
    }
    const int64_t in_count = count_nonneg(in.dims);
    const int64_t out_count = count_nonneg(out.dims);
    if (in_count != out_count) {
        throw InferenceException(context + ": element-count mismatch");
    }
    if (in_count > 0 && (in.data == nullptr || out.data == nullptr)) {
        throw InferenceException(context + ": null buffer");
    }
    CopyAll(in, out, context);
    AfterRow(outputs, context);
}

// src/kernels/pad.cpp:99-195
NERT_HIP_ROW(Pad) {
    const std::string context = "Pad (node '" + node.name + "')";
    if (inputs.size() < 2 || inputs.size() > 4 || outputs.size() != 1) {
        throw InferenceException(context + ": expected two to four inputs and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if ((in.dtype != DataType::Float32 && in.dtype != DataType::Int64) || out.dtype != in.dtype) {
        throw InferenceException(context + ": data tensors must share dtype float32 or int64");
    }
    int mode = 0;
    for (const Attribute& attr : node.attributes) {
        if (attr.name != "mode") {
            continue;
        }
        const std::string* value = std::get_if<std::string>(&attr.value);
        if (value == nullptr) {
            throw InferenceException(context + ": attribute 'mode' must be a string");
        }
        if (*value == "constant") {
            mode = 0;
        } else if (*value == "reflect") {
            mode = 1;
        } else if (*value == "edge") {
            mode = 2;
        } else {
            throw InferenceException(context + ": unsupported mode '" + *value + "'");
        }
    }
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    (void)ElementCount(in.dims, context);
    if (in.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    auto read = [&](const TensorView& view, const char* what) {
        if (view.dtype != DataType::Int64) {
            throw InferenceException(context + ": " + what + " must be int64");
        }
        const int64_t count = Count(view.dims);
        if (count > 0 && view.data == nullptr) {
            throw InferenceException(context + ": null " + std::string(what) + " buffer");
        }
        return ReadInt64(view, count, context);
    };
    const std::vector<int64_t> pads = read(inputs[1], "pads");
    std::vector<int64_t> axes;
    if (inputs.size() == 4 && inputs[3].dtype != DataType::Unknown) {
        axes = read(inputs[3], "axes");
    } else {
        for (int64_t i = 0; i < rank; ++i) {
            axes.push_back(i);
        }
    }
    if (pads.size() != axes.size() * 2) {
        throw InferenceException(context + ": pads must hold two entries per padded axis");
    }
    std::vector<int64_t> begins(static_cast<size_t>(rank), 0);
    std::vector<int64_t> ends(static_cast<size_t>(rank), 0);
    std::vector<bool> seen(static_cast<size_t>(rank), false);
    for (size_t k = 0; k < axes.size(); ++k) {
        int64_t axis = axes[k];
        if (axis < -rank || axis >= rank) {
            throw InferenceException(context + ": axis out of range");
        }
        if (axis < 0) {
            axis += rank;
        }
        if (seen[static_cast<size_t>(axis)]) {
            throw InferenceException(context + ": duplicate axis");
        }
        seen[static_cast<size_t>(axis)] = true;
        begins[static_cast<size_t>(axis)] = pads[k];
        ends[static_cast<size_t>(axis)] = pads[axes.size() + k];
    }
    std::vector<int64_t> expected = in.dims;
    for (size_t i = 0; i < expected.size(); ++i) {
        expected[i] += begins[i] + ends[i];
    }
    if (out.dims != expected) {
        throw InferenceException(context + ": output shape does not match the pads");
    }
    (void)ElementCount(out.dims, context);
    const bool has_value = inputs.size() >= 3 && inputs[2].dtype != DataType::Unknown;
    double fvalue = 0.0;
    int64_t ivalue = 0;
    if (has_value) {
        if (inputs[2].dtype != in.dtype) {
            throw InferenceException(context + ": constant_value must match the data dtype");
        }
        if (ElementCount(inputs[2].dims, context) != 1 || inputs[2].data == nullptr) {
            throw InferenceException(context + ": constant_value must be a scalar");
        }
        if (in.dtype == DataType::Float32) {
            fvalue = ReadFloat(inputs[2], 1, context)[0];
        } else {
            ivalue = ReadInt64(inputs[2], 1, context)[0];
        }
    }
    CheckStatus(nert_hip_pad(DtypeCode(in.dtype), in.data, out.data, static_cast<int>(rank), in.dims.data(),
                             out.dims.data(), begins.data(), mode, fvalue, ivalue, Stream()),
                context);
    AfterRow(outputs, context);
}

} // namespace rows
} // namespace nert_hip
