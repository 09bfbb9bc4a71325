// Resampling and contraction rows: Resize, GridSample, Einsum,
// ConvTranspose. Each row rejects the nodes its reference row rejects
// (src/kernels/{resize,grid_sample,einsum,conv_transpose}.cpp), in the same
// order and with the same messages, before it queues any work.

#include "rows.hpp"

#include <algorithm>
#include <cmath>
#include <map>

namespace nert_hip {
namespace rows {

using namespace seam;

// ---- Resize -----------------------------------------------------------------

// src/kernels/resize.cpp:162-255
NERT_HIP_ROW(Resize) {
    const std::string context = "Resize (node '" + node.name + "')";
    if (inputs.empty() || inputs.size() > 4 || outputs.size() != 1) {
        throw InferenceException(context + ": expected an input, roi, scales, and an optional sizes input");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    const std::string mode = StringAttr(node, "mode", "nearest", "Resize");
    if (mode != "nearest" && mode != "linear") {
        throw InferenceException(context + ": Resize 'mode' must be 'nearest' or 'linear' here");
    }
    const bool linear = mode == "linear";
    if (in.dtype != DataType::Float32 && !(in.dtype == DataType::Int64 && !linear)) {
        throw InferenceException(context + ": tensors must be float32 (or int64 for nearest)");
    }
    if (out.dtype != in.dtype) {
        throw InferenceException(context + ": output dtype must match the input dtype");
    }
    const std::string transform = StringAttr(node, "coordinate_transformation_mode", "half_pixel", "Resize");
    const std::string nearest = StringAttr(node, "nearest_mode", "round_prefer_floor", "Resize");
    const int64_t rank = static_cast<int64_t>(in.dims.size());
    std::vector<double> scales(static_cast<size_t>(rank), 1.0);
    const bool has_scales =
        inputs.size() > 2 && inputs[2].dtype != DataType::Unknown && CountNonNeg(inputs[2].dims, context) > 0;
    const bool has_sizes = inputs.size() > 3 && inputs[3].dtype != DataType::Unknown;
    if (has_sizes && has_scales) {
        throw InferenceException(context + ": Resize takes exactly one of scales and sizes");
    }
    if (has_sizes) {
        const TensorView& sizes_view = inputs[3];
        if (sizes_view.dtype != DataType::Int64 || CountNonNeg(sizes_view.dims, context) != rank ||
            sizes_view.data == nullptr) {
            throw InferenceException(context + ": Resize sizes must be int64 with one entry per input axis");
        }
        const std::vector<int64_t> sizes = ReadInt64(sizes_view, rank, context);
        for (int64_t i = 0; i < rank; ++i) {
            const size_t u = static_cast<size_t>(i);
            if (out.dims.size() != static_cast<size_t>(rank) || out.dims[u] != sizes[u]) {
                throw InferenceException(context + ": output shape does not match the sizes input");
            }
            scales[u] = static_cast<double>(static_cast<float>(sizes[u]) / static_cast<float>(in.dims[u]));
        }
    } else {
        if (!has_scales || inputs[2].dtype != DataType::Float32) {
            throw InferenceException(context + ": Resize requires a scales or sizes input");
        }
        const TensorView& scales_view = inputs[2];
        if (CountNonNeg(scales_view.dims, context) != rank) {
            throw InferenceException(context + ": Resize scales rank must match the input rank");
        }
        if (scales_view.data == nullptr) {
            throw InferenceException(context + ": null scales buffer");
        }
        const std::vector<float> fs = ReadFloat(scales_view, rank, context);
        std::vector<int64_t> expected(static_cast<size_t>(rank), 0);
        for (int64_t i = 0; i < rank; ++i) {
            const size_t u = static_cast<size_t>(i);
            const int64_t dim =
                static_cast<int64_t>(std::floor(static_cast<double>(in.dims[u]) * static_cast<double>(fs[u])));
            if (dim <= 0) {
                throw InferenceException(context + ": Resize produces a non-positive output dim");
            }
            expected[u] = dim;
            scales[u] = static_cast<double>(fs[u]);
        }
        if (out.dims != expected) {
            throw InferenceException(context + ": output shape does not match the scaled input");
        }
    }
    const int64_t out_count = CountNonNeg(out.dims, context);
    (void)CountNonNeg(in.dims, context);
    if (out_count > 0 && (in.data == nullptr || out.data == nullptr)) {
        throw InferenceException(context + ": null buffer");
    }
    // The reference resolves the modes while building its per-axis tables,
    // i.e. only when some axis has output positions (resize.cpp:87-93).
    bool any_positions = false;
    for (const int64_t d : out.dims) {
        any_positions = any_positions || d > 0;
    }
    int transform_code = NERT_RESIZE_HALF_PIXEL;
    int nearest_code = NERT_RESIZE_ROUND_PREFER_FLOOR;
    if (any_positions) {
        if (transform == "half_pixel") {
            transform_code = NERT_RESIZE_HALF_PIXEL;
        } else if (transform == "pytorch_half_pixel") {
            transform_code = NERT_RESIZE_PYTORCH_HALF_PIXEL;
        } else if (transform == "align_corners") {
            transform_code = NERT_RESIZE_ALIGN_CORNERS;
        } else if (transform == "asymmetric") {
            transform_code = NERT_RESIZE_ASYMMETRIC;
        } else {
            throw InferenceException(context + ": unsupported coordinate_transformation_mode '" + transform + "'");
        }
        if (!linear) {
            if (nearest == "round_prefer_floor") {
                nearest_code = NERT_RESIZE_ROUND_PREFER_FLOOR;
            } else if (nearest == "round_prefer_ceil") {
                nearest_code = NERT_RESIZE_ROUND_PREFER_CEIL;
            } else if (nearest == "floor") {
                nearest_code = NERT_RESIZE_FLOOR;
            } else if (nearest == "ceil") {
                nearest_code = NERT_RESIZE_CEIL;
            } else {
                throw InferenceException(context + ": unsupported nearest_mode '" + nearest + "'");
            }
        }
    }
    if (out_count > 0) {
        CheckStatus(nert_hip_resize(DtypeCode(in.dtype), in.data, out.data, static_cast<int>(rank), in.dims.data(),
                                    out.dims.data(), scales.data(), linear ? 1 : 0, transform_code, nearest_code,
                                    Stream()),
                    context);
    }
    AfterRow(outputs, context);
}

// ---- GridSample -------------------------------------------------------------

// src/kernels/grid_sample.cpp:77-160
NERT_HIP_ROW(GridSample) {
    const std::string context = "GridSample (node '" + node.name + "')";
    if (inputs.size() != 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected two inputs and one output");
    }
    const std::string mode = StringAttr(node, "mode", "bilinear", "GridSample");
    const std::string padding = StringAttr(node, "padding_mode", "zeros", "GridSample");
    int64_t align = 0;
    if (const Attribute* attr = FindAttr(node, "align_corners")) {
        const int64_t* v = std::get_if<int64_t>(&attr->value);
        if (v == nullptr) {
            throw InferenceException("GridSample: attribute 'align_corners' must be an int (node '" + node.name +
                                     "')");
        }
        align = *v;
    }
    if (mode != "bilinear" && mode != "nearest") {
        throw InferenceException(context + ": unsupported mode '" + mode + "'");
    }
    if (padding != "zeros" && padding != "border" && padding != "reflection") {
        throw InferenceException(context + ": unsupported padding_mode '" + padding + "'");
    }
    if (align != 0 && align != 1) {
        throw InferenceException(context + ": align_corners must be 0 or 1");
    }
    const TensorView& x = inputs[0];
    const TensorView& grid = inputs[1];
    const TensorView& out = outputs[0];
    if (x.dtype != DataType::Float32 || grid.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
        throw InferenceException(context + ": tensors must be float32");
    }
    if (x.dims.size() != 4 || grid.dims.size() != 4 || grid.dims[3] != 2) {
        throw InferenceException(context + ": expected X [N,C,H,W] and grid [N,Ho,Wo,2]");
    }
    const int64_t n = x.dims[0];
    const int64_t c = x.dims[1];
    const int64_t h = x.dims[2];
    const int64_t w = x.dims[3];
    const int64_t ho = grid.dims[1];
    const int64_t wo = grid.dims[2];
    if (grid.dims[0] != n) {
        throw InferenceException(context + ": batch sizes of X and grid differ");
    }
    if (out.dims != std::vector<int64_t>({n, c, ho, wo})) {
        throw InferenceException(context + ": output shape does not match the operands");
    }
    if (n <= 0 || c <= 0 || h <= 0 || w <= 0 || ho <= 0 || wo <= 0) {
        throw InferenceException(context + ": non-positive dimension");
    }
    if (x.data == nullptr || grid.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    const int pad_code =
        padding == "zeros" ? NERT_GRID_ZEROS : (padding == "border" ? NERT_GRID_BORDER : NERT_GRID_REFLECTION);
    CheckStatus(nert_hip_grid_sample_f32(static_cast<const float*>(x.data), static_cast<const float*>(grid.data),
                                         static_cast<float*>(out.data), n, c, h, w, ho, wo, mode == "nearest" ? 1 : 0,
                                         pad_code, static_cast<int>(align), Stream()),
                context);
    AfterRow(outputs, context);
}

// ---- Einsum -------------------------------------------------------------------
//
// Front end, from the ONNX Einsum rules: the equation is scanned once into
// terms of integer label ids. Letters keep their ASCII order as ids
// ('A'..'Z' = 0..25, 'a'..'z' = 26..51), so "alphabetical" (the implicit
// output, the summation order) is id order. An ellipsis stands for up to W
// batch slots, W being the widest ellipsis over the operands; slot s has id
// kSlotId + s, after every letter. Each operand's ellipsis dims fill the
// last slots (right-aligned, NumPy broadcasting); the slots it does not
// reach, and all slots of an operand without an ellipsis, are virtual:
// extent 1, stride 0, no storage. Slots broadcast (1 against n); letters
// must agree exactly. The row then hands the kernel one extent and one
// stride per operand for every output label and every summed label.
// Rejections, their order and their text follow src/kernels/einsum.cpp
// (the seam compares messages verbatim).

namespace {

constexpr int kLetterIds = 52;
constexpr int kSlotId = 64;

int LetterId(char c) {
    if (c >= 'A' && c <= 'Z') {
        return c - 'A';
    }
    if (c >= 'a' && c <= 'z') {
        return 26 + (c - 'a');
    }
    return -1;
}

// One subscript: its letters in order and where "..." sits among them.
struct Term {
    std::vector<int> ids;  // letter ids; -1 for a character that is no letter
    int dots_at = -1;      // index into ids before which "..." stands, -1 if none
    bool malformed_dots = false;  // dots other than exactly one "..." group
    bool foreign_char = false;    // a character that is neither a letter nor a dot

    const char* SyntaxError() const {
        if (malformed_dots) {
            return "dots must form exactly one '...' per subscript";
        }
        if (foreign_char) {
            return "invalid character in the equation";
        }
        return nullptr;
    }
};

Term ScanTerm(const std::string& text, size_t begin, size_t end) {
    Term t;
    size_t dots = 0;
    size_t first_dot = end;
    for (size_t i = begin; i < end; ++i) {
        const char c = text[i];
        if (c == '.') {
            if (dots++ == 0) {
                first_dot = i;
                t.dots_at = static_cast<int>(t.ids.size());
            }
            continue;
        }
        const int id = LetterId(c);
        t.foreign_char = t.foreign_char || id < 0;
        t.ids.push_back(id);
    }
    // Valid only as no dot at all or exactly three adjacent ones.
    if (dots != 0 && !(dots == 3 && text[first_dot + 1] == '.' && text[first_dot + 2] == '.')) {
        t.malformed_dots = true;
    }
    if (dots == 0) {
        t.dots_at = -1;
    }
    return t;
}

struct Equation {
    std::vector<Term> operands;
    Term output;
    bool explicit_output = false;
    bool any_dots = false;
};

Equation ScanEquation(const std::string& text) {
    Equation eq;
    const size_t arrow = text.find("->");
    const size_t lhs_end = arrow == std::string::npos ? text.size() : arrow;
    size_t begin = 0;
    for (size_t i = 0; i <= lhs_end; ++i) {
        if (i == lhs_end || text[i] == ',') {
            eq.operands.push_back(ScanTerm(text, begin, i));
            begin = i + 1;
        }
    }
    if (arrow != std::string::npos) {
        eq.explicit_output = true;
        eq.output = ScanTerm(text, arrow + 2, text.size());
    }
    eq.any_dots = text.find('.') != std::string::npos;
    return eq;
}

// One storage (or virtual) axis of an operand, outermost first.
struct Axis {
    int label;
    int64_t extent;
    bool is_virtual;
};

} // namespace

// src/kernels/einsum.cpp:134-258 (row), equation rules :36-132, ellipsis :291-459
NERT_HIP_ROW(Einsum) {
    const std::string context = "Einsum (node '" + node.name + "')";
    const Attribute* attr = nullptr;
    for (const Attribute& a : node.attributes) {
        if (a.name == "equation") {
            attr = &a;
        }
    }
    if (attr == nullptr) {
        throw InferenceException(context + ": missing 'equation' attribute");
    }
    const std::string* raw = std::get_if<std::string>(&attr->value);
    if (raw == nullptr) {
        throw InferenceException(context + ": attribute 'equation' must be a string");
    }
    std::string text;
    for (char c : *raw) {
        if (c != ' ') {
            text.push_back(c);
        }
    }
    const Equation eq = ScanEquation(text);
    auto fail = [&](const char* why) { throw InferenceException(context + ": " + why); };

    // Ellipsis slots: the widest operand ellipsis, checked against the ranks
    // before anything else about the labels.
    size_t slots = 0;
    std::vector<size_t> covered(eq.operands.size(), 0);  // dims each operand's ellipsis covers
    if (eq.any_dots) {
        if (!eq.explicit_output) {
            fail("implicit output with ellipsis is not supported");
        }
        for (const Term& t : eq.operands) {
            if (const char* why = t.SyntaxError()) {
                fail(why);
            }
        }
        if (const char* why = eq.output.SyntaxError()) {
            fail(why);
        }
        if (eq.operands.size() != inputs.size()) {
            fail("operand count does not match the equation");
        }
        for (size_t i = 0; i < eq.operands.size(); ++i) {
            const Term& t = eq.operands[i];
            const size_t rank = inputs[i].dims.size();
            if (rank < t.ids.size()) {
                fail("operand rank is smaller than its explicit labels");
            }
            if (t.dots_at < 0 && rank != t.ids.size()) {
                fail("operand rank does not match its subscript");
            }
            covered[i] = t.dots_at < 0 ? 0 : rank - t.ids.size();
            slots = std::max(slots, covered[i]);
        }
        // The slots must fit in the letters the equation leaves unused: an
        // equation that needs more is rejected.
        bool seen[kLetterIds] = {false};
        size_t letters = 0;
        for (char c : text) {
            const int id = LetterId(c);
            if (id >= 0 && !seen[id]) {
                seen[id] = true;
                ++letters;
            }
        }
        if (slots > kLetterIds - letters) {
            fail("equation leaves no fresh labels for the ellipsis");
        }
    } else {
        for (const Term& t : eq.operands) {
            if (t.foreign_char) {
                fail("invalid character in the equation");
            }
        }
    }

    // How often each label appears over the operands (every operand spells
    // every slot once when the equation has an ellipsis).
    std::map<int, int> uses;
    for (const Term& t : eq.operands) {
        for (int id : t.ids) {
            ++uses[id];
        }
        for (size_t s = 0; s < slots; ++s) {
            ++uses[kSlotId + static_cast<int>(s)];
        }
    }
    std::vector<int> out_labels;
    if (eq.explicit_output) {
        // The output ids in spelling order, its "..." expanded to every slot.
        std::vector<int> spelled;
        const Term& o = eq.output;
        for (size_t q = 0; q <= o.ids.size(); ++q) {
            if (static_cast<int>(q) == o.dots_at) {
                for (size_t s = 0; s < slots; ++s) {
                    spelled.push_back(kSlotId + static_cast<int>(s));
                }
            }
            if (q < o.ids.size()) {
                spelled.push_back(o.ids[q]);
            }
        }
        for (size_t q = 0; q < spelled.size(); ++q) {
            if (spelled[q] < 0 || uses.count(spelled[q]) == 0) {
                fail("output label does not appear in the inputs");
            }
            if (std::find(spelled.begin(), spelled.begin() + static_cast<std::ptrdiff_t>(q), spelled[q]) !=
                spelled.begin() + static_cast<std::ptrdiff_t>(q)) {
                fail("output label repeated");
            }
        }
        out_labels = spelled;
    } else {
        for (const auto& [id, n] : uses) {
            if (n == 1) {
                out_labels.push_back(id);
            }
        }
    }
    if (eq.operands.size() != inputs.size() || inputs.empty() || inputs.size() > 2 || outputs.size() != 1) {
        fail("operand count does not match the equation");
    }
    const TensorView& out = outputs[0];
    if (out.dtype != DataType::Float32) {
        fail("tensors must be float32");
    }

    // Bind every label to one extent, operand by operand.
    std::vector<std::vector<Axis>> axes(inputs.size());
    std::map<int, int64_t> extent;
    for (size_t i = 0; i < inputs.size(); ++i) {
        const TensorView& in = inputs[i];
        if (in.dtype != DataType::Float32) {
            fail("tensors must be float32");
        }
        if (in.data == nullptr) {
            fail("null buffer");
        }
        const Term& t = eq.operands[i];
        const size_t rank = in.dims.size();
        const size_t real_slots = t.dots_at < 0 ? 0 : covered[i];
        if (rank != t.ids.size() + real_slots) {
            fail("operand rank does not match its subscript");
        }
        size_t d = 0;
        const size_t before = t.dots_at < 0 ? t.ids.size() : static_cast<size_t>(t.dots_at);
        for (size_t q = 0; q < before; ++q) {
            axes[i].push_back(Axis{t.ids[q], in.dims[d++], false});
        }
        for (size_t s = 0; s < slots; ++s) {
            const bool real = s + real_slots >= slots;
            axes[i].push_back(Axis{kSlotId + static_cast<int>(s), real ? in.dims[d++] : 1, !real});
        }
        for (size_t q = before; q < t.ids.size(); ++q) {
            axes[i].push_back(Axis{t.ids[q], in.dims[d++], false});
        }
        for (const Axis& a : axes[i]) {
            if (a.is_virtual) {
                extent.emplace(a.label, 1);
                continue;
            }
            if (a.extent <= 0) {
                fail("non-positive dimension");
            }
            auto [it, fresh] = extent.emplace(a.label, a.extent);
            if (!fresh && it->second != a.extent) {
                const bool broadcasts = a.label >= kSlotId && (it->second == 1 || a.extent == 1);
                if (!broadcasts) {
                    fail("label bound to two different sizes");
                }
                it->second = std::max(it->second, a.extent);
            }
        }
    }
    std::vector<int64_t> out_size;
    for (int id : out_labels) {
        out_size.push_back(extent.at(id));
    }
    if (out.dims != out_size) {
        fail("output shape does not match the operands");
    }
    if (out.data == nullptr) {
        fail("null buffer");
    }

    // Element strides per label and operand: a repeated label (a diagonal)
    // adds its strides; a virtual or broadcast (extent 1) slot adds none.
    std::vector<std::map<int, int64_t>> stride(2);
    for (size_t i = 0; i < inputs.size(); ++i) {
        int64_t step = 1;
        for (size_t k = axes[i].size(); k-- > 0;) {
            const Axis& a = axes[i][k];
            if (!a.is_virtual && a.extent == extent.at(a.label)) {
                stride[i][a.label] += step;
            } else if (!a.is_virtual && !(a.label >= kSlotId && a.extent == 1)) {
                fail("broadcast diagonal is not supported");
            }
            step *= a.extent;
        }
    }
    auto stride_of = [&](size_t i, int id) {
        const auto it = stride[i].find(id);
        return it == stride[i].end() ? int64_t{0} : it->second;
    };
    std::vector<int64_t> out_sa, out_sb, sum_size, sum_sa, sum_sb;
    for (int id : out_labels) {
        out_sa.push_back(stride_of(0, id));
        out_sb.push_back(stride_of(1, id));
    }
    for (const auto& [id, n] : extent) {  // summed labels in id order
        if (std::find(out_labels.begin(), out_labels.end(), id) == out_labels.end()) {
            sum_size.push_back(n);
            sum_sa.push_back(stride_of(0, id));
            sum_sb.push_back(stride_of(1, id));
        }
    }
    if (out_size.size() > 16 || sum_size.size() > 16) {
        fail("more than 16 output or summed labels");
    }
    // Every offset the kernel forms must stay inside its operand.
    for (size_t i = 0; i < inputs.size(); ++i) {
        int64_t last = 0;
        for (size_t d = 0; d < out_size.size(); ++d) {
            last += (out_size[d] - 1) * (i == 0 ? out_sa[d] : out_sb[d]);
        }
        for (size_t d = 0; d < sum_size.size(); ++d) {
            last += (sum_size[d] - 1) * (i == 0 ? sum_sa[d] : sum_sb[d]);
        }
        if (last >= ElementCount(inputs[i].dims, context)) {
            fail("internal error: operand strides exceed the operand");
        }
    }
    CheckStatus(nert_hip_einsum_f32(static_cast<const float*>(inputs[0].data),
                                    inputs.size() == 2 ? static_cast<const float*>(inputs[1].data) : nullptr,
                                    static_cast<float*>(out.data), static_cast<int>(out_size.size()), out_size.data(),
                                    out_sa.data(), out_sb.data(), static_cast<int>(sum_size.size()), sum_size.data(),
                                    sum_sa.data(), sum_sb.data(), Stream()),
                context);
    AfterRow(outputs, context);
}

// ---- ConvTranspose ------------------------------------------------------------

// src/kernels/conv_transpose.cpp:76-158
NERT_HIP_ROW(ConvTranspose) {
    const std::string context = "ConvTranspose (node '" + node.name + "')";
    if (inputs.size() < 2 || inputs.size() > 3 || outputs.size() != 1) {
        throw InferenceException(context + ": expected input, weight, optional bias, and one output");
    }
    const TensorView& x = inputs[0];
    const TensorView& w = inputs[1];
    const TensorView* bias = inputs.size() == 3 && inputs[2].data != nullptr ? &inputs[2] : nullptr;
    const TensorView& out = outputs[0];
    if (x.dtype != DataType::Float32 || w.dtype != DataType::Float32 || out.dtype != DataType::Float32 ||
        (bias != nullptr && bias->dtype != DataType::Float32)) {
        throw InferenceException(context + ": tensors must be float32");
    }
    if (x.dims.size() != 4 || w.dims.size() != 4) {
        throw InferenceException(context + ": input and weight must be rank 4 (NCHW)");
    }
    (void)ElementCount(x.dims, context);
    (void)ElementCount(w.dims, context);
    (void)ElementCount(out.dims, context);
    const int64_t group = IntAttr(node, "group", 1, "ConvTranspose");
    const int64_t in_c = x.dims[1];
    if (group <= 0 || in_c % group != 0 || w.dims[0] != in_c) {
        throw InferenceException(context + ": weight channels do not match the input and group");
    }
    const int64_t out_c = w.dims[1] * group;
    std::vector<int64_t> strides = IntsAttr(node, "strides", "ConvTranspose");
    std::vector<int64_t> dilations = IntsAttr(node, "dilations", "ConvTranspose");
    std::vector<int64_t> out_pad = IntsAttr(node, "output_padding", "ConvTranspose");
    std::vector<int64_t> pads = IntsAttr(node, "pads", "ConvTranspose");
    if (strides.empty()) {
        strides = {1, 1};
    }
    if (dilations.empty()) {
        dilations = {1, 1};
    }
    if (out_pad.empty()) {
        out_pad = {0, 0};
    }
    if (pads.empty() || StringAttr(node, "auto_pad", "NOTSET", "ConvTranspose") == "VALID") {
        pads = {0, 0, 0, 0};
    }
    if (strides.size() != 2 || dilations.size() != 2 || out_pad.size() != 2 || pads.size() != 4) {
        throw InferenceException(context + ": strides, dilations, output_padding, and pads must be 2-D");
    }
    const int64_t k_h = w.dims[2];
    const int64_t k_w = w.dims[3];
    const int64_t out_h = strides[0] * (x.dims[2] - 1) + out_pad[0] + dilations[0] * (k_h - 1) + 1 - pads[0] - pads[2];
    const int64_t out_w = strides[1] * (x.dims[3] - 1) + out_pad[1] + dilations[1] * (k_w - 1) + 1 - pads[1] - pads[3];
    if (out.dims != std::vector<int64_t>{x.dims[0], out_c, out_h, out_w}) {
        throw InferenceException(context + ": output shape does not match the transposed window");
    }
    if (bias != nullptr && (bias->dims.size() != 1 || bias->dims[0] != out_c)) {
        throw InferenceException(context + ": bias must be rank-1 of length M");
    }
    if (x.data == nullptr || w.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    if (strides[0] <= 0 || strides[1] <= 0) {
        // The gather form needs a positive stride; the reference's scatter
        // would fold every input pixel onto one row.
        throw InferenceException(context + ": strides must be positive");
    }
    const int64_t geom[16] = {x.dims[0], in_c,       out_c,      group,      x.dims[2],    x.dims[3],
                              out_h,     out_w,      k_h,        k_w,        strides[0],   strides[1],
                              pads[0],   pads[1],    dilations[0], dilations[1]};
    CheckStatus(nert_hip_conv_transpose_f32(static_cast<const float*>(x.data), static_cast<const float*>(w.data),
                                            bias != nullptr ? static_cast<const float*>(bias->data) : nullptr,
                                            static_cast<float*>(out.data), geom, Stream()),
                context);
    AfterRow(outputs, context);
}

} // namespace rows
} // namespace nert_hip
