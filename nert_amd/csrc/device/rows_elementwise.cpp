// Elementwise rows: unary math, broadcast arithmetic, comparisons, logic,
// Where, Max/Min, Clip and Cast. Validation mirrors the reference rows in
// src/kernels/{relu,sigmoid,...,add,sub,mul,div,pow,mod,max,min,equal,greater,
// less,greater_or_equal,less_or_equal,and,or,where,clip,cast}.cpp.

#include "rows.hpp"

#include <vector>

#include <algorithm>
#include <limits>

namespace nert_hip {
namespace rows {

using namespace seam;

namespace {

std::string Ctx(const char* op, const Node& node) { return std::string(op) + " (node '" + node.name + "')"; }

// One-in/one-out float rows (Relu, Sigmoid, Tanh, Exp, Log, Sqrt, Sin, Cos,
// Floor, Erf, Elu): e.g. src/kernels/exp.cpp:26-46.
void UnaryFloat(const char* op, int code, const Node& node, const Views& inputs, const Views& outputs, double p0 = 0,
                double p1 = 0) {
    const std::string context = Ctx(op, node);
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
        throw InferenceException(context + ": tensors must be float32");
    }
    const int64_t count = ElementCount(out.dims, context);
    if (ElementCount(in.dims, context) != count) {
        throw InferenceException(context + ": element-count mismatch");
    }
    if (in.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    CheckStatus(nert_hip_unary(code, NERT_F32, in.data, out.data, count, p0, p1, Stream()), context);
    AfterRow(outputs, context);
}

// Abs / Neg / Sign over float32 or int64 (src/kernels/abs.cpp:34-58,
// sign.cpp:36-57 which also requires equal dims).
void UnaryNumeric(const char* op, int code, bool same_dims, const Node& node, const Views& inputs,
                  const Views& outputs) {
    const std::string context = Ctx(op, node);
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if ((in.dtype != DataType::Float32 && in.dtype != DataType::Int64) || out.dtype != in.dtype) {
        throw InferenceException(context + ": tensors must be float32 or int64 with matching dtype");
    }
    if (same_dims && in.dims != out.dims) {
        throw InferenceException(context + ": shape mismatch");
    }
    const int64_t count = ElementCount(out.dims, context);
    if (ElementCount(in.dims, context) != count) {
        throw InferenceException(context + ": element-count mismatch");
    }
    if (in.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    CheckStatus(nert_hip_unary(code, DtypeCode(in.dtype), in.data, out.data, count, 0, 0, Stream()), context);
    AfterRow(outputs, context);
}

std::vector<int64_t> BroadcastDims(const std::vector<int64_t>& a, const std::vector<int64_t>& b,
                                   const std::string& context) {
    const size_t rank = std::max(a.size(), b.size());
    std::vector<int64_t> out(rank, 1);
    for (size_t i = 0; i < rank; ++i) {
        const int64_t da = i < rank - a.size() ? 1 : a[i - (rank - a.size())];
        const int64_t db = i < rank - b.size() ? 1 : b[i - (rank - b.size())];
        if (da != db && da != 1 && db != 1) {
            throw InferenceException(context + ": shapes are not broadcast-compatible");
        }
        out[i] = std::max(da, db);
    }
    return out;
}

void Launch(int op, int dtype, const std::vector<const TensorView*>& ins, const TensorView& out,
            const std::string& context) {
    const void* ptrs[3] = {nullptr, nullptr, nullptr};
    const int64_t* dims[3] = {nullptr, nullptr, nullptr};
    int ranks[3] = {0, 0, 0};
    for (size_t k = 0; k < ins.size(); ++k) {
        ptrs[k] = ins[k]->data;
        dims[k] = ins[k]->dims.data();
        ranks[k] = static_cast<int>(ins[k]->dims.size());
    }
    CheckStatus(nert_hip_broadcast(op, dtype, static_cast<int>(ins.size()), ptrs, dims, ranks, out.data,
                                   static_cast<int>(out.dims.size()), out.dims.data(), Stream()),
                context);
}

enum class BinaryKind { Arith, ArithFloatOnly, Int64Only, Compare, Logic };

// Two-input broadcast rows (src/kernels/add.cpp:96-131 and siblings).
void Binary(const char* op, int code, BinaryKind kind, const Node& node, const Views& inputs, const Views& outputs) {
    const std::string context = Ctx(op, node);
    if (inputs.size() != 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected two inputs and one output");
    }
    const TensorView& a = inputs[0];
    const TensorView& b = inputs[1];
    const TensorView& out = outputs[0];
    switch (kind) {
    case BinaryKind::Arith:
        if (a.dtype != b.dtype || (a.dtype != DataType::Float32 && a.dtype != DataType::Int64) ||
            out.dtype != a.dtype) {
            throw InferenceException(context + ": tensors must share one float32 or int64 dtype");
        }
        break;
    case BinaryKind::ArithFloatOnly:
        if (a.dtype != DataType::Float32 || b.dtype != DataType::Float32 || out.dtype != DataType::Float32) {
            throw InferenceException(context + ": tensors must be float32");
        }
        break;
    case BinaryKind::Int64Only:
        if (a.dtype != DataType::Int64 || b.dtype != DataType::Int64 || out.dtype != DataType::Int64) {
            throw InferenceException(context + ": tensors must be int64");
        }
        break;
    case BinaryKind::Compare:
        if (a.dtype != b.dtype || (a.dtype != DataType::Float32 && a.dtype != DataType::Int64)) {
            throw InferenceException(context + ": inputs must share one float32 or int64 dtype");
        }
        if (out.dtype != DataType::Bool) {
            throw InferenceException(context + ": output must be bool");
        }
        break;
    case BinaryKind::Logic:
        if (a.dtype != DataType::Bool || b.dtype != DataType::Bool) {
            throw InferenceException(context + ": inputs must be bool");
        }
        if (out.dtype != DataType::Bool) {
            throw InferenceException(context + ": output must be bool");
        }
        break;
    }
    (void)ElementCount(out.dims, context);
    (void)ElementCount(a.dims, context);
    (void)ElementCount(b.dims, context);
    if (BroadcastDims(a.dims, b.dims, context) != out.dims) {
        throw InferenceException(context + ": output shape does not match the broadcast of the inputs");
    }
    if (a.data == nullptr || b.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    const bool int_division = (code == NERT_BIN_DIV || code == NERT_BIN_MOD) && a.dtype == DataType::Int64;
    // A zero divisor must throw like the reference (src/kernels/div.cpp:110).
    // A divisor with a host shadow (an initializer, a shape) is checked here;
    // otherwise the row waits for the flag the kernel raises. With an empty
    // output no division happens and nothing throws.
    bool checked_on_host = false;
    if (int_division && Count(out.dims) > 0) {
        std::vector<int64_t> divisor;
        if (HostShadowInt64(b, Count(b.dims), divisor)) {
            for (int64_t d : divisor) {
                if (d == 0) {
                    throw InferenceException(context + ": division by zero");
                }
            }
            checked_on_host = true;
        }
    }
    Launch(code, DtypeCode(a.dtype), {&a, &b}, out, context);
    if (int_division && !checked_on_host) {
        ThrowOnDeviceFlag(context, "division by zero");
    }
    AfterRow(outputs, context);
}

// Max / Min: at least one input, folded left to right with the reference's
// std::max / std::min (src/kernels/max.cpp:76-160).
void Extremum(const char* op, int code, const Node& node, const Views& inputs, const Views& outputs) {
    const std::string context = Ctx(op, node);
    if (inputs.size() < 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected at least one input and one output");
    }
    const DataType dtype = inputs[0].dtype;
    if (dtype != DataType::Float32 && dtype != DataType::Int64) {
        throw InferenceException(context + ": tensors must share one float32 or int64 dtype");
    }
    for (const TensorView& in : inputs) {
        if (in.dtype != dtype) {
            throw InferenceException(context + ": tensors must share one float32 or int64 dtype");
        }
    }
    const TensorView& out = outputs[0];
    if (out.dtype != dtype) {
        throw InferenceException(context + ": tensors must share one float32 or int64 dtype");
    }
    std::vector<int64_t> acc = inputs[0].dims;
    (void)ElementCount(inputs[0].dims, context);
    for (size_t i = 1; i < inputs.size(); ++i) {
        (void)ElementCount(inputs[i].dims, context);
        acc = BroadcastDims(acc, inputs[i].dims, context);
    }
    if (acc != out.dims) {
        throw InferenceException(context + ": output shape does not match the broadcast of the inputs");
    }
    const int64_t count = ElementCount(out.dims, context);
    for (const TensorView& in : inputs) {
        if (in.data == nullptr) {
            throw InferenceException(context + ": null buffer");
        }
    }
    if (out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    if (inputs.size() == 1) {
        CheckStatus(nert_hip_memcpy_d2d(out.data, inputs[0].data, count * ElementSize(dtype), Stream()), context);
    } else {
        Launch(code, DtypeCode(dtype), {&inputs[0], &inputs[1]}, out, context);
        for (size_t i = 2; i < inputs.size(); ++i) {
            Launch(code, DtypeCode(dtype), {&out, &inputs[i]}, out, context);
        }
    }
    AfterRow(outputs, context);
}

} // namespace

NERT_HIP_ROW(Relu) { UnaryFloat("Relu", NERT_UN_RELU, node, inputs, outputs); }
NERT_HIP_ROW(Sigmoid) { UnaryFloat("Sigmoid", NERT_UN_SIGMOID, node, inputs, outputs); }
NERT_HIP_ROW(Tanh) { UnaryFloat("Tanh", NERT_UN_TANH, node, inputs, outputs); }
NERT_HIP_ROW(Exp) { UnaryFloat("Exp", NERT_UN_EXP, node, inputs, outputs); }
NERT_HIP_ROW(Log) { UnaryFloat("Log", NERT_UN_LOG, node, inputs, outputs); }
NERT_HIP_ROW(Sqrt) { UnaryFloat("Sqrt", NERT_UN_SQRT, node, inputs, outputs); }
NERT_HIP_ROW(Sin) { UnaryFloat("Sin", NERT_UN_SIN, node, inputs, outputs); }
NERT_HIP_ROW(Cos) { UnaryFloat("Cos", NERT_UN_COS, node, inputs, outputs); }
NERT_HIP_ROW(Floor) { UnaryFloat("Floor", NERT_UN_FLOOR, node, inputs, outputs); }
NERT_HIP_ROW(Erf) { UnaryFloat("Erf", NERT_UN_ERF, node, inputs, outputs); }
NERT_HIP_ROW(Abs) { UnaryNumeric("Abs", NERT_UN_ABS, false, node, inputs, outputs); }
NERT_HIP_ROW(Neg) { UnaryNumeric("Neg", NERT_UN_NEG, false, node, inputs, outputs); }
NERT_HIP_ROW(Sign) { UnaryNumeric("Sign", NERT_UN_SIGN, true, node, inputs, outputs); }

// src/kernels/elu.cpp:38-67; alpha defaults to 1.0.
NERT_HIP_ROW(Elu) {
    const std::string context = Ctx("Elu", node);
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const float alpha = FloatAttr(node, "alpha", 1.0f, "Elu");
    UnaryFloat("Elu", NERT_UN_ELU, node, inputs, outputs, static_cast<double>(alpha));
}

// src/kernels/is_nan.cpp:26-51.
NERT_HIP_ROW(IsNaN) {
    const std::string context = Ctx("IsNaN", node);
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != DataType::Float32 || out.dtype != DataType::Bool) {
        throw InferenceException(context + ": input must be float32 and output bool");
    }
    const int64_t count = ElementCount(out.dims, context);
    if (ElementCount(in.dims, context) != count) {
        throw InferenceException(context + ": element-count mismatch");
    }
    if (in.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    CheckStatus(nert_hip_unary(NERT_UN_ISNAN, NERT_F32, in.data, out.data, count, 0, 0, Stream()), context);
    AfterRow(outputs, context);
}

// src/kernels/not.cpp:14-41.
NERT_HIP_ROW(Not) {
    const std::string context = Ctx("Not", node);
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != DataType::Bool || out.dtype != DataType::Bool) {
        throw InferenceException(context + ": input and output must be bool");
    }
    if (in.dims != out.dims) {
        throw InferenceException(context + ": output shape must match the input shape");
    }
    const int64_t count = ElementCount(in.dims, context);
    if (in.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    CheckStatus(nert_hip_unary(NERT_UN_NOT, NERT_BOOL, in.data, out.data, count, 0, 0, Stream()), context);
    AfterRow(outputs, context);
}

// src/kernels/clip.cpp:25-98: optional scalar min/max operands of the data
// dtype; omitted bounds make the clamp an identity.
NERT_HIP_ROW(Clip) {
    const std::string context = Ctx("Clip", node);
    if (inputs.empty() || inputs.size() > 3 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one to three inputs and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != out.dtype) {
        throw InferenceException(context + ": tensors must be float32");
    }
    if (in.dtype != DataType::Float32 && in.dtype != DataType::Int64) {
        throw InferenceException(context + ": tensors must be float32");
    }
    const bool is_float = in.dtype == DataType::Float32;
    const int64_t count = ElementCount(out.dims, context);
    if (ElementCount(in.dims, context) != count) {
        throw InferenceException(context + ": element-count mismatch");
    }
    if (in.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    auto present = [&](size_t i) { return i < inputs.size() && inputs[i].dtype != DataType::Unknown; };
    auto check_bound = [&](size_t i) {
        const TensorView& bound = inputs[i];
        if (bound.dtype != in.dtype) {
            throw InferenceException(context + ": min/max must be " + (is_float ? "float32" : "int64"));
        }
        if (ElementCount(bound.dims, context) != 1) {
            throw InferenceException(context + ": min/max must be scalar");
        }
        if (bound.data == nullptr) {
            throw InferenceException(context + ": null buffer");
        }
    };
    if (is_float) {
        float lo = -std::numeric_limits<float>::infinity();
        float hi = std::numeric_limits<float>::infinity();
        if (present(1)) {
            check_bound(1);
            lo = ReadFloat(inputs[1], 1, context)[0];
        }
        if (present(2)) {
            check_bound(2);
            hi = ReadFloat(inputs[2], 1, context)[0];
        }
        CheckStatus(nert_hip_unary(NERT_UN_CLIP, NERT_F32, in.data, out.data, count, lo, hi, Stream()), context);
    } else {
        int64_t lo = std::numeric_limits<int64_t>::min();
        int64_t hi = std::numeric_limits<int64_t>::max();
        if (present(1)) {
            check_bound(1);
            lo = ReadInt64(inputs[1], 1, context)[0];
        }
        if (present(2)) {
            check_bound(2);
            hi = ReadInt64(inputs[2], 1, context)[0];
        }
        CheckStatus(nert_hip_clip_i64(static_cast<const int64_t*>(in.data), static_cast<int64_t*>(out.data), count,
                                      lo, hi, Stream()),
                    context);
    }
    AfterRow(outputs, context);
}

NERT_HIP_ROW(Add) { Binary("Add", NERT_BIN_ADD, BinaryKind::Arith, node, inputs, outputs); }
NERT_HIP_ROW(Sub) { Binary("Sub", NERT_BIN_SUB, BinaryKind::Arith, node, inputs, outputs); }
NERT_HIP_ROW(Mul) { Binary("Mul", NERT_BIN_MUL, BinaryKind::Arith, node, inputs, outputs); }
NERT_HIP_ROW(Div) { Binary("Div", NERT_BIN_DIV, BinaryKind::Arith, node, inputs, outputs); }
NERT_HIP_ROW(Pow) { Binary("Pow", NERT_BIN_POW, BinaryKind::ArithFloatOnly, node, inputs, outputs); }
NERT_HIP_ROW(Equal) { Binary("Equal", NERT_BIN_EQUAL, BinaryKind::Compare, node, inputs, outputs); }
NERT_HIP_ROW(Greater) { Binary("Greater", NERT_BIN_GREATER, BinaryKind::Compare, node, inputs, outputs); }
NERT_HIP_ROW(Less) { Binary("Less", NERT_BIN_LESS, BinaryKind::Compare, node, inputs, outputs); }
NERT_HIP_ROW(GreaterOrEqual) {
    Binary("GreaterOrEqual", NERT_BIN_GREATER_EQUAL, BinaryKind::Compare, node, inputs, outputs);
}
NERT_HIP_ROW(LessOrEqual) { Binary("LessOrEqual", NERT_BIN_LESS_EQUAL, BinaryKind::Compare, node, inputs, outputs); }
NERT_HIP_ROW(And) { Binary("And", NERT_BIN_AND, BinaryKind::Logic, node, inputs, outputs); }
NERT_HIP_ROW(Or) { Binary("Or", NERT_BIN_OR, BinaryKind::Logic, node, inputs, outputs); }
NERT_HIP_ROW(Max) { Extremum("Max", NERT_BIN_MAX, node, inputs, outputs); }
NERT_HIP_ROW(Min) { Extremum("Min", NERT_BIN_MIN, node, inputs, outputs); }

// src/kernels/mod.cpp:80-113: int64 only, fmod must be 0.
NERT_HIP_ROW(Mod) {
    const std::string context = Ctx("Mod", node);
    if (inputs.size() != 2 || outputs.size() != 1) {
        throw InferenceException(context + ": expected two inputs and one output");
    }
    for (const Attribute& attr : node.attributes) {
        if (attr.name == "fmod") {
            const int64_t* value = std::get_if<int64_t>(&attr.value);
            if (value == nullptr) {
                throw InferenceException(context + ": attribute 'fmod' must be an integer");
            }
            if (*value != 0) {
                throw InferenceException(context + ": only fmod=0 (integer remainder) is supported");
            }
        }
    }
    Binary("Mod", NERT_BIN_MOD, BinaryKind::Int64Only, node, inputs, outputs);
}

// src/kernels/where.cpp:100-145.
NERT_HIP_ROW(Where) {
    const std::string context = Ctx("Where", node);
    if (inputs.size() != 3 || outputs.size() != 1) {
        throw InferenceException(context + ": expected three inputs and one output");
    }
    const TensorView& cond = inputs[0];
    const TensorView& x = inputs[1];
    const TensorView& z = inputs[2];
    const TensorView& out = outputs[0];
    if (cond.dtype != DataType::Bool) {
        throw InferenceException(context + ": condition must be bool");
    }
    if (x.dtype != z.dtype || (x.dtype != DataType::Float32 && x.dtype != DataType::Int64) || out.dtype != x.dtype) {
        throw InferenceException(context + ": value tensors must share one float32 or int64 dtype");
    }
    (void)ElementCount(out.dims, context);
    (void)ElementCount(cond.dims, context);
    (void)ElementCount(x.dims, context);
    (void)ElementCount(z.dims, context);
    if (BroadcastDims(BroadcastDims(cond.dims, x.dims, context), z.dims, context) != out.dims) {
        throw InferenceException(context + ": output shape does not match the broadcast of the inputs");
    }
    if (cond.data == nullptr || x.data == nullptr || z.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    Launch(NERT_BIN_WHERE, DtypeCode(x.dtype), {&cond, &x, &z}, out, context);
    AfterRow(outputs, context);
}

// src/kernels/cast.cpp:70-116.
NERT_HIP_ROW(Cast) {
    const std::string context = Ctx("Cast", node);
    if (inputs.size() != 1 || outputs.size() != 1) {
        throw InferenceException(context + ": expected one input and one output");
    }
    const TensorView& in = inputs[0];
    const TensorView& out = outputs[0];
    if (in.dtype != DataType::Float32 && in.dtype != DataType::Int64 && in.dtype != DataType::Bool) {
        throw InferenceException(context + ": input must be float32, int64, or bool");
    }
    const Attribute* to_attr = FindAttr(node, "to");
    if (to_attr == nullptr) {
        throw InferenceException(context + ": missing required attribute 'to'");
    }
    const int64_t* to_value = std::get_if<int64_t>(&to_attr->value);
    if (to_value == nullptr) {
        throw InferenceException(context + ": attribute 'to' must be an integer");
    }
    const int64_t to = *to_value;
    DataType want = DataType::Unknown;
    if (to == 1) {
        want = DataType::Float32;
    } else if (to == 6 || to == 7) {
        want = DataType::Int64;
    } else if (to == 9) {
        want = DataType::Bool;
    } else {
        throw InferenceException(context + ": attribute 'to' names an unsupported element type");
    }
    if (out.dtype != want) {
        throw InferenceException(context + ": output dtype does not match attribute 'to'");
    }
    const int64_t out_count = ElementCount(out.dims, context);
    const int64_t in_count = ElementCount(in.dims, context);
    if (in_count != out_count || in.dims != out.dims) {
        throw InferenceException(context + ": output shape must match the input shape");
    }
    if (in.data == nullptr || out.data == nullptr) {
        throw InferenceException(context + ": null buffer");
    }
    CheckStatus(nert_hip_cast(DtypeCode(in.dtype), DtypeCode(want), to == 6 ? 1 : 0, in.data, out.data, out_count,
                              Stream()),
                context);
    AfterRow(outputs, context);
}

} // namespace rows
} // namespace nert_hip
