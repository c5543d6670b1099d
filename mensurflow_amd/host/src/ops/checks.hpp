// Argument checks shared by the ops. Each throws std::invalid_argument with the message
// mensurflow's ops use for the same violation ("matmul: a must be 2-D, got shape [3]"), so a
// caller's error handling sees the same text.
#pragma once

#include "mensurflow/tensor.hpp"

#include <stdexcept>
#include <string>

namespace mensurflow::detail {

class OpCheck {
  public:
    explicit OpCheck(const char* op) : op_(op) {}

    [[noreturn]] void fail(const std::string& what) const {
        throw std::invalid_argument(op_ + ": " + what);
    }

    // "<op>: <name> is an undefined tensor"; then the rank: exactly `rank`, or at least `rank`.
    const OpCheck& operand(const Tensor& t, const char* name, int rank, bool at_least = false) const {
        if (!t.defined()) {
            fail(std::string(name) + " is an undefined tensor");
        }
        const bool ok = at_least ? t.dim() >= rank : t.dim() == rank;
        if (!ok) {
            fail(std::string(name) + " must be " + (at_least ? "at least " : "") +
                 std::to_string(rank) + "-D, got shape " + to_string(t.shape()));
        }
        return *this;
    }

    // "<op>: dtypes differ (f32 and i32)".
    const OpCheck& same_dtype(const Tensor& a, const Tensor& b) const {
        if (a.dtype() != b.dtype()) {
            fail(std::string("dtypes differ (") + dtype_name(a.dtype()) + " and " +
                 dtype_name(b.dtype()) + ")");
        }
        return *this;
    }

    // "<op>: tensors are on cpu:0 and rocm:0; move one with Tensor::to()".
    const OpCheck& same_device(const Tensor& a, const Tensor& b) const {
        if (a.device() != b.device()) {
            fail("tensors are on " + to_string(a.device()) + " and " + to_string(b.device()) +
                 "; move one with Tensor::to()");
        }
        return *this;
    }

    // Both checks above, after both tensors are checked to be defined ("<op>: undefined tensor").
    const OpCheck& compatible(const Tensor& a, const Tensor& b) const {
        if (!a.defined() || !b.defined()) {
            fail("undefined tensor");
        }
        return same_dtype(a, b).same_device(a, b);
    }

    const std::string& name() const { return op_; }

  private:
    std::string op_;
};

// The shapes a and b broadcast to; "<op>: cannot broadcast shapes ..." when they do not.
inline Shape broadcast_for(const OpCheck& check, const Shape& a, const Shape& b) {
    try {
        return broadcast_shapes(a, b);
    } catch (const std::invalid_argument& e) {
        check.fail(e.what());
    }
}

// Whether `shape` broadcasts to exactly `target`.
inline bool broadcasts_to(const Shape& shape, const Shape& target) {
    if (shape.size() > target.size()) {
        return false;
    }
    try {
        return broadcast_shapes(shape, target) == target;
    } catch (const std::invalid_argument&) {
        return false;
    }
}

} // namespace mensurflow::detail
