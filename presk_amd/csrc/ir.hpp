// The loop-nest IR the executor receives: PSK-Kernel's kernels, read from
// their textual form.
//
// The reference's types are crates/presk-kernel/src/ir.rs:15-322 (`Kernel`,
// `BufSpec`, `BufKind`, `Expr`, `Stmt`); the text is what its Display prints
// (ir.rs:495-595), which is also what `presk dump --stage kernel` shows.  A
// Rust host hands a kernel across the C ABI as that text plus the two facts
// the text leaves out: its storage type when no buffer shows it, and its lane
// width (`Kernel::dtype`, `Kernel::lanes`).
#pragma once

#include <cstdint>
#include <deque>
#include <memory>
#include <string>
#include <vector>

namespace presk {

// Storage types of a buffer (`Dtype` plus the index buffers of `BufKind::Idx`
// and the integer weights of `BufKind::Quant`, int8 one a byte and int4 two a
// byte, the even element in the low nibble).
enum class Ty : uint8_t { F64, F32, BF16, F16, E8M15, I64, Q8, Q4 };

const char* ty_name(Ty t);
bool ty_parse(const std::string& s, Ty* out);
int ty_bytes(Ty t);            // bytes of one stored element (e8m15: 3; int4: 1, two elements a byte)
bool ty_real(Ty t);            // everything but I64
bool ty_quant(Ty t);           // Q8 and Q4
bool ty_coded(Ty t);           // f16 and e8m15: a store into them is guarded

struct BufSpec {
    Ty ty = Ty::F32;           // the type the text shows
    bool wide = false;         // `BufKind::Wide`: narrower than the kernel's type
    // `BufKind::Quant { over, span }` (ir.rs:30): the scales are constant
    // along the `qspan` axes from axis `qover`
    int qover = 0, qspan = 1;
    std::vector<int64_t> dims;
    std::vector<std::string> names;  // "" for an unnamed axis
    int64_t numel() const;
    std::vector<int64_t> strides() const;
    // `BufSpec::scale_strides` (ir.rs:81-95): the scale of element ix is at
    // sum ix_a * s_a, zero along the span axes, the other axes row-major
    std::vector<int64_t> scale_strides() const;
    int64_t scale_count() const;   // the scales a Quant buffer's pointer holds
};

enum class Op : uint8_t { Add, Sub, Mul, Div };
enum class Un : uint8_t { Neg, Exp, Log, Tanh, Sqrt, Sin, Cos, Erf, Abs };
enum class Cmp : uint8_t { Lt, Le, Gt, Ge, Eq };

struct Expr {
    enum Kind : uint8_t { Num, Load, VLoad, Iv, Sv, Si, Vv, Bin, VBin, Unary, Compare, Select, ToF, ToI, Splat } kind;
    int id = 0;                // buffer (Load/VLoad) or variable number
    Op op = Op::Add;
    Un un = Un::Neg;
    Cmp cmp = Cmp::Lt;
    double num = 0;            // the literal's value
    bool integral = false;     // the literal is an integer (usable as i64)
    int64_t inum = 0;
    std::string lit;           // the literal as written
    std::vector<const Expr*> kids;   // index expressions, or operands
};

struct Stmt {
    enum Kind : uint8_t { For, Set, SetI, SetL, VSet, Store, VStore, If } kind;
    int var = 0;               // loop/real/int/vector variable
    int64_t bound = 0;         // For
    int buf = 0;               // Store/VStore
    std::vector<const Expr*> index;
    const Expr* value = nullptr;     // also the condition of If
    std::vector<const Stmt*> body;   // For / If
};

struct Kernel {
    std::string name;
    Ty dtype = Ty::F32;        // the storage type of its real buffers
    int lanes = 1;
    std::string arith;         // formats other than the native ones ("" = native)
    std::vector<BufSpec> inputs;
    BufSpec output;
    std::vector<const Stmt*> body;
    int nloops = 0, nreal = 0, nint = 0, nvec = 0;

    int out_buf() const { return (int)inputs.size(); }
    // the KernelFn slot of input b's scales (a Quant input), after the output
    // in input order (crates/presk-cranelift/src/lib.rs:1619-1624), or -1
    int scale_slot(int b) const;
    int n_quant() const;
    // the slot of the overflow flag: after the scales
    int flag_slot() const { return out_buf() + 1 + n_quant(); }
    const BufSpec& buf(int b) const { return b == out_buf() ? output : inputs[b]; }
    // `Kernel::guarded` (ir.rs:332-334): stores reals into f16 or e8m15.
    bool guarded() const { return ty_coded(dtype) && output.ty != Ty::I64; }

    // node storage
    std::deque<Expr> exprs;
    std::deque<Stmt> stmts;
};

// Parses one kernel's text.  `dtype` names the storage type ("f32", ...), or is
// empty to take it from the output (or the widest real input).  Returns
// nullptr and sets `err` on malformed text.
std::unique_ptr<Kernel> parse_kernel(const std::string& text, const std::string& dtype, int lanes, std::string* err);

// The text of a kernel, as the reference prints it (the round trip that pins
// the reader).
std::string show_kernel(const Kernel& k);
std::string show_expr(const Expr& e);

// `Kernel::parallel_outer` (ir.rs:336-373): the outermost loop's bound when
// splitting it is exact, else -1.
int64_t parallel_outer(const Kernel& k);

// `Kernel::writes_disjoint` for the loop variable `v` over statements `body`
// (ir.rs:396-492): every access to the output indexes one position by c*v+t,
// 0 <= t, t + span <= c.
bool writes_disjoint(const Kernel& k, int v, const std::vector<const Stmt*>& body);

}  // namespace presk
