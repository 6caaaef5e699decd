// The generic HIP printer (see hipgen.hpp).
#include "hipgen.hpp"

#include <cctype>
#include <cmath>
#include <cstdio>
#include <algorithm>
#include <functional>
#include <map>
#include <set>
#include <sstream>

namespace presk {

namespace {

std::string hexlit(double x) {
    if (std::isnan(x)) return "__builtin_nan(\"\")";
    if (std::isinf(x)) return x > 0 ? "__builtin_inf()" : "(-__builtin_inf())";
    char buf[64];
    std::snprintf(buf, sizeof buf, "%a", x);
    return buf;
}

// The text of an index list, to compare accesses.
std::string index_key(const std::vector<const Expr*>& ix) {
    std::string s;
    for (auto e : ix) s += show_expr(*e) + ";";
    return s;
}

struct Printer {
    const Kernel& k;
    std::string A;              // arithmetic type
    std::vector<std::vector<int64_t>> strides;
    std::string err;
    // The output element a thread owns across its sequential loops, held in
    // the register `cell` (its value as stored, i.e. rounded to the storage
    // type) instead of memory: `cell_key` is its index list's text.
    std::string cell_key;
    // In a coarsened nest (VEC iterations of the innermost grid loop per
    // thread, `u` the iteration): input loads read ahead into `pre<n>[u]`
    // (key: buffer and index text), and the output's one store goes to
    // `post[u]`, written back after the iterations (key: its index text).
    std::map<std::string, int> pre;
    std::string post_key;
    // FAST mode: f32 exponentials and error functions by pk_expf_fast and
    // pk_erff_fast (within a stated bound of the interpreter's, not its
    // bits); `used_fast` records whether the kernel called one
    bool fast_fns = false;
    bool used_fast = false;

    explicit Printer(const Kernel& k) : k(k) {
        A = k.dtype == Ty::F64 ? "double" : "float";
        for (size_t b = 0; b <= k.inputs.size(); ++b) strides.push_back(k.buf((int)b).strides());
    }

    // Buffer b as the kernel's local pointer `pb<b>`.  They are declared
    // __restrict__: the output is never one of the inputs (the host lends
    // inputs and owns the output, crates/presk-kernel/src/host.rs:28-95), so
    // loads may move past stores of other iterations and merge.
    std::string ptr(int b) const { return "pb" + std::to_string(b); }

    // The buffers as __restrict__ parameters of the body function (only
    // parameters carry the no-alias fact into the compiler), and the casts
    // the kernel passes them with.
    std::string ptr_type(int b) const {
        const char* c = b == k.out_buf() ? "" : "const ";
        switch (k.buf(b).ty) {
            case Ty::F64: return std::string(c) + "double*";
            case Ty::F32: return std::string(c) + "float*";
            case Ty::BF16: case Ty::F16: return std::string(c) + "unsigned short*";
            case Ty::E8M15: case Ty::Q4: return std::string(c) + "unsigned char*";
            case Ty::Q8: return std::string(c) + "signed char*";
            case Ty::I64: return std::string(c) + "long long*";
        }
        return "";
    }
    // the scales of a Quant input b, `ps<b>`, in the slot after the output
    std::string sptr(int b) const { return "ps" + std::to_string(b); }
    std::string ptr_params() const {
        std::string d;
        for (int b = 0; b <= (int)k.inputs.size(); ++b) d += ", " + ptr_type(b) + " __restrict__ pb" + std::to_string(b);
        for (int b = 0; b < (int)k.inputs.size(); ++b)
            if (ty_quant(k.inputs[b].ty)) d += ", const float* __restrict__ " + sptr(b);
        return d;
    }
    std::string ptr_args() const {
        std::string d;
        for (int b = 0; b <= (int)k.inputs.size(); ++b) d += ", (" + ptr_type(b) + ")a.buf[" + std::to_string(b) + "]";
        for (int b = 0; b < (int)k.inputs.size(); ++b)
            if (ty_quant(k.inputs[b].ty)) d += ", (const float*)a.buf[" + std::to_string(k.scale_slot(b)) + "]";
        return d;
    }

    // element ix (moved `lane` along the last axis) of a Quant input as the
    // realization denotes it: f32(q) * s, one f32 multiplication
    // (crates/presk-rt/src/quant.rs:248-252, crates/presk-cranelift/src/
    // lib.rs:687-720); int4's element e the nibble of byte e/2, low when e
    // is even, sign-extended
    std::string quant_load(int b, const std::vector<const Expr*>& ix, const std::string& lane) {
        const BufSpec& q = k.buf(b);
        std::string off = offset(b, ix), soff = "(0LL";
        const auto ss = q.scale_strides();
        for (size_t p = 0; p < ix.size() && p < ss.size(); ++p)
            if (ss[p]) soff += " + (" + intx(ix[p]) + ")*" + std::to_string(ss[p]) + "LL";
        soff += ")";
        if (!lane.empty()) {
            off += " + " + lane;
            if (!ss.empty() && ss.back()) soff += " + (" + lane + ")*" + std::to_string(ss.back()) + "LL";
        }
        const std::string code = q.ty == Ty::Q8 ? "(float)" + ptr(b) + "[" + off + "]"
                                                : "(float)pk_nibble(" + ptr(b) + ", " + off + ")";
        return "(" + code + " * " + sptr(b) + "[" + soff + "])";
    }

    std::string offset(int b, const std::vector<const Expr*>& ix) {
        std::string s = "(0LL";
        for (size_t p = 0; p < ix.size() && p < strides[b].size(); ++p)
            s += " + (" + intx(ix[p]) + ")*" + std::to_string(strides[b][p]) + "LL";
        return s + ")";
    }

    // element `off` of buffer b widened exactly to its own arithmetic type
    std::string load_stored(int b, const std::string& off) {
        if (k.buf(b).ty == Ty::E8M15) return "pk_e8m15_to_f32(pk_ld24(" + ptr(b) + ", " + off + "))";
        return widen(b, ptr(b) + "[" + off + "]");
    }
    // a stored element `src` (a code) of buffer b as its arithmetic value
    std::string widen(int b, const std::string& src) const {
        switch (k.buf(b).ty) {
            case Ty::F64: case Ty::F32: return src;
            case Ty::BF16: return "pk_bf16_to_f32(" + src + ")";
            case Ty::F16: return "pk_f16_to_f32(" + src + ")";
            case Ty::I64: return "((double)" + src + ")";
            case Ty::E8M15: case Ty::Q8: case Ty::Q4: break;
        }
        return "";
    }
    // the read-ahead register holding load (b, ix), if there is one
    std::string pre_of(int b, const std::vector<const Expr*>& ix) const {
        auto it = pre.find(std::to_string(b) + "|" + index_key(ix));
        return it == pre.end() ? "" : "pre" + std::to_string(it->second) + "[u]";
    }

    // a / c in f32 arithmetic, c a finite nonzero constant: the quotient
    // rounded once from the f64 product a * RN64(1/c), which equals the
    // correctly rounded f32 quotient for every a (the product is within
    // 2^-52 of a/c relative, a quotient that is not a midpoint of the f32
    // grid lies at least 2^-49 relative from the nearest one, and one that
    // is, a double of at most 25 bits, is the product's rounding exactly);
    // pk_div_rc's three full-rate instructions in place of the division's
    // sequence.  "" where the form does not apply, and for a power of two,
    // whose exact product the compiler makes itself.
    std::string div_by_const(const Expr* e, const std::string& a, const Expr* den = nullptr) const {
        if (!den) den = e->kids[1];
        if (e->op != Op::Div || A != "float" || den->kind != Expr::Num) return "";
        const float c = (float)den->num;
        int ex = 0;
        if (!std::isfinite(c) || c == 0.0f || std::fabs(std::frexp(c, &ex)) == 0.5f) return "";
        return "pk_div_rc(" + a + ", " + hexlit(1.0 / (double)c) + ")";
    }

    std::string real(const Expr* e) {
        switch (e->kind) {
            case Expr::Num: return "((" + A + ")" + hexlit(e->num) + ")";
            case Expr::Load: {
                if (!cell_key.empty() && e->id == k.out_buf() && index_key(e->kids) == cell_key) return "cell";
                const std::string r = pre_of(e->id, e->kids);
                if (!r.empty()) {
                    if (k.buf(e->id).ty == Ty::I64) return "((" + A + ")(double)" + r + ")";
                    return "((" + A + ")" + widen(e->id, r) + ")";
                }
                if (ty_quant(k.buf(e->id).ty)) return "((" + A + ")" + quant_load(e->id, e->kids, "") + ")";
                std::string off = offset(e->id, e->kids);
                if (k.buf(e->id).ty == Ty::I64) return "((" + A + ")(double)" + ptr(e->id) + "[" + off + "])";
                return "((" + A + ")" + load_stored(e->id, off) + ")";
            }
            case Expr::Sv: return "s" + std::to_string(e->id);
            case Expr::Iv: case Expr::Si: return "((" + A + ")(double)(" + intx(e) + "))";
            case Expr::Bin: {
                static const char* ops[] = {"+", "-", "*", "/"};
                const std::string a = real(e->kids[0]);
                if (const std::string d = div_by_const(e, a); !d.empty()) return d;
                return "(" + a + " " + ops[(int)e->op] + " " + real(e->kids[1]) + ")";
            }
            case Expr::Unary: {
                std::string a = real(e->kids[0]);
                bool f = A == "float";
                switch (e->un) {
                    case Un::Neg: return "(-" + a + ")";
                    case Un::Abs: return std::string(f ? "__builtin_fabsf(" : "__builtin_fabs(") + a + ")";
                    case Un::Sqrt: return std::string(f ? "__builtin_sqrtf(" : "__builtin_sqrt(") + a + ")";
                    // f32 arithmetic: the f32 functions; f64: the double ones
                    // (exec.rs:115-130, musl's exp/log/tanh/erf/sin/cos)
                    case Un::Exp:
                        if (f && fast_fns) return used_fast = true, "pk_expf_fast(" + a + ")";
                        return std::string(f ? "pk_expf(" : "pk_exp(") + a + ")";
                    case Un::Log: return std::string(f ? "pk_logf(" : "pk_log(") + a + ")";
                    case Un::Tanh: return std::string(f ? "pk_tanhf(" : "pk_tanh(") + a + ")";
                    case Un::Erf:
                        if (f && fast_fns) return used_fast = true, "pk_erff_fast(" + a + ")";
                        return std::string(f ? "pk_erff(" : "pk_erf(") + a + ")";
                    case Un::Sin: return std::string(f ? "pk_sinf(" : "pk_sin(") + a + ")";
                    case Un::Cos: return std::string(f ? "pk_cosf(" : "pk_cos(") + a + ")";
                }
                err = "the function " + show_expr(*e) + " is not on this executor yet";
                return "0";
            }
            case Expr::Select: return "(" + boolx(e->kids[0]) + " ? " + real(e->kids[1]) + " : " + real(e->kids[2]) + ")";
            case Expr::ToF: return "((" + A + ")(double)(" + intx(e->kids[0]) + "))";
            case Expr::ToI: return "((" + A + ")(double)pk_i64((double)" + real(e->kids[0]) + "))";
            case Expr::Compare: return "((" + A + ")(long long)" + boolx(e) + ")";
            default: break;
        }
        err = "a vector expression in a scalar position: " + show_expr(*e);
        return "0";
    }

    std::string intx(const Expr* e) {
        switch (e->kind) {
            case Expr::Num:
                if (e->integral) return "(" + std::to_string(e->inum) + "LL)";
                return "pk_i64(" + hexlit(e->num) + ")";
            case Expr::Iv: return "i" + std::to_string(e->id);
            case Expr::Si: return "n" + std::to_string(e->id);
            case Expr::Load: {
                const std::string r = pre_of(e->id, e->kids);
                if (!r.empty()) {
                    if (k.buf(e->id).ty == Ty::I64) return r;
                    return "pk_i64((double)" + widen(e->id, r) + ")";
                }
                if (ty_quant(k.buf(e->id).ty)) return "pk_i64((double)((" + A + ")" + quant_load(e->id, e->kids, "") + "))";
                std::string off = offset(e->id, e->kids);
                if (k.buf(e->id).ty == Ty::I64) return ptr(e->id) + "[" + off + "]";
                return "pk_i64((double)" + load_stored(e->id, off) + ")";
            }
            case Expr::Bin:
                if (e->op == Op::Add) return "(" + intx(e->kids[0]) + " + " + intx(e->kids[1]) + ")";
                if (e->op == Op::Mul) return "(" + intx(e->kids[0]) + " * " + intx(e->kids[1]) + ")";
                break;
            case Expr::Select: return "(" + boolx(e->kids[0]) + " ? " + intx(e->kids[1]) + " : " + intx(e->kids[2]) + ")";
            case Expr::ToI: return "pk_i64((double)" + real(e->kids[0]) + ")";
            default: break;
        }
        return "pk_i64((double)" + real(e) + ")";   // exec.rs:707, a real read as an index
    }

    std::string boolx(const Expr* e) {
        if (e->kind == Expr::Compare) {
            static const char* ops[] = {"<", "<=", ">", ">=", "=="};
            return "(" + real(e->kids[0]) + " " + ops[(int)e->cmp] + " " + real(e->kids[1]) + ")";
        }
        return "(" + intx(e) + " != 0)";
    }

    // the expression of lane `l`
    std::string vec(const Expr* e) {
        switch (e->kind) {
            case Expr::Vv: return "v" + std::to_string(e->id) + "[l]";
            case Expr::VLoad: {
                if (ty_quant(k.buf(e->id).ty)) return "((" + A + ")" + quant_load(e->id, e->kids, "l") + ")";
                std::string off = offset(e->id, e->kids) + " + l";
                return "((" + A + ")" + load_stored(e->id, off) + ")";
            }
            case Expr::Splat: return real(e->kids[0]);
            case Expr::VBin: {
                static const char* ops[] = {"+", "-", "*", "/"};
                const Expr* den = e->kids[1]->kind == Expr::Splat ? e->kids[1]->kids[0] : e->kids[1];
                const std::string a = vec(e->kids[0]);
                if (const std::string d = div_by_const(e, a, den); !d.empty()) return d;
                return "(" + a + " " + ops[(int)e->op] + " " + vec(e->kids[1]) + ")";
            }
            default: return real(e);
        }
    }

    std::string store(int b, const std::string& off, const std::string& val) {
        std::string p = ptr(b);
        switch (k.buf(b).ty) {
            case Ty::F64: case Ty::F32: case Ty::I64: return p + "[" + off + "] = " + val + ";";
            case Ty::BF16: return p + "[" + off + "] = pk_f32_to_bf16(" + val + ");";
            case Ty::F16: return "{ float t_ = " + val + "; ovf |= pk_overflows_f16(t_); " + p + "[" + off + "] = pk_f32_to_f16(t_); }";
            case Ty::E8M15: return "{ float t_ = " + val + "; ovf |= pk_overflows_e8m15(t_); pk_st24(" + p + ", " + off + ", pk_f32_to_e8m15(t_)); }";
        }
        return "";
    }

    // `cell = t` as a store of t would leave it: rounded to the storage type,
    // under the overflow guard
    std::string cell_round(const std::string& t) const {
        switch (k.output.ty) {
            case Ty::F64: case Ty::F32: return "cell = " + t + ";";
            case Ty::BF16: return "cell = pk_bf16_to_f32(pk_f32_to_bf16(" + t + "));";
            case Ty::F16: return "ovf |= pk_overflows_f16(" + t + "); cell = pk_f16_to_f32(pk_f32_to_f16(" + t + "));";
            case Ty::E8M15: return "ovf |= pk_overflows_e8m15(" + t + "); cell = pk_e8m15_to_f32(pk_f32_to_e8m15(" + t + "));";
            case Ty::I64: break;
        }
        return "";
    }

    void stmts(const std::vector<const Stmt*>& body, int depth, std::string& out) {
        std::string pad(4 * depth, ' ');
        for (auto s : body) {
            switch (s->kind) {
                case Stmt::For: {
                    std::string v = "i" + std::to_string(s->var);
                    out += pad + "for (" + v + " = 0; " + v + " < " + std::to_string(s->bound) + "LL; ++" + v + ") {\n";
                    stmts(s->body, depth + 1, out);
                    out += pad + "}\n";
                    break;
                }
                case Stmt::If:
                    out += pad + "if (" + boolx(s->value) + ") {\n";
                    stmts(s->body, depth + 1, out);
                    out += pad + "}\n";
                    break;
                case Stmt::Set: out += pad + "s" + std::to_string(s->var) + " = " + real(s->value) + ";\n"; break;
                case Stmt::SetI: out += pad + "n" + std::to_string(s->var) + " = " + intx(s->value) + ";\n"; break;
                case Stmt::SetL:
                    out += pad + "{ long long t_ = " + intx(s->value) + "; i" + std::to_string(s->var) + " = t_ < 0 ? 0 : t_; }\n";
                    break;
                case Stmt::VSet: {
                    std::string L = std::to_string(k.lanes);
                    out += pad + "{ " + A + " t_[" + L + "]; for (int l = 0; l < " + L + "; ++l) t_[l] = " + vec(s->value) +
                           "; for (int l = 0; l < " + L + "; ++l) v" + std::to_string(s->var) + "[l] = t_[l]; }\n";
                    break;
                }
                case Stmt::Store: {
                    if (!post_key.empty() && s->buf == k.out_buf() && index_key(s->index) == post_key) {
                        const std::string v = real(s->value);
                        switch (k.output.ty) {
                            case Ty::BF16: out += pad + "post[u] = pk_f32_to_bf16(" + v + ");\n"; break;
                            case Ty::F16:
                                out += pad + "{ float t_ = " + v + "; ovf |= pk_overflows_f16(t_); post[u] = pk_f32_to_f16(t_); }\n";
                                break;
                            default: out += pad + "post[u] = " + v + ";\n"; break;
                        }
                        break;
                    }
                    if (!cell_key.empty() && s->buf == k.out_buf() && index_key(s->index) == cell_key) {
                        out += pad + "{ " + A + " t_ = " + real(s->value) + "; " + cell_round("t_") + " stored = true; }\n";
                        break;
                    }
                    std::string off = offset(s->buf, s->index);
                    bool idx = k.buf(s->buf).ty == Ty::I64;
                    out += pad + store(s->buf, off, idx ? intx(s->value) : real(s->value)) + "\n";
                    break;
                }
                case Stmt::VStore: {
                    std::string L = std::to_string(k.lanes), off = offset(s->buf, s->index);
                    out += pad + "{ " + A + " w_[" + L + "]; for (int l = 0; l < " + L + "; ++l) w_[l] = " + vec(s->value) + ";\n";
                    out += pad + "  for (int l = 0; l < " + L + "; ++l) " + store(s->buf, off + " + l", "w_[l]") + " }\n";
                    break;
                }
            }
        }
    }
};

// Variables a statement list reads before it writes them (in execution order;
// writes under an `if` are not definite).  Keys: 'i'/'s'/'n'/'v' + number.
void exposed(const std::vector<const Stmt*>& body, std::set<std::string>& defined, std::set<std::string>& out) {
    std::function<void(const Expr*)> ex = [&](const Expr* e) {
        std::string key;
        switch (e->kind) {
            case Expr::Iv: key = "i"; break;
            case Expr::Sv: key = "s"; break;
            case Expr::Si: key = "n"; break;
            case Expr::Vv: key = "v"; break;
            default: break;
        }
        if (!key.empty()) {
            key += std::to_string(e->id);
            if (!defined.count(key)) out.insert(key);
        }
        for (auto c : e->kids) ex(c);
    };
    for (auto s : body) {
        switch (s->kind) {
            case Stmt::For: {
                std::string key = "i" + std::to_string(s->var);
                bool had = defined.count(key);
                defined.insert(key);
                exposed(s->body, defined, out);
                if (!had && s->bound == 0) defined.erase(key);
                break;
            }
            case Stmt::If: {
                ex(s->value);
                std::set<std::string> inner = defined;
                exposed(s->body, inner, out);
                break;
            }
            case Stmt::Store: case Stmt::VStore:
                for (auto e : s->index) ex(e);
                ex(s->value);
                break;
            default: {
                ex(s->value);
                char c = s->kind == Stmt::Set ? 's' : s->kind == Stmt::SetI ? 'n' : s->kind == Stmt::SetL ? 'i' : 'v';
                defined.insert(std::string(1, c) + std::to_string(s->var));
            }
        }
    }
}

std::set<std::string> writes(const std::vector<const Stmt*>& body) {
    std::set<std::string> w;
    std::function<void(const std::vector<const Stmt*>&)> walk = [&](const std::vector<const Stmt*>& b) {
        for (auto s : b) {
            switch (s->kind) {
                case Stmt::For: w.insert("i" + std::to_string(s->var)); walk(s->body); break;
                case Stmt::If: walk(s->body); break;
                case Stmt::Set: w.insert("s" + std::to_string(s->var)); break;
                case Stmt::SetI: w.insert("n" + std::to_string(s->var)); break;
                case Stmt::SetL: w.insert("i" + std::to_string(s->var)); break;
                case Stmt::VSet: w.insert("v" + std::to_string(s->var)); break;
                default: break;
            }
        }
    };
    walk(body);
    return w;
}

// An index expression as sum_v c_v * i_v + c over loop variables, if it is one.
struct Affine {
    std::map<int, int64_t> coef;
    int64_t c = 0;
    bool ok = true;
};

Affine affine_of(const Expr* e) {
    Affine a;
    switch (e->kind) {
        case Expr::Num:
            if (e->integral) a.c = e->inum;
            else a.ok = false;
            return a;
        case Expr::Iv: a.coef[e->id] = 1; return a;
        case Expr::Bin: {
            Affine x = affine_of(e->kids[0]), y = affine_of(e->kids[1]);
            if (!x.ok || !y.ok) { a.ok = false; return a; }
            if (e->op == Op::Add) {
                a = x;
                for (auto& kv : y.coef) a.coef[kv.first] += kv.second;
                a.c += y.c;
                return a;
            }
            if (e->op == Op::Mul) {
                const Affine* v = nullptr;
                int64_t f = 0;
                if (x.coef.empty()) { f = x.c; v = &y; }
                else if (y.coef.empty()) { f = y.c; v = &x; }
                else { a.ok = false; return a; }
                a = *v;
                for (auto& kv : a.coef) kv.second *= f;
                a.c *= f;
                return a;
            }
            a.ok = false;
            return a;
        }
        default: a.ok = false; return a;
    }
}

// Every access to the output in `body`: (index list, is a vector access).
void output_accesses(const Kernel& k, const std::vector<const Stmt*>& body,
                     std::vector<std::pair<const std::vector<const Expr*>*, bool>>& acc) {
    std::function<void(const Expr*)> ex = [&](const Expr* e) {
        if ((e->kind == Expr::Load || e->kind == Expr::VLoad) && e->id == k.out_buf()) acc.push_back({&e->kids, e->kind == Expr::VLoad});
        for (auto c : e->kids) ex(c);
    };
    for (auto s : body) {
        if ((s->kind == Stmt::Store || s->kind == Stmt::VStore) && s->buf == k.out_buf())
            acc.push_back({&s->index, s->kind == Stmt::VStore});
        for (auto e : s->index) ex(e);
        if (s->value) ex(s->value);
        output_accesses(k, s->body, acc);
    }
}

// Whether every access to the output in `body` is a scalar element whose
// index moves by exactly one element when loop `var` does, in its last
// position only: consecutive iterations of `var` write consecutive elements.
bool output_unit_stride(const Kernel& k, const std::vector<const Stmt*>& body, int var) {
    std::vector<std::pair<const std::vector<const Expr*>*, bool>> acc;
    output_accesses(k, body, acc);
    if (acc.empty()) return false;
    for (auto& a : acc) {
        if (a.second || a.first->empty()) return false;
        const auto& ix = *a.first;
        for (size_t p = 0; p < ix.size(); ++p) {
            Affine f = affine_of(ix[p]);
            if (!f.ok) return false;
            const int64_t c = f.coef.count(var) ? f.coef[var] : 0;
            if (c != (p + 1 == ix.size() ? 1 : 0)) return false;
        }
    }
    return true;
}

// Storage bytes and C element type of a buffer's elements.
int elem_bytes(Ty t) {
    switch (t) {
        case Ty::F64: case Ty::I64: return 8;
        case Ty::F32: return 4;
        case Ty::BF16: case Ty::F16: return 2;
        case Ty::E8M15: return 3;
        case Ty::Q8: case Ty::Q4: return 1;
    }
    return 0;
}
const char* elem_type(Ty t) {
    switch (t) {
        case Ty::F64: return "double";
        case Ty::F32: return "float";
        case Ty::BF16: case Ty::F16: return "unsigned short";
        case Ty::I64: return "long long";
        case Ty::E8M15: case Ty::Q4: return "unsigned char";
        case Ty::Q8: return "signed char";
    }
    return "";
}

// Whether an index list, affine over the loops of `bounds` alone, stays in
// buffer b's shape over all their iterations (so the element may be read
// whether or not the nest reads it).
bool in_bounds(const Kernel& k, int b, const std::vector<const Expr*>& ix, const std::map<int, int64_t>& bounds) {
    const auto& dims = k.buf(b).dims;
    if (ix.size() != dims.size()) return false;
    for (size_t p = 0; p < ix.size(); ++p) {
        Affine f = affine_of(ix[p]);
        if (!f.ok) return false;
        int64_t lo = f.c, hi = f.c;
        for (auto& kv : f.coef) {
            auto it = bounds.find(kv.first);
            if (it == bounds.end()) return false;
            const int64_t span = kv.second * (it->second - 1);
            (span < 0 ? lo : hi) += span;
        }
        if (lo < 0 || hi >= dims[p]) return false;
    }
    return true;
}

// The loads of an expression tree.
void loads_of(const Expr* e, std::vector<const Expr*>& out) {
    if (e->kind == Expr::Load) out.push_back(e);
    for (auto c : e->kids) loads_of(c, out);
}

// The loops of `chain` that one output index, shared by every access to the
// output, maps injectively: each index position that is an affine function
// of chain loops alone, whose coefficients form a mixed radix over the loops'
// bounds (c_1 = 1 >= ..., each c_j > sum of the smaller c_i (n_i - 1)), makes
// its loops distinguishable.  Two iterations that differ in such a loop then
// touch different elements -- a sufficient condition for running them on
// different threads, wider than `writes_disjoint`'s c*v + t form (it takes
// `hh*hd + d` of merge_heads).
std::set<int> injective_loops(const Kernel& k, const std::vector<const Stmt*>& chain, const std::vector<const Stmt*>& body) {
    std::set<int> out;
    std::vector<std::pair<const std::vector<const Expr*>*, bool>> acc;
    output_accesses(k, body, acc);
    if (acc.empty()) return out;
    const std::string key = index_key(*acc[0].first);
    for (auto& a : acc)
        if (a.second || index_key(*a.first) != key) return out;
    std::map<int, int64_t> bound;
    for (auto l : chain) bound[l->var] = l->bound;
    for (auto e : *acc[0].first) {
        Affine a = affine_of(e);
        if (!a.ok || a.coef.empty()) continue;
        std::vector<std::pair<int64_t, int>> terms;
        bool mine = true;
        for (auto& kv : a.coef) {
            if (!bound.count(kv.first) || kv.second <= 0) mine = false;
            terms.push_back({kv.second, kv.first});
        }
        if (!mine) continue;
        std::sort(terms.begin(), terms.end());
        int64_t reach = 0;   // the largest value the smaller terms add
        bool radix = true;
        for (auto& t : terms) {
            if (t.first <= reach) radix = false;
            reach += t.first * (bound[t.second] - 1);
        }
        if (!radix) continue;
        for (auto& t : terms) out.insert(t.second);
    }
    return out;
}

// Whether every access to the output in `body` is the scalar element at one
// index built from the loops `grid` alone: that element is the thread's own,
// and it may live in a register across the thread's sequential loops.
bool owns_one_element(const Kernel& k, const std::vector<const Stmt*>& body, const std::set<int>& grid, std::string* key) {
    std::vector<std::pair<const std::vector<const Expr*>*, bool>> acc;
    output_accesses(k, body, acc);
    if (acc.empty() || k.output.ty == Ty::I64) return false;
    *key = index_key(*acc[0].first);
    for (auto& a : acc)
        if (a.second || index_key(*a.first) != *key) return false;
    for (auto e : *acc[0].first) {
        Affine a = affine_of(e);
        if (!a.ok) return false;
        for (auto& kv : a.coef)
            if (!grid.count(kv.first)) return false;
    }
    return true;
}

}  // namespace

bool generate_hip(const Kernel& k, Generated* out, std::string* err, bool fast_fns) {
    if (!k.arith.empty()) {
        *err = "E7005: the kernel `" + k.name + "` rounds to formats other than its storage type's arithmetic (" + k.arith +
               "); the kernel interpreter emulates those";
        return false;
    }
    if ((int)k.inputs.size() + 1 + k.n_quant() > kMaxBufs) {
        *err = "E10001: more than " + std::to_string(kMaxBufs) + " buffers and scales";
        return false;
    }
    Printer P(k);
    P.fast_fns = fast_fns;
    // The phases: each top-level statement its own launch when none reads a
    // variable an earlier one wrote; otherwise one sequential phase.
    std::vector<std::vector<const Stmt*>> groups;
    {
        bool independent = k.body.size() > 1;
        std::set<std::string> before;
        for (size_t i = 0; i < k.body.size() && independent; ++i) {
            std::set<std::string> def, exp;
            exposed({k.body[i]}, def, exp);
            for (auto& v : exp)
                if (before.count(v)) independent = false;
            if (k.body[i]->kind != Stmt::For) independent = false;
            auto w = writes({k.body[i]});
            before.insert(w.begin(), w.end());
        }
        if (independent)
            for (auto s : k.body) groups.push_back({s});
        else
            groups.push_back(k.body);
    }
    const int64_t split_bound = parallel_outer(k);
    std::string src = "#include \"devfmt.hpp\"\n";
    src += "struct PkArgs { void* buf[" + std::to_string(kMaxBufs) + "]; unsigned* flag; long long lo, hi; };\n";
    src += "typedef unsigned int pk_u32x4 __attribute__((ext_vector_type(4)));\n";
    int index = 0;
    for (auto& g : groups) {
        Phase ph;
        // named after the nest, for profiles: pk_<name>_p<phase>
        std::string tag;
        for (char c : k.name) tag += std::isalnum((unsigned char)c) ? c : '_';
        if (tag.size() > 40) tag.resize(40);
        ph.fn = "pk_" + tag + "_p" + std::to_string(index++);
        // The grid: the loops of the perfect nest at the top of the group whose
        // iterations write disjoint output elements (ir.rs:375-492).  When the
        // nest's innermost body carries no scalar from one iteration to the
        // next, every such loop goes to the grid wherever it sits in the nest,
        // and the others run in their order inside each thread (`sum_to`'s
        // and `embed_vjp`'s column loops are promoted past their token
        // loops): each output element is still updated by the same statements
        // in the same order.  Otherwise only the disjoint prefix goes to the
        // grid.
        std::vector<const Stmt*> chain;
        const std::vector<const Stmt*>* level = &g;
        while (level->size() == 1 && (*level)[0]->kind == Stmt::For) {
            chain.push_back((*level)[0]);
            level = &(*level)[0]->body;
        }
        std::vector<const Stmt*> loops, serial;
        bool whole = !chain.empty();
        {
            std::set<std::string> def, exp;
            for (auto l : chain) def.insert("i" + std::to_string(l->var));
            exposed(*level, def, exp);
            whole = whole && exp.empty();
        }
        if (whole) {
            const std::set<int> inj = injective_loops(k, chain, *level);
            for (auto f : chain) (writes_disjoint(k, f->var, f->body) || inj.count(f->var) ? loops : serial).push_back(f);
        } else {
            loops.clear();
            const std::vector<const Stmt*>* lv = &g;
            while (lv->size() == 1 && (*lv)[0]->kind == Stmt::For) {
                const Stmt* f = (*lv)[0];
                if (!writes_disjoint(k, f->var, f->body)) break;
                std::set<std::string> def, exp;
                for (auto l : loops) def.insert("i" + std::to_string(l->var));
                def.insert("i" + std::to_string(f->var));
                exposed(f->body, def, exp);
                if (!exp.empty()) break;
                loops.push_back(f);
                lv = &f->body;
            }
            level = lv;
        }
        ph.split = !loops.empty() && groups.size() == 1 && split_bound >= 0 && loops[0] == k.body[0];
        // Each thread takes VEC consecutive iterations of the innermost grid
        // loop when the nest is all grid (no loop left in the thread) and
        // those iterations write consecutive output elements: the loads and
        // stores of the unrolled iterations merge into 16-byte accesses.
        // The iterations are independent, so running them in one thread in
        // order changes nothing.
        // A nest too small to fill the CUs a thread an iteration (under 64 K
        // iterations a VEC, e.g. RoPE's sin and cos over 2 048 x 64) is
        // latency-bound, not bandwidth-bound: it keeps a thread an iteration.
        int vec = 1;
        if (!loops.empty() && serial.empty() && !(loops.size() == 1 && ph.split)) {
            const int want = k.output.ty == Ty::F32 ? 4 : (k.output.ty == Ty::BF16 || k.output.ty == Ty::F16) ? 8 : 1;
            const Stmt* inner = loops.back();
            double iters = 1;
            for (auto l : loops) iters *= (double)l->bound;
            if (want > 1 && iters >= 65536.0 * want && inner->bound % want == 0 && output_unit_stride(k, *level, inner->var))
                vec = want;
        }
        for (auto l : loops) ph.bounds.push_back(l->bound);
        if (vec > 1) ph.bounds.back() /= vec;
        std::string body;
        body += "__device__ __forceinline__ void " + ph.fn + "_body(const PkArgs& a" + P.ptr_params() + ") {\n";
        for (int v = 0; v < k.nloops; ++v) body += "    long long i" + std::to_string(v) + " = 0; (void)i" + std::to_string(v) + ";\n";
        for (int v = 0; v < k.nreal; ++v) body += "    " + P.A + " s" + std::to_string(v) + " = 0; (void)s" + std::to_string(v) + ";\n";
        for (int v = 0; v < k.nint; ++v) body += "    long long n" + std::to_string(v) + " = 0; (void)n" + std::to_string(v) + ";\n";
        for (int v = 0; v < k.nvec; ++v)
            body += "    " + P.A + " v" + std::to_string(v) + "[" + std::to_string(k.lanes) + "] = {}; (void)v" + std::to_string(v) + ";\n";
        body += "    bool ovf = false; (void)ovf;\n";
        if (!loops.empty()) {
            body += "    long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;\n";
            // the outermost loop runs over [lo, hi) when split, else its bound
            const int vec0 = loops.size() == 1 ? vec : 1;  // the outermost loop is also the innermost
            // (named apart from the nest's own integer scalars n<k>)
            body += "    const long long grid_n0 = " + std::string(ph.split ? "a.hi - a.lo" : std::to_string(loops[0]->bound / vec0) + "LL") + ";\n";
            std::string total = "grid_n0";
            for (size_t d = 1; d < loops.size(); ++d)
                total += " * " + std::to_string(d + 1 == loops.size() ? loops[d]->bound / vec : loops[d]->bound) + "LL";
            body += "    if (t >= " + total + ") return;\n";
            for (size_t d = loops.size(); d-- > 1;) {
                std::string b = std::to_string(d + 1 == loops.size() ? loops[d]->bound / vec : loops[d]->bound) + "LL";
                body += "    i" + std::to_string(loops[d]->var) + " = t % " + b + (d + 1 == loops.size() && vec > 1 ? " * " + std::to_string(vec) + "LL" : "") + "; t /= " + b + ";\n";
            }
            body += "    i" + std::to_string(loops[0]->var) + " = t" + (vec0 > 1 ? " * " + std::to_string(vec0) + "LL" : "") + (ph.split ? " + a.lo" : "") + ";\n";
            // the loops left in the thread, in their order around the body;
            // the thread's own output element in a register across them
            std::set<int> grid;
            for (auto l : loops) grid.insert(l->var);
            std::string key;
            const bool cell = !serial.empty() && owns_one_element(k, *level, grid, &key);
            std::vector<const Expr*> cell_ix;
            if (cell) {
                std::vector<std::pair<const std::vector<const Expr*>*, bool>> acc;
                output_accesses(k, *level, acc);
                cell_ix = *acc[0].first;
                body += "    " + P.A + " cell = ((" + P.A + ")" + P.load_stored(k.out_buf(), P.offset(k.out_buf(), cell_ix)) + ");\n";
                body += "    bool stored = false;\n";
                P.cell_key = key;
            }
            std::string close;
            int depth = 1;
            for (auto f : serial) {
                std::string pad(4 * depth, ' '), v = "i" + std::to_string(f->var);
                body += pad + "for (" + v + " = 0; " + v + " < " + std::to_string(f->bound) + "LL; ++" + v + ") {\n";
                close = pad + "}\n" + close;
                ++depth;
            }
            if (vec > 1) {
                const int iv = loops.back()->var;
                const std::string v = "i" + std::to_string(iv), V = std::to_string(vec);
                body += "    const long long " + v + "_0 = " + v + ";\n";
                // Read ahead: each input element the iterations read at unit
                // stride along the coarsened loop, whose index is affine in
                // the grid loops and in bounds over all of them, is loaded for
                // all VEC iterations at once (16-byte loads when aligned).
                std::map<int, int64_t> gb;
                for (auto l : loops) gb[l->var] = l->bound;
                std::vector<const Expr*> lds;
                for (auto st : *level) {
                    if (st->kind == Stmt::For || st->kind == Stmt::If) continue;
                    for (auto e : st->index) loads_of(e, lds);
                    if (st->value) loads_of(st->value, lds);
                }
                for (auto e : lds) {
                    const int b = e->id;
                    const Ty ty = k.buf(b).ty;
                    if (b == k.out_buf() || ty == Ty::E8M15 || ty_quant(ty) || !in_bounds(k, b, e->kids, gb)) continue;
                    bool unit = !e->kids.empty();  // (a scalar buffer is the same element for every u)
                    for (size_t p = 0; p < e->kids.size(); ++p) {
                        Affine f = affine_of(e->kids[p]);
                        const int64_t c = f.coef.count(iv) ? f.coef[iv] : 0;
                        if (c != (p + 1 == e->kids.size() ? 1 : 0)) unit = false;
                    }
                    const std::string key = std::to_string(b) + "|" + index_key(e->kids);
                    if (!unit || P.pre.count(key)) continue;
                    const int n = (int)P.pre.size();
                    const std::string T = elem_type(ty), pn = "pre" + std::to_string(n);
                    const int bytes = vec * elem_bytes(ty);
                    body += "    " + T + " " + pn + "[" + V + "];\n";
                    body += "    { const " + T + "* p_ = " + P.ptr(b) + " + " + P.offset(b, e->kids) + ";\n";
                    if (bytes % 16 == 0) {
                        body += "      if ((((unsigned long long)p_) & 15ULL) == 0) {\n";
                        body += "#pragma unroll\n        for (int c = 0; c < " + std::to_string(bytes / 16) +
                                "; ++c) { pk_u32x4 w_ = ((const pk_u32x4*)p_)[c]; __builtin_memcpy((char*)" + pn + " + 16 * c, &w_, 16); }\n";
                        body += "      } else {\n#pragma unroll\n        for (int u = 0; u < " + V + "; ++u) " + pn + "[u] = p_[u];\n      }\n";
                    } else {
                        body += "#pragma unroll\n      for (int u = 0; u < " + V + "; ++u) " + pn + "[u] = p_[u];\n";
                    }
                    body += "    }\n";
                    P.pre[key] = n;
                }
                // The one store of the output, unconditional and read by
                // nothing: buffered and written back in 16-byte stores.
                std::vector<std::pair<const std::vector<const Expr*>*, bool>> oacc;
                output_accesses(k, *level, oacc);
                const Stmt* ost = nullptr;
                for (auto st : *level)
                    if (st->kind == Stmt::Store && st->buf == k.out_buf()) ost = st;
                const bool post = oacc.size() == 1 && ost && (elem_bytes(k.output.ty) * vec) % 16 == 0;
                const std::string OT = elem_type(k.output.ty);
                if (post) {
                    P.post_key = index_key(ost->index);
                    body += "    " + OT + " post[" + V + "];\n";
                    body += "    const long long o_ = " + P.offset(k.out_buf(), ost->index) + ";\n";
                }
                body += "#pragma unroll\n    for (int u = 0; u < " + V + "; ++u) {\n";
                body += "    " + v + " = " + v + "_0 + u;\n";
                P.stmts(*level, depth + 1, body);
                body += "    }\n";
                if (post) {
                    const int chunks = elem_bytes(k.output.ty) * vec / 16;
                    body += "    { " + OT + "* p_ = " + P.ptr(k.out_buf()) + " + o_;\n";
                    body += "      if ((((unsigned long long)p_) & 15ULL) == 0) {\n";
                    body += "#pragma unroll\n        for (int c = 0; c < " + std::to_string(chunks) +
                            "; ++c) { pk_u32x4 w_; __builtin_memcpy(&w_, (const char*)post + 16 * c, 16); ((pk_u32x4*)p_)[c] = w_; }\n";
                    body += "      } else {\n#pragma unroll\n        for (int u = 0; u < " + V + "; ++u) p_[u] = post[u];\n      }\n    }\n";
                }
                P.pre.clear();
                P.post_key.clear();
            } else {
                P.stmts(*level, depth, body);
            }
            body += close;
            if (cell) {
                P.cell_key.clear();
                // the value is already the stored one: converting it back is exact
                std::string off = P.offset(k.out_buf(), cell_ix), val;
                switch (k.output.ty) {
                    case Ty::BF16: val = "pk_f32_to_bf16(cell)"; break;
                    case Ty::F16: val = "pk_f32_to_f16(cell)"; break;
                    default: val = "cell"; break;
                }
                if (k.output.ty == Ty::E8M15)
                    body += "    if (stored) pk_st24(" + P.ptr(k.out_buf()) + ", " + off + ", pk_f32_to_e8m15(cell));\n";
                else
                    body += "    if (stored) " + P.ptr(k.out_buf()) + "[" + off + "] = " + val + ";\n";
            }
        } else {
            body += "    if (blockIdx.x != 0 || threadIdx.x != 0) return;\n";
            P.stmts(g, 1, body);
        }
        if (k.guarded()) body += "    if (ovf) atomicOr(a.flag, 1u);\n";
        body += "}\n";
        body += "extern \"C\" __global__ void __launch_bounds__(256) " + ph.fn + "(PkArgs a) { " + ph.fn + "_body(a" + P.ptr_args() + "); }\n";
        src += body;
        out->phases.push_back(ph);
    }
    if (!P.err.empty()) {
        *err = "E10001: " + P.err;
        return false;
    }
    out->src = src;
    out->fast_fns = P.used_fast;
    return true;
}

}  // namespace presk
