// The generic HIP printer (see hipgen.hpp).
#include "hipgen.hpp"

#include <cmath>
#include <cstdio>
#include <functional>
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

struct Printer {
    const Kernel& k;
    std::string A;              // arithmetic type
    std::vector<std::vector<int64_t>> strides;
    std::string err;

    explicit Printer(const Kernel& k) : k(k) {
        A = k.dtype == Ty::F64 ? "double" : "float";
        for (size_t b = 0; b <= k.inputs.size(); ++b) strides.push_back(k.buf((int)b).strides());
    }

    std::string ptr(int b) const {
        const BufSpec& s = k.buf(b);
        const char* c = b == k.out_buf() ? "" : "const ";
        switch (s.ty) {
            case Ty::F64: return std::string("((") + c + "double*)a.buf[" + std::to_string(b) + "])";
            case Ty::F32: return std::string("((") + c + "float*)a.buf[" + std::to_string(b) + "])";
            case Ty::BF16: case Ty::F16: return std::string("((") + c + "unsigned short*)a.buf[" + std::to_string(b) + "])";
            case Ty::E8M15: return std::string("((") + c + "unsigned char*)a.buf[" + std::to_string(b) + "])";
            case Ty::I64: return std::string("((") + c + "long long*)a.buf[" + std::to_string(b) + "])";
        }
        return "";
    }

    std::string offset(int b, const std::vector<const Expr*>& ix) {
        std::string s = "(0LL";
        for (size_t p = 0; p < ix.size() && p < strides[b].size(); ++p)
            s += " + (" + intx(ix[p]) + ")*" + std::to_string(strides[b][p]) + "LL";
        return s + ")";
    }

    // element `off` of buffer b widened exactly to its own arithmetic type
    std::string load_stored(int b, const std::string& off) {
        switch (k.buf(b).ty) {
            case Ty::F64: case Ty::F32: return ptr(b) + "[" + off + "]";
            case Ty::BF16: return "pk_bf16_to_f32(" + ptr(b) + "[" + off + "])";
            case Ty::F16: return "pk_f16_to_f32(" + ptr(b) + "[" + off + "])";
            case Ty::E8M15: return "pk_e8m15_to_f32(pk_ld24(" + ptr(b) + ", " + off + "))";
            case Ty::I64: return "((double)" + ptr(b) + "[" + off + "])";
        }
        return "";
    }

    std::string real(const Expr* e) {
        switch (e->kind) {
            case Expr::Num: return "((" + A + ")" + hexlit(e->num) + ")";
            case Expr::Load: {
                std::string off = offset(e->id, e->kids);
                if (k.buf(e->id).ty == Ty::I64) return "((" + A + ")(double)" + ptr(e->id) + "[" + off + "])";
                return "((" + A + ")" + load_stored(e->id, off) + ")";
            }
            case Expr::Sv: return "s" + std::to_string(e->id);
            case Expr::Iv: case Expr::Si: return "((" + A + ")(double)(" + intx(e) + "))";
            case Expr::Bin: {
                static const char* ops[] = {"+", "-", "*", "/"};
                return "(" + real(e->kids[0]) + " " + ops[(int)e->op] + " " + real(e->kids[1]) + ")";
            }
            case Expr::Unary: {
                std::string a = real(e->kids[0]);
                bool f = A == "float";
                switch (e->un) {
                    case Un::Neg: return "(-" + a + ")";
                    case Un::Abs: return std::string(f ? "__builtin_fabsf(" : "__builtin_fabs(") + a + ")";
                    case Un::Sqrt: return std::string(f ? "__builtin_sqrtf(" : "__builtin_sqrt(") + a + ")";
                    case Un::Exp: if (f) return "pk_expf(" + a + ")"; break;
                    case Un::Log: if (f) return "pk_logf(" + a + ")"; break;
                    case Un::Tanh: if (f) return "pk_tanhf(" + a + ")"; break;
                    case Un::Erf: if (f) return "pk_erff(" + a + ")"; break;
                    case Un::Sin: case Un::Cos: break;
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
                std::string off = offset(e->id, e->kids) + " + l";
                return "((" + A + ")" + load_stored(e->id, off) + ")";
            }
            case Expr::Splat: return real(e->kids[0]);
            case Expr::VBin: {
                static const char* ops[] = {"+", "-", "*", "/"};
                return "(" + vec(e->kids[0]) + " " + ops[(int)e->op] + " " + vec(e->kids[1]) + ")";
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

}  // namespace

bool generate_hip(const Kernel& k, Generated* out, std::string* err) {
    if (!k.arith.empty()) {
        *err = "E7005: the kernel `" + k.name + "` rounds to formats other than its storage type's arithmetic (" + k.arith +
               "); the kernel interpreter emulates those";
        return false;
    }
    if ((int)k.inputs.size() + 1 > kMaxBufs) {
        *err = "E10001: more than " + std::to_string(kMaxBufs - 1) + " inputs";
        return false;
    }
    Printer P(k);
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
    int index = 0;
    for (auto& g : groups) {
        Phase ph;
        ph.fn = "pk_phase" + std::to_string(index++);
        // the perfect nest of parallel loops at the top of the group
        std::vector<const Stmt*> loops;
        const std::vector<const Stmt*>* level = &g;
        while (level->size() == 1 && (*level)[0]->kind == Stmt::For) {
            const Stmt* f = (*level)[0];
            if (!writes_disjoint(k, f->var, f->body)) break;
            // no scalar may flow from one iteration to the next
            std::set<std::string> def, exp;
            for (auto l : loops) def.insert("i" + std::to_string(l->var));
            def.insert("i" + std::to_string(f->var));
            exposed(f->body, def, exp);
            if (!exp.empty()) break;
            loops.push_back(f);
            level = &f->body;
        }
        for (auto l : loops) ph.bounds.push_back(l->bound);
        ph.split = !loops.empty() && groups.size() == 1 && split_bound >= 0 && loops[0] == k.body[0];
        std::string body;
        body += "extern \"C\" __global__ void __launch_bounds__(256) " + ph.fn + "(PkArgs a) {\n";
        for (int v = 0; v < k.nloops; ++v) body += "    long long i" + std::to_string(v) + " = 0; (void)i" + std::to_string(v) + ";\n";
        for (int v = 0; v < k.nreal; ++v) body += "    " + P.A + " s" + std::to_string(v) + " = 0; (void)s" + std::to_string(v) + ";\n";
        for (int v = 0; v < k.nint; ++v) body += "    long long n" + std::to_string(v) + " = 0; (void)n" + std::to_string(v) + ";\n";
        for (int v = 0; v < k.nvec; ++v)
            body += "    " + P.A + " v" + std::to_string(v) + "[" + std::to_string(k.lanes) + "] = {}; (void)v" + std::to_string(v) + ";\n";
        body += "    bool ovf = false; (void)ovf;\n";
        if (!loops.empty()) {
            body += "    long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;\n";
            // the outermost loop runs over [lo, hi) when split, else its bound
            body += "    const long long n0 = " + std::string(ph.split ? "a.hi - a.lo" : std::to_string(loops[0]->bound) + "LL") + ";\n";
            std::string total = "n0";
            for (size_t d = 1; d < loops.size(); ++d) total += " * " + std::to_string(loops[d]->bound) + "LL";
            body += "    if (t >= " + total + ") return;\n";
            for (size_t d = loops.size(); d-- > 1;) {
                std::string b = std::to_string(loops[d]->bound) + "LL";
                body += "    i" + std::to_string(loops[d]->var) + " = t % " + b + "; t /= " + b + ";\n";
            }
            body += "    i" + std::to_string(loops[0]->var) + " = t" + (ph.split ? " + a.lo" : "") + ";\n";
            P.stmts(*level, 1, body);
        } else {
            body += "    if (blockIdx.x != 0 || threadIdx.x != 0) return;\n";
            P.stmts(g, 1, body);
        }
        if (k.guarded()) body += "    if (ovf) atomicOr(a.flag, 1u);\n";
        body += "}\n";
        src += body;
        out->phases.push_back(ph);
    }
    if (!P.err.empty()) {
        *err = "E10001: " + P.err;
        return false;
    }
    out->src = src;
    return true;
}

}  // namespace presk
