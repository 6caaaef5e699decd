// Reader and printer of PSK-Kernel text (crates/presk-kernel/src/ir.rs:495-595)
// and the two parallel-loop analyses the executor maps to the HIP grid
// (ir.rs:336-492).
#include "ir.hpp"

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <sstream>
#include <stdexcept>

namespace presk {

const char* ty_name(Ty t) {
    switch (t) {
        case Ty::F64: return "f64";
        case Ty::F32: return "f32";
        case Ty::BF16: return "bf16";
        case Ty::F16: return "f16";
        case Ty::E8M15: return "e8m15";
        case Ty::I64: return "i64";
        case Ty::Q8: return "int8";
        case Ty::Q4: return "int4";
    }
    return "?";
}

bool ty_parse(const std::string& s, Ty* out) {
    static const std::pair<const char*, Ty> table[] = {{"f64", Ty::F64}, {"f32", Ty::F32}, {"bf16", Ty::BF16},
                                                        {"f16", Ty::F16}, {"e8m15", Ty::E8M15}, {"i64", Ty::I64}};
    for (auto& p : table)
        if (s == p.first) { *out = p.second; return true; }
    return false;
}

int ty_bytes(Ty t) {
    switch (t) {
        case Ty::F64: case Ty::I64: return 8;
        case Ty::F32: return 4;
        case Ty::BF16: case Ty::F16: return 2;
        case Ty::E8M15: return 3;
        case Ty::Q8: case Ty::Q4: return 1;
    }
    return 0;
}

bool ty_real(Ty t) { return t != Ty::I64; }
bool ty_quant(Ty t) { return t == Ty::Q8 || t == Ty::Q4; }
bool ty_coded(Ty t) { return t == Ty::F16 || t == Ty::E8M15; }

// Precision rank of a real type: a buffer of lower rank than the kernel's type
// is `BufKind::Wide` (ir.rs:31-49).
static int ty_rank(Ty t) {
    switch (t) {
        case Ty::F64: return 3;
        case Ty::F32: return 2;
        default: return 1;  // bf16, f16, e8m15: storage types of f32 arithmetic
    }
}

int64_t BufSpec::numel() const {
    int64_t n = 1;
    for (auto d : dims) n *= d;
    return n;
}

std::vector<int64_t> BufSpec::strides() const {
    std::vector<int64_t> s(dims.size(), 1);
    for (int i = (int)dims.size() - 2; i >= 0; --i) s[i] = s[i + 1] * dims[i + 1];
    return s;
}

std::vector<int64_t> BufSpec::scale_strides() const {
    std::vector<int64_t> s(dims.size(), 0);
    if (!ty_quant(ty)) return s;
    int64_t acc = 1;
    for (int a = (int)dims.size() - 1; a >= 0; --a)
        if (!(a >= qover && a < qover + qspan)) {
            s[a] = acc;
            acc *= dims[a];
        }
    return s;
}

int64_t BufSpec::scale_count() const {
    int64_t n = 1;
    for (int a = 0; a < (int)dims.size(); ++a)
        if (!(a >= qover && a < qover + qspan)) n *= dims[a];
    return n;
}

int Kernel::scale_slot(int b) const {
    if (b < 0 || b >= (int)inputs.size() || !ty_quant(inputs[b].ty)) return -1;
    int slot = out_buf() + 1;
    for (int i = 0; i < b; ++i) slot += ty_quant(inputs[i].ty) ? 1 : 0;
    return slot;
}

int Kernel::n_quant() const {
    int n = 0;
    for (auto& b : inputs) n += ty_quant(b.ty) ? 1 : 0;
    return n;
}

namespace {

struct ParseError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

// ---- tokens ----------------------------------------------------------------
struct Lexer {
    std::vector<std::string> toks;
    size_t pos = 0;

    explicit Lexer(const std::string& s) {
        size_t i = 0, n = s.size();
        auto starts = [&](const char* p) { return s.compare(i, std::strlen(p), p) == 0; };
        while (i < n) {
            char c = s[i];
            if (c == ' ') { ++i; continue; }
            const char* multi[] = {"<v=", "<v>", "<=", ">=", "==", ".."};
            bool hit = false;
            for (auto m : multi)
                if (starts(m)) { toks.emplace_back(m); i += std::strlen(m); hit = true; break; }
            if (hit) continue;
            // numbers: -?digits(.digits)?, inf, -inf, NaN (a Sub is always spaced)
            if (std::isdigit((unsigned char)c) || (c == '-' && i + 1 < n && (std::isdigit((unsigned char)s[i + 1]) || s[i + 1] == 'i'))) {
                size_t j = i + 1;
                if (c == '-' && s[j] == 'i') {
                    j += 3;  // -inf
                } else {
                    while (j < n && std::isdigit((unsigned char)s[j])) ++j;
                    if (j + 1 < n && s[j] == '.' && std::isdigit((unsigned char)s[j + 1])) {
                        ++j;
                        while (j < n && std::isdigit((unsigned char)s[j])) ++j;
                    }
                }
                toks.push_back(s.substr(i, j - i));
                i = j;
                continue;
            }
            if (c == '%') {
                size_t j = i + 1;
                while (j < n && std::isdigit((unsigned char)s[j])) ++j;
                toks.push_back(s.substr(i, j - i));
                i = j;
                continue;
            }
            if (std::isalpha((unsigned char)c) || c == '_') {
                size_t j = i + 1;
                while (j < n && (std::isalnum((unsigned char)s[j]) || s[j] == '_')) ++j;
                toks.push_back(s.substr(i, j - i));
                i = j;
                continue;
            }
            if (std::strchr("()[],<>+-*/=", c)) {
                toks.emplace_back(1, c);
                ++i;
                continue;
            }
            throw ParseError("cannot read '" + s.substr(i) + "'");
        }
    }
    const std::string* peek() const { return pos < toks.size() ? &toks[pos] : nullptr; }
    std::string take() {
        if (pos >= toks.size()) throw ParseError("unexpected end of line");
        return toks[pos++];
    }
    void expect(const char* t) {
        std::string got = take();
        if (got != t) throw ParseError(std::string("expected '") + t + "', found '" + got + "'");
    }
    bool at(const char* t) const { return peek() && *peek() == t; }
};

bool is_number(const std::string& t) {
    if (t == "inf" || t == "-inf" || t == "NaN") return true;
    size_t i = t[0] == '-' ? 1 : 0;
    return i < t.size() && std::isdigit((unsigned char)t[i]);
}

struct Parser {
    Kernel& k;
    explicit Parser(Kernel& k) : k(k) {}

    Expr* node(Expr::Kind kind) {
        k.exprs.emplace_back();
        Expr* e = &k.exprs.back();
        e->kind = kind;
        return e;
    }

    std::vector<const Expr*> index(Lexer& L) {
        L.expect("[");
        std::vector<const Expr*> ix;
        if (!L.at("]")) {
            ix.push_back(expr(L));
            while (L.at(",")) { L.take(); ix.push_back(expr(L)); }
        }
        L.expect("]");
        return ix;
    }

    const Expr* expr(Lexer& L) {
        std::string t = L.take();
        if (is_number(t)) {
            Expr* e = node(Expr::Num);
            e->lit = t;
            if (t == "NaN") e->num = NAN;
            else if (t == "inf") e->num = INFINITY;
            else if (t == "-inf") e->num = -INFINITY;
            else e->num = std::strtod(t.c_str(), nullptr);
            if (t.find('.') == std::string::npos && t != "inf" && t != "-inf" && t != "NaN") {
                e->integral = true;
                e->inum = std::strtoll(t.c_str(), nullptr, 10);
            }
            return e;
        }
        if (t[0] == '%') {
            int b = std::atoi(t.c_str() + 1);
            auto ix = index(L);
            Expr* e = node(Expr::Load);
            if (L.at("<v>")) { L.take(); e->kind = Expr::VLoad; }
            e->id = b;
            e->kids = std::move(ix);
            return e;
        }
        if (t == "(") {
            const Expr* a = expr(L);
            std::string op = L.take();
            const Expr* b = expr(L);
            L.expect(")");
            if (op == "+" || op == "-" || op == "*" || op == "/") {
                Expr* e = node(Expr::Bin);
                e->op = op == "+" ? Op::Add : op == "-" ? Op::Sub : op == "*" ? Op::Mul : Op::Div;
                if (L.at("<v>")) { L.take(); e->kind = Expr::VBin; }
                e->kids = {a, b};
                return e;
            }
            Expr* e = node(Expr::Compare);
            if (op == "<") e->cmp = Cmp::Lt;
            else if (op == "<=") e->cmp = Cmp::Le;
            else if (op == ">") e->cmp = Cmp::Gt;
            else if (op == ">=") e->cmp = Cmp::Ge;
            else if (op == "==") e->cmp = Cmp::Eq;
            else throw ParseError("unknown operator '" + op + "'");
            e->kids = {a, b};
            return e;
        }
        static const std::pair<const char*, Un> unary[] = {{"neg", Un::Neg}, {"exp", Un::Exp}, {"log", Un::Log},
                                                           {"tanh", Un::Tanh}, {"sqrt", Un::Sqrt}, {"sin", Un::Sin},
                                                           {"cos", Un::Cos}, {"erf", Un::Erf}, {"abs", Un::Abs}};
        for (auto& u : unary) {
            if (t == u.first) {
                L.expect("(");
                const Expr* a = expr(L);
                L.expect(")");
                Expr* e = node(Expr::Unary);
                e->un = u.second;
                e->kids = {a};
                return e;
            }
        }
        if (t == "real" || t == "int" || t == "splat") {
            L.expect("(");
            const Expr* a = expr(L);
            L.expect(")");
            Expr* e = node(t == "real" ? Expr::ToF : t == "int" ? Expr::ToI : Expr::Splat);
            e->kids = {a};
            return e;
        }
        if (t == "select") {
            L.expect("(");
            const Expr* c = expr(L);
            L.expect(",");
            const Expr* a = expr(L);
            L.expect(",");
            const Expr* b = expr(L);
            L.expect(")");
            Expr* e = node(Expr::Select);
            e->kids = {c, a, b};
            return e;
        }
        if (t.size() >= 2 && std::strchr("isnv", t[0]) && std::isdigit((unsigned char)t[1])) {
            Expr::Kind kind = t[0] == 'i' ? Expr::Iv : t[0] == 's' ? Expr::Sv : t[0] == 'n' ? Expr::Si : Expr::Vv;
            Expr* e = node(kind);
            e->id = std::atoi(t.c_str() + 1);
            return e;
        }
        throw ParseError("unexpected token '" + t + "'");
    }

    const Expr* full_expr(const std::string& s) {
        Lexer L(s);
        const Expr* e = expr(L);
        if (L.peek()) throw ParseError("trailing text in '" + s + "'");
        return e;
    }

    Stmt* snode(Stmt::Kind kind) {
        k.stmts.emplace_back();
        Stmt* s = &k.stmts.back();
        s->kind = kind;
        return s;
    }

    // Statements at indentation `depth` from line `pos`, up to the closing brace.
    std::vector<const Stmt*> body(const std::vector<std::string>& lines, size_t& pos, int depth) {
        std::vector<const Stmt*> out;
        std::string pad(2 * depth, ' '), close(2 * (depth - 1), ' ');
        close += "}";
        while (pos < lines.size()) {
            const std::string& line = lines[pos];
            if (line == close) { ++pos; return out; }
            if (line.compare(0, pad.size(), pad) != 0) throw ParseError("bad indentation: '" + line + "'");
            std::string s = line.substr(pad.size());
            if (s.compare(0, 5, "for i") == 0) {
                // for iV in 0..B {
                int v = 0;
                long long b = 0;
                char tail[4] = {0};
                if (std::sscanf(s.c_str(), "for i%d in 0..%lld %3s", &v, &b, tail) != 3 || std::strcmp(tail, "{") != 0)
                    throw ParseError("bad loop: '" + s + "'");
                Stmt* st = snode(Stmt::For);
                st->var = v;
                st->bound = b;
                ++pos;
                st->body = body(lines, pos, depth + 1);
                out.push_back(st);
                continue;
            }
            if (s.compare(0, 3, "if ") == 0 && s.size() > 5 && s.compare(s.size() - 2, 2, " {") == 0) {
                Stmt* st = snode(Stmt::If);
                st->value = full_expr(s.substr(3, s.size() - 5));
                ++pos;
                st->body = body(lines, pos, depth + 1);
                out.push_back(st);
                continue;
            }
            if (s[0] == '%') {
                Lexer L(s);
                std::string b = L.take();
                Stmt* st = snode(Stmt::Store);
                st->buf = std::atoi(b.c_str() + 1);
                st->index = index(L);
                std::string op = L.take();
                if (op == "<v=") st->kind = Stmt::VStore;
                else if (op != "=") throw ParseError("bad store: '" + s + "'");
                st->value = expr(L);
                if (L.peek()) throw ParseError("trailing text in '" + s + "'");
                ++pos;
                out.push_back(st);
                continue;
            }
            size_t eq = s.find(" = ");
            if (eq != std::string::npos && eq >= 2 && std::strchr("isnv", s[0])) {
                Stmt::Kind kind = s[0] == 's' ? Stmt::Set : s[0] == 'n' ? Stmt::SetI : s[0] == 'i' ? Stmt::SetL : Stmt::VSet;
                Stmt* st = snode(kind);
                st->var = std::atoi(s.c_str() + 1);
                st->value = full_expr(s.substr(eq + 3));
                ++pos;
                out.push_back(st);
                continue;
            }
            throw ParseError("cannot read statement '" + s + "'");
        }
        throw ParseError("missing closing brace");
    }
};

BufSpec parse_spec(const std::string& s) {
    // T[axes]
    size_t lb = s.find('['), rb = s.rfind(']');
    if (lb == std::string::npos || rb == std::string::npos || rb < lb) throw ParseError("bad buffer spec '" + s + "'");
    BufSpec b;
    std::string ty = s.substr(0, lb);
    if ((ty.compare(0, 5, "int8/") == 0 || ty.compare(0, 5, "int4/") == 0) && ty.size() > 5) {
        // `int{bits}/{over}` or `int{bits}/{over}..{end}` (ir.rs:506-507)
        b.ty = ty[3] == '8' ? Ty::Q8 : Ty::Q4;
        const std::string r = ty.substr(5);
        const size_t dd = r.find("..");
        char* e = nullptr;
        b.qover = (int)std::strtol(r.c_str(), &e, 10);
        if (e == r.c_str() || b.qover < 0) throw ParseError("bad quantised buffer type '" + ty + "'");
        if (dd != std::string::npos) {
            const int end = (int)std::strtol(r.c_str() + dd + 2, &e, 10);
            if (end <= b.qover || *e) throw ParseError("bad quantised buffer type '" + ty + "'");
            b.qspan = end - b.qover;
        } else if (*e) {
            throw ParseError("bad quantised buffer type '" + ty + "'");
        }
    } else if (!ty_parse(ty, &b.ty)) {
        throw ParseError("E7005: the buffer type '" + ty + "' is not one the executor computes");
    }
    std::string axes = s.substr(lb + 1, rb - lb - 1);
    size_t i = 0;
    while (i < axes.size()) {
        size_t j = axes.find(", ", i);
        std::string a = axes.substr(i, j == std::string::npos ? std::string::npos : j - i);
        size_t c = a.find(": ");
        if (c != std::string::npos) {
            b.names.push_back(a.substr(0, c));
            b.dims.push_back(std::strtoll(a.c_str() + c + 2, nullptr, 10));
        } else {
            b.names.push_back("");
            b.dims.push_back(std::strtoll(a.c_str(), nullptr, 10));
        }
        if (j == std::string::npos) break;
        i = j + 2;
    }
    return b;
}

void count_vars(Kernel& k, const std::vector<const Stmt*>& body) {
    std::function<void(const Expr*)> ex = [&](const Expr* e) {
        switch (e->kind) {
            case Expr::Iv: k.nloops = std::max(k.nloops, e->id + 1); break;
            case Expr::Sv: k.nreal = std::max(k.nreal, e->id + 1); break;
            case Expr::Si: k.nint = std::max(k.nint, e->id + 1); break;
            case Expr::Vv: k.nvec = std::max(k.nvec, e->id + 1); break;
            default: break;
        }
        for (auto c : e->kids) ex(c);
    };
    for (auto s : body) {
        switch (s->kind) {
            case Stmt::For: k.nloops = std::max(k.nloops, s->var + 1); break;
            case Stmt::Set: k.nreal = std::max(k.nreal, s->var + 1); break;
            case Stmt::SetI: k.nint = std::max(k.nint, s->var + 1); break;
            case Stmt::SetL: k.nloops = std::max(k.nloops, s->var + 1); break;
            case Stmt::VSet: k.nvec = std::max(k.nvec, s->var + 1); break;
            default: break;
        }
        for (auto e : s->index) ex(e);
        if (s->value) ex(s->value);
        count_vars(k, s->body);
    }
}

}  // namespace

std::unique_ptr<Kernel> parse_kernel(const std::string& text, const std::string& dtype, int lanes, std::string* err) {
    auto k = std::make_unique<Kernel>();
    try {
        std::vector<std::string> lines;
        {
            std::string cur;
            for (char c : text) {
                if (c == '\n') { lines.push_back(cur); cur.clear(); }
                else cur += c;
            }
            if (!cur.empty()) lines.push_back(cur);
        }
        if (lines.empty()) throw ParseError("empty kernel text");
        const std::string& head = lines[0];
        if (head.compare(0, 7, "kernel ") != 0 || head.back() != '{') throw ParseError("not a kernel header: '" + head + "'");
        size_t arrow = head.find(" -> %");
        if (arrow == std::string::npos) throw ParseError("no output in the header");
        size_t open = head.rfind(" (", arrow);
        if (open == std::string::npos || open < 7) throw ParseError("no input list in the header");
        k->name = head.substr(7, open - 7);
        std::string ins = head.substr(open + 2, arrow - 1 - (open + 2));
        // split the input list at top-level commas
        {
            int depth = 0;
            std::string cur;
            std::vector<std::string> parts;
            for (char c : ins) {
                if (c == '[') ++depth;
                if (c == ']') --depth;
                if (c == ',' && depth == 0) { parts.push_back(cur); cur.clear(); }
                else cur += c;
            }
            if (!cur.empty()) parts.push_back(cur);
            for (size_t i = 0; i < parts.size(); ++i) {
                std::string p = parts[i];
                while (!p.empty() && p[0] == ' ') p.erase(0, 1);
                std::string pre = "%" + std::to_string(i) + " : ";
                if (p.compare(0, pre.size(), pre) != 0) throw ParseError("bad input spec '" + p + "'");
                k->inputs.push_back(parse_spec(p.substr(pre.size())));
            }
        }
        std::string rest = head.substr(arrow + 4, head.size() - 1 - (arrow + 4));
        while (!rest.empty() && rest.back() == ' ') rest.pop_back();
        std::string pre = "%" + std::to_string(k->inputs.size()) + " : ";
        if (rest.compare(0, pre.size(), pre) != 0) throw ParseError("bad output '" + rest + "'");
        rest = rest.substr(pre.size());
        size_t rb = rest.find(']');
        if (rb == std::string::npos) throw ParseError("bad output spec '" + rest + "'");
        k->output = parse_spec(rest.substr(0, rb + 1));
        if (rb + 1 < rest.size()) {
            k->arith = rest.substr(rb + 2);
            if (k->arith.compare(0, 6, "arith ") != 0) throw ParseError("bad formats '" + k->arith + "'");
        }
        // the storage type
        if (!dtype.empty()) {
            if (!ty_parse(dtype, &k->dtype) || k->dtype == Ty::I64) throw ParseError("unknown storage type '" + dtype + "'");
        } else if (k->output.ty != Ty::I64) {
            k->dtype = k->output.ty;
        } else {
            int best = -1;
            for (auto& b : k->inputs)
                if (b.ty != Ty::I64 && !ty_quant(b.ty) && ty_rank(b.ty) > best) { best = ty_rank(b.ty); k->dtype = b.ty; }
            if (best < 0) k->dtype = Ty::F32;
        }
        for (size_t i = 0; i <= k->inputs.size(); ++i) {
            BufSpec& b = i == k->inputs.size() ? k->output : k->inputs[i];
            if (b.ty == Ty::I64 || b.ty == k->dtype) continue;
            if (ty_quant(b.ty)) {
                if (i == k->inputs.size()) throw ParseError("an integer output buffer");
                if (b.qover + b.qspan > (int)b.dims.size()) throw ParseError("a quantised buffer's scale axes past its rank");
                continue;
            }
            if (ty_rank(b.ty) < ty_rank(k->dtype) && i < k->inputs.size()) b.wide = true;
            else throw ParseError(std::string("buffer %") + std::to_string(i) + " of type " + ty_name(b.ty) + " in a " + ty_name(k->dtype) + " kernel");
        }
        k->lanes = lanes < 1 ? 1 : lanes;
        Parser P(*k);
        size_t pos = 1;
        k->body = P.body(lines, pos, 1);
        if (pos != lines.size()) throw ParseError("text after the kernel's closing brace");
        count_vars(*k, k->body);
    } catch (const std::exception& e) {
        if (err) *err = e.what();
        return nullptr;
    }
    return k;
}

// ---- printing ------------------------------------------------------------------
std::string show_expr(const Expr& e) {
    auto join = [](const std::vector<const Expr*>& v) {
        std::string s;
        for (size_t i = 0; i < v.size(); ++i) {
            if (i) s += ", ";
            s += show_expr(*v[i]);
        }
        return s;
    };
    static const char* ops = "+-*/";
    switch (e.kind) {
        case Expr::Num: return e.lit;
        case Expr::Load: return "%" + std::to_string(e.id) + "[" + join(e.kids) + "]";
        case Expr::VLoad: return "%" + std::to_string(e.id) + "[" + join(e.kids) + "]<v>";
        case Expr::Iv: return "i" + std::to_string(e.id);
        case Expr::Sv: return "s" + std::to_string(e.id);
        case Expr::Si: return "n" + std::to_string(e.id);
        case Expr::Vv: return "v" + std::to_string(e.id);
        case Expr::Bin:
        case Expr::VBin: {
            std::string s = "(" + show_expr(*e.kids[0]) + " " + ops[(int)e.op] + " " + show_expr(*e.kids[1]) + ")";
            return e.kind == Expr::VBin ? s + "<v>" : s;
        }
        case Expr::Unary: {
            static const char* names[] = {"neg", "exp", "log", "tanh", "sqrt", "sin", "cos", "erf", "abs"};
            return std::string(names[(int)e.un]) + "(" + show_expr(*e.kids[0]) + ")";
        }
        case Expr::Compare: {
            static const char* names[] = {"<", "<=", ">", ">=", "=="};
            return "(" + show_expr(*e.kids[0]) + " " + names[(int)e.cmp] + " " + show_expr(*e.kids[1]) + ")";
        }
        case Expr::Select: return "select(" + join(e.kids) + ")";
        case Expr::ToF: return "real(" + show_expr(*e.kids[0]) + ")";
        case Expr::ToI: return "int(" + show_expr(*e.kids[0]) + ")";
        case Expr::Splat: return "splat(" + show_expr(*e.kids[0]) + ")";
    }
    return "?";
}

static void show_body(const std::vector<const Stmt*>& body, int depth, std::string& out) {
    std::string pad(2 * depth, ' ');
    for (auto s : body) {
        switch (s->kind) {
            case Stmt::For:
                out += pad + "for i" + std::to_string(s->var) + " in 0.." + std::to_string(s->bound) + " {\n";
                show_body(s->body, depth + 1, out);
                out += pad + "}\n";
                break;
            case Stmt::If:
                out += pad + "if " + show_expr(*s->value) + " {\n";
                show_body(s->body, depth + 1, out);
                out += pad + "}\n";
                break;
            case Stmt::Store:
            case Stmt::VStore: {
                std::string ix;
                for (size_t i = 0; i < s->index.size(); ++i) ix += (i ? ", " : "") + show_expr(*s->index[i]);
                out += pad + "%" + std::to_string(s->buf) + "[" + ix + "] " + (s->kind == Stmt::VStore ? "<v= " : "= ") + show_expr(*s->value) + "\n";
                break;
            }
            default: {
                char v = s->kind == Stmt::Set ? 's' : s->kind == Stmt::SetI ? 'n' : s->kind == Stmt::SetL ? 'i' : 'v';
                out += pad + v + std::to_string(s->var) + " = " + show_expr(*s->value) + "\n";
            }
        }
    }
}

static std::string show_spec(const BufSpec& b) {
    std::string s = ty_name(b.ty);
    if (ty_quant(b.ty)) {
        s += "/" + std::to_string(b.qover);
        if (b.qspan != 1) s += ".." + std::to_string(b.qover + b.qspan);
    }
    s += "[";
    for (size_t i = 0; i < b.dims.size(); ++i) {
        if (i) s += ", ";
        if (!b.names[i].empty()) s += b.names[i] + ": ";
        s += std::to_string(b.dims[i]);
    }
    return s + "]";
}

std::string show_kernel(const Kernel& k) {
    std::string s = "kernel " + k.name + " (";
    for (size_t i = 0; i < k.inputs.size(); ++i) s += (i ? ", %" : "%") + std::to_string(i) + " : " + show_spec(k.inputs[i]);
    s += ") -> %" + std::to_string(k.inputs.size()) + " : " + show_spec(k.output);
    if (!k.arith.empty()) s += " " + k.arith;
    s += " {\n";
    show_body(k.body, 1, s);
    return s + "}\n";
}

// ---- parallel loops ----------------------------------------------------------
int64_t parallel_outer(const Kernel& k) {
    if (k.body.size() != 1 || k.body[0]->kind != Stmt::For) return -1;
    int var = k.body[0]->var;
    int stores = 0;
    bool ok = true;
    std::function<void(const std::vector<const Stmt*>&)> walk = [&](const std::vector<const Stmt*>& b) {
        for (auto s : b) {
            switch (s->kind) {
                case Stmt::For: case Stmt::If: walk(s->body); break;
                case Stmt::Store: case Stmt::VStore: {
                    ++stores;
                    bool direct = false;
                    for (auto e : s->index)
                        if (e->kind == Expr::Iv && e->id == var) direct = true;
                    if (!direct) ok = false;
                    break;
                }
                case Stmt::SetL: if (s->var == var) ok = false; break;
                default: break;
            }
        }
    };
    walk(k.body[0]->body);
    return ok && stores > 0 ? k.body[0]->bound : -1;
}

bool writes_disjoint(const Kernel& k, int v, const std::vector<const Stmt*>& body) {
    const int out = k.out_buf();
    struct Access { std::vector<const Expr*> ix; bool vector; };
    std::vector<Access> acc;
    int stores = 0;
    bool assigned = false;
    std::function<void(const Expr*)> ex = [&](const Expr* e) {
        if ((e->kind == Expr::Load || e->kind == Expr::VLoad) && e->id == out) acc.push_back({e->kids, e->kind == Expr::VLoad});
        for (auto c : e->kids) ex(c);
    };
    std::function<void(const std::vector<const Stmt*>&)> walk = [&](const std::vector<const Stmt*>& b) {
        for (auto s : b) {
            switch (s->kind) {
                case Stmt::For: walk(s->body); break;
                case Stmt::If: ex(s->value); walk(s->body); break;
                case Stmt::Store: case Stmt::VStore:
                    if (s->buf == out) { ++stores; acc.push_back({s->index, s->kind == Stmt::VStore}); }
                    for (auto e : s->index) ex(e);
                    ex(s->value);
                    break;
                case Stmt::SetL: if (s->var == v) assigned = true; ex(s->value); break;
                default: ex(s->value); break;
            }
        }
    };
    walk(body);
    if (assigned || stores == 0) return false;
    // c*v + t at an index position
    auto affine = [&](const Expr* e, int64_t* c, int64_t* t) -> bool {
        auto iv = [&](const Expr* x) { return x->kind == Expr::Iv && x->id == v; };
        auto lit = [&](const Expr* x, int64_t* n) { if (x->kind == Expr::Num && x->integral) { *n = x->inum; return true; } return false; };
        if (iv(e)) { *c = 1; *t = 0; return true; }
        if (e->kind == Expr::Bin && e->op == Op::Mul) {
            if (iv(e->kids[0]) && lit(e->kids[1], c)) { *t = 0; return true; }
            if (iv(e->kids[1]) && lit(e->kids[0], c)) { *t = 0; return true; }
            return false;
        }
        if (e->kind == Expr::Bin && e->op == Op::Add && lit(e->kids[1], t)) {
            const Expr* m = e->kids[0];
            if (m->kind == Expr::Bin && m->op == Op::Mul) {
                if (iv(m->kids[0]) && lit(m->kids[1], c)) return true;
                if (iv(m->kids[1]) && lit(m->kids[0], c)) return true;
            }
        }
        return false;
    };
    const size_t rank = k.output.dims.size();
    for (size_t p = 0; p < rank; ++p) {
        bool all = true;
        for (auto& a : acc) {
            int64_t span = a.vector && p + 1 == rank ? k.lanes : 1, c = 0, t = 0;
            if (p >= a.ix.size() || !affine(a.ix[p], &c, &t) || !(c >= 1 && t >= 0 && t + span <= c)) { all = false; break; }
        }
        if (all) return true;
    }
    return false;
}

}  // namespace presk
