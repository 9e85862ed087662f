// yl_jinja.cpp -- a small Jinja renderer for GGUF chat templates (see
// yl_jinja.h for the supported subset and the minijinja defaults followed).
#include "yl_jinja.h"

#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <functional>

namespace yl {
namespace jinja {
namespace {

// ------------------------------------------------------------------ lexer
enum TokKind { T_TEXT, T_VAR_BEGIN, T_VAR_END, T_BLOCK_BEGIN, T_BLOCK_END, T_NAME, T_STR, T_INT, T_FLOAT, T_OP, T_EOF };

struct Tok {
    TokKind kind;
    std::string text;
    int64_t i = 0;
    double f = 0.0;
};

struct RenderError {
    std::string msg;
};
[[noreturn]] void fail(const std::string& m) { throw RenderError{m}; }

bool is_ws(char c) { return c == ' ' || c == '\t' || c == '\n' || c == '\r' || c == '\f' || c == '\v'; }

std::string trim_ws(const std::string& s, bool left = true, bool right = true);
// whitespace control strips Unicode White_Space, as Rust's trim_start/trim_end
void rstrip(std::string& s) { s = trim_ws(s, false, true); }

std::vector<Tok> lex(std::string src) {
    // keep_trailing_newline = false: one trailing newline is dropped
    if (!src.empty() && src.back() == '\n') {
        src.pop_back();
        if (!src.empty() && src.back() == '\r') src.pop_back();
    }
    std::vector<Tok> out;
    size_t p = 0;
    const size_t n = src.size();
    bool lstrip_next = false;   // the previous tag ended with '-'
    auto push_text = [&](std::string t) {
        if (lstrip_next) {
            t = trim_ws(t, true, false);
            lstrip_next = false;
        }
        if (!t.empty()) out.push_back(Tok{T_TEXT, std::move(t)});
    };
    auto strip_prev_text = [&]() {
        if (!out.empty() && out.back().kind == T_TEXT) {
            rstrip(out.back().text);
            if (out.back().text.empty()) out.pop_back();
        }
    };
    while (p < n) {
        size_t q = p;
        while (q + 1 < n && !(src[q] == '{' && (src[q + 1] == '{' || src[q + 1] == '%' || src[q + 1] == '#'))) q++;
        if (q + 1 >= n) {
            push_text(src.substr(p));
            break;
        }
        push_text(src.substr(p, q - p));
        const char kind = src[q + 1];
        p = q + 2;
        if (p < n && src[p] == '-') { strip_prev_text(); p++; }
        else if (p < n && src[p] == '+') p++;
        if (kind == '#') {
            const size_t e = src.find("#}", p);
            if (e == std::string::npos) fail("unterminated comment");
            if (e > p && src[e - 1] == '-') lstrip_next = true;
            p = e + 2;
            continue;
        }
        const char close = kind == '{' ? '}' : '%';
        out.push_back(Tok{kind == '{' ? T_VAR_BEGIN : T_BLOCK_BEGIN, ""});
        const size_t first_tok = out.size();
        bool closed = false;
        while (p < n) {
            const char c = src[p];
            if (is_ws(c)) { p++; continue; }
            // end of tag, with optional whitespace control
            if ((c == '-' || c == '+') && src.compare(p + 1, 2, std::string(1, close) + "}") == 0) {
                if (c == '-') lstrip_next = true;
                p += 3;
                closed = true;
                break;
            }
            if (c == close && p + 1 < n && src[p + 1] == '}') {
                p += 2;
                closed = true;
                break;
            }
            if (isalpha((unsigned char)c) || c == '_') {
                size_t e = p;
                while (e < n && (isalnum((unsigned char)src[e]) || src[e] == '_')) e++;
                out.push_back(Tok{T_NAME, src.substr(p, e - p)});
                p = e;
                continue;
            }
            if (isdigit((unsigned char)c)) {
                size_t e = p;
                bool flt = false;
                while (e < n && (isdigit((unsigned char)src[e]) || src[e] == '_')) e++;
                if (e + 1 < n && src[e] == '.' && isdigit((unsigned char)src[e + 1])) {
                    flt = true;
                    e++;
                    while (e < n && isdigit((unsigned char)src[e])) e++;
                }
                std::string num;
                for (size_t k = p; k < e; k++)
                    if (src[k] != '_') num += src[k];
                Tok t{flt ? T_FLOAT : T_INT, num};
                if (flt) t.f = strtod(num.c_str(), nullptr);
                else t.i = strtoll(num.c_str(), nullptr, 10);
                out.push_back(t);
                p = e;
                continue;
            }
            if (c == '\'' || c == '"') {
                std::string s;
                size_t e = p + 1;
                bool done = false;
                while (e < n) {
                    const char d = src[e];
                    if (d == c) { done = true; e++; break; }
                    if (d == '\\' && e + 1 < n) {
                        const char x = src[e + 1];
                        switch (x) {
                        case 'n': s += '\n'; break;
                        case 't': s += '\t'; break;
                        case 'r': s += '\r'; break;
                        case '\\': s += '\\'; break;
                        case '\'': s += '\''; break;
                        case '"': s += '"'; break;
                        case '0': s += '\0'; break;
                        default: s += '\\'; s += x; break;
                        }
                        e += 2;
                        continue;
                    }
                    s += d;
                    e++;
                }
                if (!done) fail("unterminated string literal");
                out.push_back(Tok{T_STR, s});
                p = e;
                continue;
            }
            static const char* ops2[] = {"==", "!=", "<=", ">=", "//", "**", nullptr};
            bool matched = false;
            for (int k = 0; ops2[k]; k++)
                if (src.compare(p, 2, ops2[k]) == 0) {
                    out.push_back(Tok{T_OP, ops2[k]});
                    p += 2;
                    matched = true;
                    break;
                }
            if (matched) continue;
            if (strchr("()[]{}.,:|~+-*/%<>=!", c)) {
                out.push_back(Tok{T_OP, std::string(1, c)});
                p++;
                continue;
            }
            fail(std::string("unexpected character '") + c + "' in a tag");
        }
        if (!closed) fail("unterminated tag");
        out.push_back(Tok{kind == '{' ? T_VAR_END : T_BLOCK_END, ""});
        // {% raw %} ... {% endraw %}: the text in between is literal
        if (kind == '%' && out.size() == first_tok + 2 && out[first_tok].kind == T_NAME && out[first_tok].text == "raw") {
            out.resize(first_tok - 1);
            size_t s = p;
            for (;;) {
                const size_t b = src.find("{%", s);
                if (b == std::string::npos) fail("missing endraw");
                size_t k = b + 2;
                bool strip = false;
                if (k < n && (src[k] == '-' || src[k] == '+')) { strip = src[k] == '-'; k++; }
                while (k < n && is_ws(src[k])) k++;
                if (src.compare(k, 6, "endraw") == 0) {
                    std::string body = src.substr(p, b - p);
                    if (strip) rstrip(body);
                    push_text(body);
                    k += 6;
                    while (k < n && is_ws(src[k])) k++;
                    if (k < n && src[k] == '-') { lstrip_next = true; k++; }
                    if (src.compare(k, 2, "%}") != 0) fail("malformed endraw");
                    p = k + 2;
                    break;
                }
                s = b + 2;
            }
        }
    }
    out.push_back(Tok{T_EOF, ""});
    return out;
}

// -------------------------------------------------------------------- AST
struct Expr;
using ExprP = std::shared_ptr<Expr>;
struct Expr {
    enum K { Lit, Name, Attr, Item, Slice, Call, Filter, Test, Unary, Binary, Cond, ListE, MapE } k;
    Value lit;
    std::string name;                  // Name, Attr, Filter, Test, Unary/Binary op
    ExprP a, b, c;                     // operands (Slice: a[b:c], Cond: b if a else c)
    std::vector<ExprP> args;           // Call/Filter/Test positional, ListE items, MapE keys
    std::vector<ExprP> args2;          // MapE values
    std::vector<std::pair<std::string, ExprP>> kwargs;
    bool neg = false;                  // Test: `is not`
};

struct Node;
using NodeP = std::shared_ptr<Node>;
struct Node {
    enum K { Text, Out, If, For, Set } k;
    std::string text;
    ExprP e;                                            // Out / Set value / For iterable
    std::vector<std::pair<ExprP, std::vector<NodeP>>> branches;   // If
    std::vector<NodeP> body, else_body;                 // For / If else
    std::vector<std::string> targets;                   // For loop vars / Set: name or [ns, attr]
    ExprP filter;                                       // For ... if filter
};

class Parser {
public:
    explicit Parser(std::vector<Tok> t) : t_(std::move(t)) {}

    std::vector<NodeP> parse_all() {
        std::vector<NodeP> body;
        std::string end;
        parse_body(&body, {}, &end);
        if (!end.empty()) fail("unexpected {% " + end + " %}");
        return body;
    }

private:
    std::vector<Tok> t_;
    size_t p_ = 0;

    const Tok& peek(int k = 0) const { return t_[std::min(p_ + k, t_.size() - 1)]; }
    Tok next() { return t_[p_ < t_.size() - 1 ? p_++ : p_]; }
    bool is_op(const char* op, int k = 0) const { return peek(k).kind == T_OP && peek(k).text == op; }
    bool is_name(const char* nm, int k = 0) const { return peek(k).kind == T_NAME && peek(k).text == nm; }
    void expect_op(const char* op) {
        if (!is_op(op)) fail(std::string("expected '") + op + "'");
        p_++;
    }
    void expect(TokKind k, const char* what) {
        if (peek().kind != k) fail(std::string("expected ") + what);
        p_++;
    }
    std::string expect_name() {
        if (peek().kind != T_NAME) fail("expected a name");
        return next().text;
    }

    // Parses nodes until a block tag whose keyword is in `stops`; returns it in *end
    void parse_body(std::vector<NodeP>* body, const std::vector<std::string>& stops, std::string* end) {
        end->clear();
        for (;;) {
            const Tok& t = peek();
            if (t.kind == T_EOF) return;
            if (t.kind == T_TEXT) {
                auto n = std::make_shared<Node>();
                n->k = Node::Text;
                n->text = t.text;
                body->push_back(n);
                p_++;
                continue;
            }
            if (t.kind == T_VAR_BEGIN) {
                p_++;
                auto n = std::make_shared<Node>();
                n->k = Node::Out;
                n->e = parse_expr();
                expect(T_VAR_END, "'}}'");
                body->push_back(n);
                continue;
            }
            if (t.kind != T_BLOCK_BEGIN) fail("unexpected token");
            p_++;
            const std::string kw = expect_name();
            if (std::find(stops.begin(), stops.end(), kw) != stops.end()) {
                *end = kw;
                return;   // the caller consumes the rest of the tag
            }
            if (kw == "if") body->push_back(parse_if());
            else if (kw == "for") body->push_back(parse_for());
            else if (kw == "set") body->push_back(parse_set());
            else fail("unsupported tag {% " + kw + " %}");
        }
    }

    NodeP parse_if() {
        auto n = std::make_shared<Node>();
        n->k = Node::If;
        ExprP cond = parse_expr();
        expect(T_BLOCK_END, "'%}'");
        for (;;) {
            std::vector<NodeP> body;
            std::string end;
            parse_body(&body, {"elif", "else", "endif"}, &end);
            if (end.empty()) fail("missing endif");
            n->branches.push_back({cond, body});
            if (end == "elif") {
                cond = parse_expr();
                expect(T_BLOCK_END, "'%}'");
                continue;
            }
            expect(T_BLOCK_END, "'%}'");
            if (end == "else") {
                parse_body(&n->else_body, {"endif"}, &end);
                if (end.empty()) fail("missing endif");
                expect(T_BLOCK_END, "'%}'");
            }
            return n;
        }
    }

    NodeP parse_for() {
        auto n = std::make_shared<Node>();
        n->k = Node::For;
        n->targets.push_back(expect_name());
        while (is_op(",")) {
            p_++;
            n->targets.push_back(expect_name());
        }
        if (!is_name("in")) fail("expected 'in'");
        p_++;
        n->e = parse_or_cond(false);
        if (is_name("if")) {
            p_++;
            n->filter = parse_or_cond(false);
        }
        if (is_name("recursive")) fail("recursive loops are not supported");
        expect(T_BLOCK_END, "'%}'");
        std::string end;
        parse_body(&n->body, {"else", "endfor"}, &end);
        if (end.empty()) fail("missing endfor");
        expect(T_BLOCK_END, "'%}'");
        if (end == "else") {
            parse_body(&n->else_body, {"endfor"}, &end);
            if (end.empty()) fail("missing endfor");
            expect(T_BLOCK_END, "'%}'");
        }
        return n;
    }

    NodeP parse_set() {
        auto n = std::make_shared<Node>();
        n->k = Node::Set;
        n->targets.push_back(expect_name());
        if (is_op(".")) {
            p_++;
            n->targets.push_back(expect_name());
        }
        if (!is_op("=")) fail("block {% set %} is not supported");
        p_++;
        n->e = parse_expr();
        expect(T_BLOCK_END, "'%}'");
        return n;
    }

    // expression grammar (Jinja's precedence)
    ExprP parse_expr() { return parse_or_cond(true); }
    ExprP parse_or_cond(bool allow_cond) {
        ExprP e = parse_or();
        if (allow_cond && is_name("if")) {
            p_++;
            auto c = std::make_shared<Expr>();
            c->k = Expr::Cond;
            c->b = e;
            c->a = parse_or();
            if (is_name("else")) {
                p_++;
                c->c = parse_or_cond(true);
            }
            return c;
        }
        return e;
    }
    ExprP bin(const std::string& op, ExprP l, ExprP r) {
        auto e = std::make_shared<Expr>();
        e->k = Expr::Binary;
        e->name = op;
        e->a = l;
        e->b = r;
        return e;
    }
    ExprP parse_or() {
        ExprP l = parse_and();
        while (is_name("or")) { p_++; l = bin("or", l, parse_and()); }
        return l;
    }
    ExprP parse_and() {
        ExprP l = parse_not();
        while (is_name("and")) { p_++; l = bin("and", l, parse_not()); }
        return l;
    }
    ExprP parse_not() {
        if (is_name("not")) {
            p_++;
            auto e = std::make_shared<Expr>();
            e->k = Expr::Unary;
            e->name = "not";
            e->a = parse_not();
            return e;
        }
        return parse_compare();
    }
    ExprP parse_compare() {
        ExprP l = parse_math1();
        for (;;) {
            if (peek().kind == T_OP && (peek().text == "==" || peek().text == "!=" || peek().text == "<" ||
                                        peek().text == ">" || peek().text == "<=" || peek().text == ">=")) {
                const std::string op = next().text;
                l = bin(op, l, parse_math1());
            } else if (is_name("in")) {
                p_++;
                l = bin("in", l, parse_math1());
            } else if (is_name("not") && is_name("in", 1)) {
                p_ += 2;
                l = bin("notin", l, parse_math1());
            } else {
                return l;
            }
        }
    }
    ExprP parse_math1() {
        ExprP l = parse_concat();
        while (is_op("+") || is_op("-")) {
            const std::string op = next().text;
            l = bin(op, l, parse_concat());
        }
        return l;
    }
    ExprP parse_concat() {
        ExprP l = parse_math2();
        while (is_op("~")) { p_++; l = bin("~", l, parse_math2()); }
        return l;
    }
    ExprP parse_math2() {
        ExprP l = parse_pow();
        while (is_op("*") || is_op("/") || is_op("//") || is_op("%")) {
            const std::string op = next().text;
            l = bin(op, l, parse_pow());
        }
        return l;
    }
    ExprP parse_pow() {
        ExprP l = parse_unary();
        while (is_op("**")) { p_++; l = bin("**", l, parse_unary()); }
        return l;
    }
    ExprP parse_unary() {
        if (is_op("-") || is_op("+")) {
            const std::string op = next().text;
            auto e = std::make_shared<Expr>();
            e->k = Expr::Unary;
            e->name = op;
            e->a = parse_unary();
            return parse_filters(e);
        }
        return parse_filters(parse_postfix(parse_primary()));
    }
    void parse_args(std::vector<ExprP>* args, std::vector<std::pair<std::string, ExprP>>* kwargs) {
        expect_op("(");
        while (!is_op(")")) {
            if (peek().kind == T_NAME && is_op("=", 1)) {
                const std::string k = next().text;
                p_++;
                kwargs->push_back({k, parse_expr()});
            } else {
                args->push_back(parse_expr());
            }
            if (is_op(",")) p_++;
            else break;
        }
        expect_op(")");
    }
    ExprP parse_primary() {
        const Tok t = peek();
        auto e = std::make_shared<Expr>();
        if (t.kind == T_STR) {
            p_++;
            std::string s = t.text;
            while (peek().kind == T_STR) s += next().text;   // adjacent literals concatenate
            e->k = Expr::Lit;
            e->lit = Value::str(s);
            return e;
        }
        if (t.kind == T_INT) { p_++; e->k = Expr::Lit; e->lit = Value::integer(t.i); return e; }
        if (t.kind == T_FLOAT) { p_++; e->k = Expr::Lit; e->lit = Value::number(t.f); return e; }
        if (t.kind == T_NAME) {
            p_++;
            e->k = Expr::Lit;
            if (t.text == "true" || t.text == "True") { e->lit = Value::boolean(true); return e; }
            if (t.text == "false" || t.text == "False") { e->lit = Value::boolean(false); return e; }
            if (t.text == "none" || t.text == "None") { e->lit = Value::none(); return e; }
            e->k = Expr::Name;
            e->name = t.text;
            return e;
        }
        if (is_op("(")) {
            p_++;
            ExprP in = parse_expr();
            if (is_op(",")) {   // tuple -> list
                auto l = std::make_shared<Expr>();
                l->k = Expr::ListE;
                l->args.push_back(in);
                while (is_op(",")) {
                    p_++;
                    if (is_op(")")) break;
                    l->args.push_back(parse_expr());
                }
                in = l;
            }
            expect_op(")");
            return in;
        }
        if (is_op("[")) {
            p_++;
            e->k = Expr::ListE;
            while (!is_op("]")) {
                e->args.push_back(parse_expr());
                if (is_op(",")) p_++;
                else break;
            }
            expect_op("]");
            return e;
        }
        if (is_op("{")) {
            p_++;
            e->k = Expr::MapE;
            while (!is_op("}")) {
                e->args.push_back(parse_expr());
                expect_op(":");
                e->args2.push_back(parse_expr());
                if (is_op(",")) p_++;
                else break;
            }
            expect_op("}");
            return e;
        }
        fail("unexpected token in expression: '" + t.text + "'");
    }
    ExprP parse_postfix(ExprP e) {
        for (;;) {
            if (is_op(".")) {
                p_++;
                auto a = std::make_shared<Expr>();
                a->k = Expr::Attr;
                a->a = e;
                if (peek().kind == T_INT) a->name = std::to_string(next().i);
                else a->name = expect_name();
                e = a;
            } else if (is_op("[")) {
                p_++;
                ExprP lo, hi;
                bool slice = false;
                if (!is_op(":")) lo = parse_expr();
                if (is_op(":")) {
                    slice = true;
                    p_++;
                    if (!is_op("]") && !is_op(":")) hi = parse_expr();
                    if (is_op(":")) fail("slice steps are not supported");
                }
                expect_op("]");
                auto a = std::make_shared<Expr>();
                a->k = slice ? Expr::Slice : Expr::Item;
                a->a = e;
                a->b = lo;
                a->c = hi;
                e = a;
            } else if (is_op("(")) {
                auto c = std::make_shared<Expr>();
                c->k = Expr::Call;
                c->a = e;
                parse_args(&c->args, &c->kwargs);
                e = c;
            } else {
                return e;
            }
        }
    }
    ExprP parse_filters(ExprP e) {
        for (;;) {
            if (is_op("|")) {
                p_++;
                auto f = std::make_shared<Expr>();
                f->k = Expr::Filter;
                f->a = e;
                f->name = expect_name();
                if (is_op("(")) parse_args(&f->args, &f->kwargs);
                e = f;
            } else if (is_name("is")) {
                p_++;
                auto t = std::make_shared<Expr>();
                t->k = Expr::Test;
                t->a = e;
                if (is_name("not")) { p_++; t->neg = true; }
                t->name = expect_name();
                if (is_op("(")) parse_args(&t->args, &t->kwargs);
                else if (peek().kind == T_STR || peek().kind == T_INT || peek().kind == T_FLOAT ||
                         (peek().kind == T_NAME && !is_name("and") && !is_name("or") && !is_name("else") &&
                          !is_name("if") && !is_name("is") && !is_name("in") && !is_name("not")))
                    t->args.push_back(parse_postfix(parse_primary()));   // `x is divisibleby 3`
                e = t;
            } else {
                return e;
            }
        }
    }
};

// ------------------------------------------------------------- evaluation
bool truthy(const Value& v) {
    switch (v.kind) {
    case Value::kUndef: case Value::kNone: return false;
    case Value::kBool: return v.b;
    case Value::kInt: return v.i != 0;
    case Value::kFloat: return v.f != 0.0;
    case Value::kStr: return !v.s.empty();
    case Value::kList: return !v.l->empty();
    case Value::kMap: return !v.m->empty();
    default: return true;
    }
}

std::string kind_name(const Value& v) {
    static const char* nm[] = {"undefined", "none", "bool", "number", "number", "string", "sequence", "map",
                               "namespace", "function"};
    return nm[v.kind];
}

std::string fmt_float(double d) {
    if (isnan(d)) return "NaN";
    if (isinf(d)) return d > 0 ? "inf" : "-inf";
    char buf[64];
    for (int prec = 1; prec <= 17; prec++) {   // shortest round-trip form
        snprintf(buf, sizeof buf, "%.*g", prec, d);
        if (strtod(buf, nullptr) == d) break;
    }
    std::string s = buf;
    if (s.find_first_of(".eEn") == std::string::npos) s += ".0";
    return s;
}

std::string repr(const Value& v);
std::string to_str(const Value& v) {
    switch (v.kind) {
    case Value::kUndef: return "";
    case Value::kNone: return "none";
    case Value::kBool: return v.b ? "true" : "false";
    case Value::kInt: return std::to_string(v.i);
    case Value::kFloat: return fmt_float(v.f);
    case Value::kStr: return v.s;
    default: return repr(v);
    }
}
std::string quote(const std::string& s) {
    std::string o = "\"";
    for (char c : s) {
        if (c == '"' || c == '\\') o += '\\';
        if (c == '\n') { o += "\\n"; continue; }
        o += c;
    }
    return o + "\"";
}
std::string repr(const Value& v) {
    if (v.kind == Value::kStr) return quote(v.s);
    if (v.kind == Value::kList) {
        std::string o = "[";
        for (size_t k = 0; k < v.l->size(); k++) o += (k ? ", " : "") + repr((*v.l)[k]);
        return o + "]";
    }
    if (v.kind == Value::kMap || v.kind == Value::kNs) {
        std::string o = "{";
        for (size_t k = 0; k < v.m->size(); k++) o += (k ? ", " : "") + quote((*v.m)[k].first) + ": " + repr((*v.m)[k].second);
        return o + "}";
    }
    return to_str(v);
}

// JSON as minijinja's tojson writes it (HTML-sensitive characters escaped)
std::string to_json(const Value& v) {
    switch (v.kind) {
    case Value::kUndef: case Value::kNone: return "null";
    case Value::kBool: return v.b ? "true" : "false";
    case Value::kInt: return std::to_string(v.i);
    case Value::kFloat: return fmt_float(v.f);
    case Value::kStr: {
        std::string o = "\"";
        for (unsigned char c : v.s) {
            switch (c) {
            case '"': o += "\\\""; break;
            case '\\': o += "\\\\"; break;
            case '\n': o += "\\n"; break;
            case '\r': o += "\\r"; break;
            case '\t': o += "\\t"; break;
            case '<': o += "\\u003c"; break;
            case '>': o += "\\u003e"; break;
            case '&': o += "\\u0026"; break;
            case '\'': o += "\\u0027"; break;
            default:
                if (c < 0x20) { char b[8]; snprintf(b, sizeof b, "\\u%04x", c); o += b; }
                else o += (char)c;
            }
        }
        return o + "\"";
    }
    case Value::kList: {
        std::string o = "[";
        for (size_t k = 0; k < v.l->size(); k++) o += (k ? "," : "") + to_json((*v.l)[k]);
        return o + "]";
    }
    case Value::kMap: case Value::kNs: {
        std::string o = "{";
        for (size_t k = 0; k < v.m->size(); k++) o += (k ? "," : "") + to_json(Value::str((*v.m)[k].first)) + ":" + to_json((*v.m)[k].second);
        return o + "}";
    }
    default: fail("cannot serialize a function");
    }
}

bool equal(const Value& a, const Value& b) {
    const bool an = a.kind == Value::kInt || a.kind == Value::kFloat || a.kind == Value::kBool;
    const bool bn = b.kind == Value::kInt || b.kind == Value::kFloat || b.kind == Value::kBool;
    if (an && bn) {
        if (a.kind == Value::kFloat || b.kind == Value::kFloat) {
            const double x = a.kind == Value::kFloat ? a.f : (double)(a.kind == Value::kInt ? a.i : a.b);
            const double y = b.kind == Value::kFloat ? b.f : (double)(b.kind == Value::kInt ? b.i : b.b);
            return x == y;
        }
        return (a.kind == Value::kInt ? a.i : a.b) == (b.kind == Value::kInt ? b.i : b.b);
    }
    if (a.kind != b.kind) return false;
    switch (a.kind) {
    case Value::kUndef: case Value::kNone: return true;
    case Value::kStr: return a.s == b.s;
    case Value::kList:
        if (a.l->size() != b.l->size()) return false;
        for (size_t k = 0; k < a.l->size(); k++)
            if (!equal((*a.l)[k], (*b.l)[k])) return false;
        return true;
    case Value::kMap: case Value::kNs:
        if (a.m->size() != b.m->size()) return false;
        for (size_t k = 0; k < a.m->size(); k++)
            if ((*a.m)[k].first != (*b.m)[k].first || !equal((*a.m)[k].second, (*b.m)[k].second)) return false;
        return true;
    default: return a.s == b.s;
    }
}

const Value* map_get(const Value& m, const std::string& k) {
    for (const auto& kv : *m.m)
        if (kv.first == k) return &kv.second;
    return nullptr;
}

// UTF-8 scalar values of s (invalid bytes pass as single units)
std::vector<std::string> utf8_chars(const std::string& s) {
    std::vector<std::string> out;
    for (size_t p = 0; p < s.size();) {
        const unsigned char c = (unsigned char)s[p];
        size_t len = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 1;
        if (p + len > s.size()) len = 1;
        out.push_back(s.substr(p, len));
        p += len;
    }
    return out;
}

// Rust str::trim (Unicode White_Space at both ends)
bool utf8_is_space_at(const std::string& s, size_t p, size_t* len);
std::string trim_ws(const std::string& s, bool left, bool right) {
    size_t b = 0, e = s.size(), len = 0;
    if (left)
        while (b < e && utf8_is_space_at(s, b, &len)) b += len;
    if (right)
        for (;;) {
            // find the start of the last character
            if (e <= b) break;
            size_t k = e - 1;
            while (k > b && ((unsigned char)s[k] & 0xC0) == 0x80) k--;
            if (!utf8_is_space_at(s, k, &len) || k + len != e) break;
            e = k;
        }
    return s.substr(b, e - b);
}
bool utf8_is_space_at(const std::string& s, size_t p, size_t* len) {
    const unsigned char c = (unsigned char)s[p];
    if (c < 0x80) {
        *len = 1;
        return (c >= 9 && c <= 13) || c == 32;
    }
    uint32_t cp = 0;
    size_t l = 0;
    if ((c >> 5) == 6 && p + 1 < s.size()) { cp = ((c & 0x1F) << 6) | (s[p + 1] & 0x3F); l = 2; }
    else if ((c >> 4) == 14 && p + 2 < s.size()) { cp = ((c & 0x0F) << 12) | ((s[p + 1] & 0x3F) << 6) | (s[p + 2] & 0x3F); l = 3; }
    else { *len = 1; return false; }
    *len = l;
    return cp == 0x85 || cp == 0xA0 || cp == 0x1680 || (cp >= 0x2000 && cp <= 0x200A) || cp == 0x2028 ||
           cp == 0x2029 || cp == 0x202F || cp == 0x205F || cp == 0x3000;
}

struct LoopInfo {
    int64_t index0 = 0, length = 0;
    Value prev, next;
};

class Renderer {
public:
    Renderer(const Value& ctx) : ctx_(ctx) { scopes_.emplace_back(); }

    void run(const std::vector<NodeP>& body, std::string* out) {
        for (const auto& n : body) exec(*n, out);
    }

private:
    const Value& ctx_;
    std::vector<std::map<std::string, Value>> scopes_;

    Value lookup(const std::string& nm) {
        for (auto it = scopes_.rbegin(); it != scopes_.rend(); ++it) {
            auto f = it->find(nm);
            if (f != it->end()) return f->second;
        }
        if (ctx_.kind == Value::kMap)
            if (const Value* v = map_get(ctx_, nm)) return *v;
        if (nm == "namespace" || nm == "range") {
            Value f;
            f.kind = Value::kFunc;
            f.s = nm;
            return f;
        }
        return Value::undef();
    }

    void exec(const Node& n, std::string* out) {
        switch (n.k) {
        case Node::Text: *out += n.text; break;
        case Node::Out: *out += to_str(eval(*n.e)); break;
        case Node::If:
            for (const auto& br : n.branches)
                if (truthy(eval(*br.first))) {
                    run(br.second, out);
                    return;
                }
            run(n.else_body, out);
            break;
        case Node::Set: {
            Value v = eval(*n.e);
            if (n.targets.size() == 1) {
                scopes_.back()[n.targets[0]] = v;
            } else {
                Value ns = lookup(n.targets[0]);
                if (ns.kind != Value::kNs) fail("cannot assign an attribute of a non-namespace value");
                for (auto& kv : *ns.m)
                    if (kv.first == n.targets[1]) { kv.second = v; return; }
                ns.m->push_back({n.targets[1], v});
            }
            break;
        }
        case Node::For: exec_for(n, out); break;
        }
    }

    std::vector<Value> iterate(const Value& v) {
        std::vector<Value> items;
        switch (v.kind) {
        case Value::kUndef: break;
        case Value::kList: items = *v.l; break;
        case Value::kMap: case Value::kNs: for (const auto& kv : *v.m) items.push_back(Value::str(kv.first)); break;
        case Value::kStr: for (auto& c : utf8_chars(v.s)) items.push_back(Value::str(c)); break;
        default: fail("cannot iterate over " + kind_name(v));
        }
        return items;
    }

    void exec_for(const Node& n, std::string* out) {
        std::vector<Value> items = iterate(eval(*n.e));
        if (n.filter) {
            std::vector<Value> kept;
            for (auto& it : items) {
                scopes_.emplace_back();
                bind_targets(n, it);
                if (truthy(eval(*n.filter))) kept.push_back(it);
                scopes_.pop_back();
            }
            items.swap(kept);
        }
        if (items.empty()) {
            run(n.else_body, out);
            return;
        }
        const int64_t len = (int64_t)items.size();
        for (int64_t k = 0; k < len; k++) {
            scopes_.emplace_back();
            bind_targets(n, items[k]);
            Map loop;
            loop.push_back({"index", Value::integer(k + 1)});
            loop.push_back({"index0", Value::integer(k)});
            loop.push_back({"revindex", Value::integer(len - k)});
            loop.push_back({"revindex0", Value::integer(len - k - 1)});
            loop.push_back({"first", Value::boolean(k == 0)});
            loop.push_back({"last", Value::boolean(k == len - 1)});
            loop.push_back({"length", Value::integer(len)});
            loop.push_back({"depth", Value::integer(1)});
            loop.push_back({"depth0", Value::integer(0)});
            loop.push_back({"previtem", k > 0 ? items[k - 1] : Value::undef()});
            loop.push_back({"nextitem", k + 1 < len ? items[k + 1] : Value::undef()});
            scopes_.back()["loop"] = Value::map(std::move(loop));
            run(n.body, out);
            scopes_.pop_back();
        }
    }

    void bind_targets(const Node& n, const Value& it) {
        if (n.targets.size() == 1) {
            scopes_.back()[n.targets[0]] = it;
            return;
        }
        std::vector<Value> parts = iterate(it);
        if (parts.size() != n.targets.size()) fail("cannot unpack a loop item");
        for (size_t k = 0; k < parts.size(); k++) scopes_.back()[n.targets[k]] = parts[k];
    }

    static double num(const Value& v) {
        if (v.kind == Value::kInt) return (double)v.i;
        if (v.kind == Value::kFloat) return v.f;
        if (v.kind == Value::kBool) return v.b ? 1.0 : 0.0;
        fail("expected a number, got " + kind_name(v));
    }
    static bool is_num(const Value& v) { return v.kind == Value::kInt || v.kind == Value::kFloat || v.kind == Value::kBool; }

    Value get_item(const Value& o, const Value& key) {
        if (o.kind == Value::kUndef) fail("undefined value has no items");
        if (o.kind == Value::kNone) fail("none has no items");
        if (o.kind == Value::kMap || o.kind == Value::kNs) {
            const Value* v = map_get(o, to_str(key));
            return v ? *v : Value::undef();
        }
        if ((o.kind == Value::kList || o.kind == Value::kStr) && key.kind == Value::kInt) {
            if (o.kind == Value::kList) {
                int64_t k = key.i < 0 ? key.i + (int64_t)o.l->size() : key.i;
                return k >= 0 && k < (int64_t)o.l->size() ? (*o.l)[k] : Value::undef();
            }
            auto cs = utf8_chars(o.s);
            int64_t k = key.i < 0 ? key.i + (int64_t)cs.size() : key.i;
            return k >= 0 && k < (int64_t)cs.size() ? Value::str(cs[k]) : Value::undef();
        }
        return Value::undef();
    }

    Value eval(const Expr& e) {
        switch (e.k) {
        case Expr::Lit: return e.lit;
        case Expr::Name: return lookup(e.name);
        case Expr::Attr: {
            Value o = eval(*e.a);
            if (o.kind == Value::kUndef) fail("undefined value has no attribute '" + e.name + "'");
            if (o.kind == Value::kNone) fail("none has no attribute '" + e.name + "'");
            if (o.kind == Value::kMap || o.kind == Value::kNs) {
                const Value* v = map_get(o, e.name);
                return v ? *v : Value::undef();
            }
            if (o.kind == Value::kList && !e.name.empty() && isdigit((unsigned char)e.name[0]))
                return get_item(o, Value::integer(strtoll(e.name.c_str(), nullptr, 10)));
            return Value::undef();
        }
        case Expr::Item: return get_item(eval(*e.a), eval(*e.b));
        case Expr::Slice: {
            Value o = eval(*e.a);
            const bool str = o.kind == Value::kStr;
            std::vector<Value> items;
            if (str) for (auto& c : utf8_chars(o.s)) items.push_back(Value::str(c));
            else if (o.kind == Value::kList) items = *o.l;
            else if (o.kind == Value::kUndef) return Value::undef();
            else fail("cannot slice " + kind_name(o));
            const int64_t n = (int64_t)items.size();
            auto clampi = [&](const ExprP& x, int64_t dflt) {
                if (!x) return dflt;
                Value v = eval(*x);
                if (v.kind == Value::kNone) return dflt;
                int64_t k = (int64_t)num(v);
                if (k < 0) k += n;
                return std::max<int64_t>(0, std::min<int64_t>(n, k));
            };
            const int64_t lo = clampi(e.b, 0), hi = clampi(e.c, n);
            std::vector<Value> sub;
            for (int64_t k = lo; k < hi; k++) sub.push_back(items[k]);
            if (str) {
                std::string s;
                for (auto& c : sub) s += c.s;
                return Value::str(s);
            }
            return Value::list(sub);
        }
        case Expr::Call: return call(e);
        case Expr::Filter: return filter(e);
        case Expr::Test: {
            const bool r = test(e);
            return Value::boolean(e.neg ? !r : r);
        }
        case Expr::Unary: {
            Value v = eval(*e.a);
            if (e.name == "not") return Value::boolean(!truthy(v));
            if (e.name == "-") {
                if (v.kind == Value::kInt) return Value::integer(-v.i);
                return Value::number(-num(v));
            }
            return v;
        }
        case Expr::Binary: return binary(e);
        case Expr::Cond:
            if (truthy(eval(*e.a))) return eval(*e.b);
            return e.c ? eval(*e.c) : Value::undef();
        case Expr::ListE: {
            List l;
            for (auto& x : e.args) l.push_back(eval(*x));
            return Value::list(l);
        }
        case Expr::MapE: {
            Map m;
            for (size_t k = 0; k < e.args.size(); k++) {
                const std::string key = to_str(eval(*e.args[k]));
                Value v = eval(*e.args2[k]);
                bool set = false;
                for (auto& kv : m)
                    if (kv.first == key) { kv.second = v; set = true; }
                if (!set) m.push_back({key, v});
            }
            return Value::map(m);
        }
        }
        fail("bad expression");
    }

    Value call(const Expr& e) {
        if (e.a->k == Expr::Attr) {
            Value o = eval(*e.a->a);
            fail("unknown method: " + kind_name(o) + " has no method named " + e.a->name);
        }
        Value f = eval(*e.a);
        if (f.kind != Value::kFunc) fail("cannot call " + kind_name(f) + " (" + (e.a->k == Expr::Name ? e.a->name : "") + ")");
        if (f.s == "namespace") {
            Value ns;
            ns.kind = Value::kNs;
            ns.m = std::make_shared<Map>();
            for (auto& a : e.args) {
                Value m = eval(*a);
                if (m.kind == Value::kMap) for (auto& kv : *m.m) ns.m->push_back(kv);
            }
            for (auto& kv : e.kwargs) ns.m->push_back({kv.first, eval(*kv.second)});
            return ns;
        }
        // range
        std::vector<int64_t> a;
        for (auto& x : e.args) a.push_back((int64_t)num(eval(*x)));
        int64_t lo = 0, hi = 0, st = 1;
        if (a.size() == 1) hi = a[0];
        else if (a.size() >= 2) { lo = a[0]; hi = a[1]; if (a.size() > 2) st = a[2]; }
        if (st == 0) fail("range step is zero");
        List l;
        for (int64_t k = lo; st > 0 ? k < hi : k > hi; k += st) {
            l.push_back(Value::integer(k));
            if (l.size() > 100000) fail("range too large");
        }
        return Value::list(l);
    }

    Value binary(const Expr& e) {
        if (e.name == "and") {
            Value l = eval(*e.a);
            return truthy(l) ? eval(*e.b) : l;
        }
        if (e.name == "or") {
            Value l = eval(*e.a);
            return truthy(l) ? l : eval(*e.b);
        }
        Value l = eval(*e.a), r = eval(*e.b);
        const std::string& op = e.name;
        if (op == "==") return Value::boolean(equal(l, r));
        if (op == "!=") return Value::boolean(!equal(l, r));
        if (op == "in" || op == "notin") {
            bool found = false;
            if (r.kind == Value::kStr) found = r.s.find(to_str(l)) != std::string::npos;
            else if (r.kind == Value::kList) { for (auto& x : *r.l) if (equal(x, l)) { found = true; break; } }
            else if (r.kind == Value::kMap || r.kind == Value::kNs) found = map_get(r, to_str(l)) != nullptr;
            else if (r.kind == Value::kUndef) found = false;
            else fail("cannot test membership in " + kind_name(r));
            return Value::boolean(op == "in" ? found : !found);
        }
        if (op == "~") return Value::str(to_str(l) + to_str(r));
        if (op == "<" || op == ">" || op == "<=" || op == ">=") {
            int c;
            if (l.kind == Value::kStr && r.kind == Value::kStr) c = l.s < r.s ? -1 : (l.s > r.s ? 1 : 0);
            else {
                const double x = num(l), y = num(r);
                c = x < y ? -1 : (x > y ? 1 : 0);
            }
            return Value::boolean(op == "<" ? c < 0 : op == ">" ? c > 0 : op == "<=" ? c <= 0 : c >= 0);
        }
        if (op == "+") {
            if (l.kind == Value::kStr && r.kind == Value::kStr) return Value::str(l.s + r.s);
            if (l.kind == Value::kList && r.kind == Value::kList) {
                List x = *l.l;
                x.insert(x.end(), r.l->begin(), r.l->end());
                return Value::list(x);
            }
            if (!is_num(l) || !is_num(r)) fail("unsupported operation: " + kind_name(l) + " + " + kind_name(r));
        }
        if (!is_num(l) || !is_num(r)) fail("unsupported operation " + op + " on " + kind_name(l) + " and " + kind_name(r));
        const bool ints = l.kind != Value::kFloat && r.kind != Value::kFloat;
        const int64_t li = l.kind == Value::kBool ? l.b : l.i, ri = r.kind == Value::kBool ? r.b : r.i;
        if (op == "+") return ints ? Value::integer(li + ri) : Value::number(num(l) + num(r));
        if (op == "-") return ints ? Value::integer(li - ri) : Value::number(num(l) - num(r));
        if (op == "*") {
            return ints ? Value::integer(li * ri) : Value::number(num(l) * num(r));
        }
        if (op == "/") {
            if (num(r) == 0.0) fail("division by zero");
            return Value::number(num(l) / num(r));
        }
        if (op == "//") {
            if (num(r) == 0.0) fail("division by zero");
            if (ints) {
                int64_t q = li / ri;
                if ((li % ri != 0) && ((li < 0) != (ri < 0))) q--;
                return Value::integer(q);
            }
            return Value::number(floor(num(l) / num(r)));
        }
        if (op == "%") {
            if (num(r) == 0.0) fail("division by zero");
            if (ints) {
                int64_t m = li % ri;
                if (m != 0 && ((m < 0) != (ri < 0))) m += ri;
                return Value::integer(m);
            }
            return Value::number(fmod(num(l), num(r)));
        }
        if (op == "**") return ints && ri >= 0 ? Value::integer((int64_t)llround(pow((double)li, (double)ri)))
                                               : Value::number(pow(num(l), num(r)));
        fail("unknown operator " + op);
    }

    bool test(const Expr& e) {
        const std::string& t = e.name;
        if (t == "defined") return eval(*e.a).kind != Value::kUndef;
        if (t == "undefined") return eval(*e.a).kind == Value::kUndef;
        Value v = eval(*e.a);
        if (t == "none") return v.kind == Value::kNone;
        if (t == "string") return v.kind == Value::kStr;
        if (t == "number") return v.kind == Value::kInt || v.kind == Value::kFloat;
        if (t == "integer") return v.kind == Value::kInt;
        if (t == "float") return v.kind == Value::kFloat;
        if (t == "boolean") return v.kind == Value::kBool;
        if (t == "true") return v.kind == Value::kBool && v.b;
        if (t == "false") return v.kind == Value::kBool && !v.b;
        if (t == "mapping") return v.kind == Value::kMap || v.kind == Value::kNs;
        if (t == "sequence") return v.kind == Value::kList || v.kind == Value::kStr;
        if (t == "iterable") return v.kind == Value::kList || v.kind == Value::kStr || v.kind == Value::kMap;
        if (t == "callable") return v.kind == Value::kFunc;
        if (t == "odd" || t == "even") {
            const int64_t k = (int64_t)num(v);
            return (k % 2 != 0) == (t == "odd");
        }
        std::vector<Value> a;
        for (auto& x : e.args) a.push_back(eval(*x));
        if (t == "divisibleby") {
            if (a.empty() || num(a[0]) == 0.0) fail("divisibleby needs a nonzero argument");
            return fmod(num(v), num(a[0])) == 0.0;
        }
        if (a.empty()) fail("unknown test: " + t);
        if (t == "eq" || t == "equalto" || t == "sameas") return equal(v, a[0]);
        if (t == "ne") return !equal(v, a[0]);
        if (t == "lt" || t == "lessthan") return num(v) < num(a[0]);
        if (t == "gt" || t == "greaterthan") return num(v) > num(a[0]);
        if (t == "le") return num(v) <= num(a[0]);
        if (t == "ge") return num(v) >= num(a[0]);
        if (t == "in") {
            Expr b;
            b.k = Expr::Binary;
            b.name = "in";
            auto lit = [](const Value& x) { auto p = std::make_shared<Expr>(); p->k = Expr::Lit; p->lit = x; return p; };
            b.a = lit(v);
            b.b = lit(a[0]);
            return truthy(binary(b));
        }
        if (t == "startingwith") return v.kind == Value::kStr && v.s.rfind(to_str(a[0]), 0) == 0;
        if (t == "endingwith") {
            const std::string suf = to_str(a[0]);
            return v.kind == Value::kStr && v.s.size() >= suf.size() && v.s.compare(v.s.size() - suf.size(), suf.size(), suf) == 0;
        }
        fail("unknown test: " + t);
    }

    Value filter(const Expr& e) {
        const std::string& f = e.name;
        Value v = eval(*e.a);
        std::vector<Value> a;
        for (auto& x : e.args) a.push_back(eval(*x));
        auto kw = [&](const char* name) -> const ExprP* {
            for (auto& kv : e.kwargs)
                if (kv.first == name) return &kv.second;
            return nullptr;
        };
        if (f == "default" || f == "d") {
            const bool boolean = (a.size() > 1 && truthy(a[1])) || (kw("boolean") && truthy(eval(**kw("boolean"))));
            const Value dflt = a.empty() ? Value::str("") : a[0];
            if (v.kind == Value::kUndef || (boolean && !truthy(v))) return dflt;
            return v;
        }
        if (f == "safe" || f == "escape" || f == "e") return v.kind == Value::kStr ? v : Value::str(to_str(v));
        if (f == "trim") {
            if (v.kind == Value::kUndef) return Value::str("");
            const std::string s = to_str(v);
            if (a.empty()) return Value::str(trim_ws(s));
            const std::string chars = to_str(a[0]);
            size_t b = s.find_first_not_of(chars);
            if (b == std::string::npos) return Value::str("");
            size_t en = s.find_last_not_of(chars);
            return Value::str(s.substr(b, en - b + 1));
        }
        if (f == "length" || f == "count") {
            if (v.kind == Value::kStr) return Value::integer((int64_t)utf8_chars(v.s).size());
            if (v.kind == Value::kList) return Value::integer((int64_t)v.l->size());
            if (v.kind == Value::kMap || v.kind == Value::kNs) return Value::integer((int64_t)v.m->size());
            if (v.kind == Value::kUndef) return Value::integer(0);
            fail("cannot take the length of " + kind_name(v));
        }
        if (f == "upper" || f == "lower") {
            std::string s = to_str(v);
            for (auto& c : s)
                if ((unsigned char)c < 0x80) c = f == "upper" ? (char)toupper(c) : (char)tolower(c);
            return Value::str(s);
        }
        if (f == "capitalize") {
            std::string s = to_str(v);
            for (size_t k = 0; k < s.size(); k++)
                if ((unsigned char)s[k] < 0x80) s[k] = k == 0 ? (char)toupper(s[k]) : (char)tolower(s[k]);
            return Value::str(s);
        }
        if (f == "title") {
            std::string s = to_str(v);
            bool start = true;
            for (auto& c : s) {
                if ((unsigned char)c >= 0x80) { start = false; continue; }
                if (isalnum((unsigned char)c)) { c = start ? (char)toupper(c) : (char)tolower(c); start = false; }
                else start = true;
            }
            return Value::str(s);
        }
        if (f == "replace") {
            if (a.size() < 2) fail("replace needs two arguments");
            std::string s = to_str(v);
            const std::string from = to_str(a[0]), to = to_str(a[1]);
            if (from.empty()) return Value::str(s);
            std::string o;
            size_t p = 0, q;
            while ((q = s.find(from, p)) != std::string::npos) {
                o += s.substr(p, q - p) + to;
                p = q + from.size();
            }
            return Value::str(o + s.substr(p));
        }
        if (f == "first" || f == "last") {
            std::vector<Value> it = iterate(v);
            if (it.empty()) return Value::undef();
            return f == "first" ? it.front() : it.back();
        }
        if (f == "join") {
            std::vector<Value> it = iterate(v);
            const std::string sep = a.empty() ? "" : to_str(a[0]);
            std::string o;
            for (size_t k = 0; k < it.size(); k++) o += (k ? sep : "") + to_str(it[k]);
            return Value::str(o);
        }
        if (f == "reverse") {
            if (v.kind == Value::kStr) {
                auto cs = utf8_chars(v.s);
                std::string o;
                for (auto it = cs.rbegin(); it != cs.rend(); ++it) o += *it;
                return Value::str(o);
            }
            std::vector<Value> it = iterate(v);
            std::reverse(it.begin(), it.end());
            return Value::list(it);
        }
        if (f == "list") return Value::list(iterate(v));
        if (f == "string") return Value::str(to_str(v));
        if (f == "int") {
            if (v.kind == Value::kStr) return Value::integer(strtoll(trim_ws(v.s).c_str(), nullptr, 10));
            if (v.kind == Value::kUndef || v.kind == Value::kNone) return Value::integer(0);
            return Value::integer((int64_t)num(v));
        }
        if (f == "float") {
            if (v.kind == Value::kStr) return Value::number(strtod(v.s.c_str(), nullptr));
            return Value::number(num(v));
        }
        if (f == "abs") return v.kind == Value::kInt ? Value::integer(v.i < 0 ? -v.i : v.i) : Value::number(fabs(num(v)));
        if (f == "items") {
            if (v.kind != Value::kMap && v.kind != Value::kNs) fail("items needs a map");
            List l;
            for (auto& kv : *v.m) l.push_back(Value::list({Value::str(kv.first), kv.second}));
            return Value::list(l);
        }
        if (f == "tojson") return Value::str(to_json(v));
        fail("unknown filter: " + f);
    }
};

}  // namespace

bool render(const std::string& source, const Value& ctx, std::string* out, std::string* err) {
    try {
        Parser p(lex(source));
        std::vector<NodeP> body = p.parse_all();
        Renderer r(ctx);
        out->clear();
        r.run(body, out);
        return true;
    } catch (const RenderError& e) {
        *err = "chat template: " + e.msg;
        return false;
    }
}

}  // namespace jinja
}  // namespace yl
