// yl_jinja.h -- the subset of Jinja that GGUF chat templates use, for the
// tokenizer's chat-template path (tokenizer.rs:391-456, which renders
// `tokenizer.chat_template` with minijinja 2.x defaults and the context
// {"messages": [{"role", "content"}...], "add_generation_prompt": bool}).
//
// Semantics follow minijinja's defaults: lenient undefined values (print as
// "", iterate as empty, are false; reading an attribute of one is an error),
// no Python string methods (`.strip()` and the like are errors without the
// pycompat extension), a single trailing newline of the template dropped,
// no auto-escaping.  Supported: {{ }}, {% if/elif/else %}, {% for %} (with
// `loop`, an `if` filter and `else`), {% set %} (names and namespace
// attributes), {# #}, whitespace control (- on either side), literals,
// lists, dicts, attribute/item/slice access, the Jinja operator precedence,
// tests (defined, none, string, ...) and the common filters.  Anything else
// is a render error, as an unsupported construct would be for a host.
#pragma once

#include <stdint.h>

#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace yl {
namespace jinja {

struct Value;
using List = std::vector<Value>;
using Map = std::vector<std::pair<std::string, Value>>;   // insertion-ordered

struct Value {
    enum Kind { kUndef, kNone, kBool, kInt, kFloat, kStr, kList, kMap, kNs, kFunc } kind = kUndef;
    bool b = false;
    int64_t i = 0;
    double f = 0.0;
    std::string s;                 // kStr text, kFunc name
    std::shared_ptr<List> l;       // kList
    std::shared_ptr<Map> m;        // kMap, kNs (a namespace is a mutable map)

    static Value undef() { return Value(); }
    static Value none() { Value v; v.kind = kNone; return v; }
    static Value boolean(bool x) { Value v; v.kind = kBool; v.b = x; return v; }
    static Value integer(int64_t x) { Value v; v.kind = kInt; v.i = x; return v; }
    static Value number(double x) { Value v; v.kind = kFloat; v.f = x; return v; }
    static Value str(std::string x) { Value v; v.kind = kStr; v.s = std::move(x); return v; }
    static Value list(List x) { Value v; v.kind = kList; v.l = std::make_shared<List>(std::move(x)); return v; }
    static Value map(Map x) { Value v; v.kind = kMap; v.m = std::make_shared<Map>(std::move(x)); return v; }
};

// Renders `source` with the context map `ctx`.  Returns false and sets *err
// on a syntax or render error.
bool render(const std::string& source, const Value& ctx, std::string* out, std::string* err);

}  // namespace jinja
}  // namespace yl
