// A small JSON reader (document model + strict recursive-descent parser),
// shared by the .intfer metadata reader and the serve loop's request lines.
#pragma once
#include <cerrno>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

namespace ifrh {

struct JNode {
  enum Kind { Null, Bool, Int, Real, Str, Arr, Obj } kind = Null;
  bool b = false;
  int64_t i = 0;
  double d = 0;
  std::string s;
  std::vector<JNode> items;                           // Arr
  std::vector<std::pair<std::string, JNode>> fields;  // Obj, file order

  // First field named `key` (as the reference's lookup), or nullptr.
  const JNode* at(const char* key) const {
    if (kind != Obj) return nullptr;
    for (const auto& f : fields)
      if (f.first == key) return &f.second;
    return nullptr;
  }
  const JNode* at(const char* key, Kind k) const {
    const JNode* n = at(key);
    return n && n->kind == k ? n : nullptr;
  }
};

class JReader {
 public:
  JReader(const char* b, const char* e) : p_(b), e_(e) {}
  bool document(JNode& out) {
    if (!value(out, 0)) return false;
    ws();
    return p_ == e_;  // nothing but whitespace after the root
  }

 private:
  const char* p_;
  const char* e_;

  void ws() {
    while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
  }
  bool lit(const char* w) {
    const size_t n = std::strlen(w);
    if ((size_t)(e_ - p_) < n || std::memcmp(p_, w, n) != 0) return false;
    p_ += n;
    return true;
  }
  bool value(JNode& v, int depth) {
    if (depth > 64) return false;
    ws();
    if (p_ >= e_) return false;
    switch (*p_) {
      case '{': return object(v, depth);
      case '[': return array(v, depth);
      case '"': v.kind = JNode::Str; return string(v.s);
      case 't': v.kind = JNode::Bool; v.b = true; return lit("true");
      case 'f': v.kind = JNode::Bool; v.b = false; return lit("false");
      case 'n': v.kind = JNode::Null; return lit("null");
      default: return number(v);
    }
  }
  bool object(JNode& v, int depth) {
    v.kind = JNode::Obj;
    ++p_;
    ws();
    if (p_ < e_ && *p_ == '}') { ++p_; return true; }
    for (;;) {
      ws();
      std::string key;
      if (p_ >= e_ || *p_ != '"' || !string(key)) return false;
      ws();
      if (p_ >= e_ || *p_ != ':') return false;
      ++p_;
      v.fields.emplace_back(std::move(key), JNode());
      if (!value(v.fields.back().second, depth + 1)) return false;
      ws();
      if (p_ < e_ && *p_ == ',') { ++p_; continue; }
      if (p_ < e_ && *p_ == '}') { ++p_; return true; }
      return false;
    }
  }
  bool array(JNode& v, int depth) {
    v.kind = JNode::Arr;
    ++p_;
    ws();
    if (p_ < e_ && *p_ == ']') { ++p_; return true; }
    for (;;) {
      v.items.emplace_back();
      if (!value(v.items.back(), depth + 1)) return false;
      ws();
      if (p_ < e_ && *p_ == ',') { ++p_; continue; }
      if (p_ < e_ && *p_ == ']') { ++p_; return true; }
      return false;
    }
  }
  static void utf8(std::string& o, uint32_t cp) {
    if (cp < 0x80) {
      o += (char)cp;
    } else if (cp < 0x800) {
      o += (char)(0xC0 | cp >> 6);
      o += (char)(0x80 | (cp & 0x3F));
    } else {
      o += (char)(0xE0 | cp >> 12);
      o += (char)(0x80 | ((cp >> 6) & 0x3F));
      o += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool string(std::string& o) {
    ++p_;  // opening quote
    while (p_ < e_ && *p_ != '"') {
      const char c = *p_++;
      if (c != '\\') { o += c; continue; }
      if (p_ >= e_) return false;
      const char x = *p_++;
      switch (x) {
        case '"': o += '"'; break;
        case '\\': o += '\\'; break;
        case '/': o += '/'; break;
        case 'b': o += '\b'; break;
        case 'f': o += '\f'; break;
        case 'n': o += '\n'; break;
        case 'r': o += '\r'; break;
        case 't': o += '\t'; break;
        case 'u': {
          if (e_ - p_ < 4) return false;
          uint32_t cp = 0;
          for (int k = 0; k < 4; ++k) {
            const char h = *p_++;
            cp <<= 4;
            if (h >= '0' && h <= '9') cp |= (uint32_t)(h - '0');
            else if (h >= 'a' && h <= 'f') cp |= (uint32_t)(h - 'a' + 10);
            else if (h >= 'A' && h <= 'F') cp |= (uint32_t)(h - 'A' + 10);
            else return false;
          }
          utf8(o, cp);
          break;
        }
        default: return false;
      }
    }
    if (p_ >= e_) return false;
    ++p_;  // closing quote
    return true;
  }
  // JSON number; integral tokens (no '.', 'e', 'E') become Int, as in the
  // reference reader, so a field it reads as an integer is read the same here.
  bool number(JNode& v) {
    const char* s = p_;
    if (p_ < e_ && *p_ == '-') ++p_;
    const char* digits = p_;
    while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
    if (p_ == digits) return false;
    bool real = false;
    if (p_ < e_ && *p_ == '.') {
      real = true;
      ++p_;
      const char* f = p_;
      while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
      if (p_ == f) return false;
    }
    if (p_ < e_ && (*p_ == 'e' || *p_ == 'E')) {
      real = true;
      ++p_;
      if (p_ < e_ && (*p_ == '+' || *p_ == '-')) ++p_;
      const char* x = p_;
      while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
      if (p_ == x) return false;
    }
    const std::string tok(s, p_);
    char* end = nullptr;
    errno = 0;
    if (real) {
      v.kind = JNode::Real;
      v.d = std::strtod(tok.c_str(), &end);
    } else {
      v.kind = JNode::Int;
      v.i = std::strtoll(tok.c_str(), &end, 10);
      if (errno == ERANGE) return false;
    }
    return end == tok.c_str() + tok.size();
  }
};

}  // namespace ifrh
