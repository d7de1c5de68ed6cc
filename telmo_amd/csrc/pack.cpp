// Reader of the reference's weight files ("packs", src/pack.rs), so that a model's int8 / Q8_0
// matrices go from the file to the device in one upload each.
//
// The file (src/pack.rs:1-13): "TELMOPAK", a little-endian u32 version (1), 4 zero bytes; the
// entries' data at offsets that are multiples of 64; a JSON index; the index's offset and length
// as little-endian u64s, then "TELMOIDX". The checks and their messages follow Pack::parse
// (src/pack.rs:98-259) in order, and the JSON reader follows src/json.rs:146-390 (depth limit
// 128, duplicate keys refused, strings validated as UTF-8, numbers kept as text). The file is
// mapped read-only; entries are views into the mapping, valid until tg_pack_close.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <utility>
#include <vector>

#include "../../include/telmo_hip.h"

namespace {

thread_local std::string g_pack_error;

int pack_fail(int code, const std::string &msg) {
    g_pack_error = msg;
    return code;
}

// ---------------------------------------------------------------------------- JSON (src/json.rs)

struct JValue {
    enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
    bool b = false;
    std::string text;  // number text or string value
    std::vector<JValue> items;
    std::vector<std::pair<std::string, JValue>> members;

    const JValue *get(const char *key) const {
        if (kind != Object) return nullptr;
        for (const auto &m : members)
            if (m.first == key) return &m.second;
        return nullptr;
    }
    // Value::as_u64 (src/json.rs:68-73): the number text parses as a u64 (digits only).
    bool as_u64(uint64_t &out) const {
        if (kind != Number || text.empty()) return false;
        uint64_t v = 0;
        for (char c : text) {
            if (c < '0' || c > '9') return false;
            const uint64_t d = (uint64_t)(c - '0');
            if (v > (UINT64_MAX - d) / 10) return false;
            v = v * 10 + d;
        }
        out = v;
        return true;
    }
};

struct JsonError {
    size_t offset;
    const char *message;
};

bool valid_utf8(const std::string &s) {
    size_t i = 0, n = s.size();
    while (i < n) {
        const unsigned char c = (unsigned char)s[i];
        size_t len;
        uint32_t cp;
        if (c < 0x80) {
            i++;
            continue;
        } else if ((c & 0xe0) == 0xc0) {
            len = 2;
            cp = c & 0x1f;
        } else if ((c & 0xf0) == 0xe0) {
            len = 3;
            cp = c & 0x0f;
        } else if ((c & 0xf8) == 0xf0) {
            len = 4;
            cp = c & 0x07;
        } else {
            return false;
        }
        if (i + len > n) return false;
        for (size_t j = 1; j < len; j++) {
            const unsigned char cc = (unsigned char)s[i + j];
            if ((cc & 0xc0) != 0x80) return false;
            cp = (cp << 6) | (cc & 0x3f);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) || cp > 0x10ffff ||
            (cp >= 0xd800 && cp < 0xe000))
            return false;
        i += len;
    }
    return true;
}

void put_utf8(std::string &out, uint32_t cp) {
    if (cp < 0x80) {
        out += (char)cp;
    } else if (cp < 0x800) {
        out += (char)(0xc0 | (cp >> 6));
        out += (char)(0x80 | (cp & 0x3f));
    } else if (cp < 0x10000) {
        out += (char)(0xe0 | (cp >> 12));
        out += (char)(0x80 | ((cp >> 6) & 0x3f));
        out += (char)(0x80 | (cp & 0x3f));
    } else {
        out += (char)(0xf0 | (cp >> 18));
        out += (char)(0x80 | ((cp >> 12) & 0x3f));
        out += (char)(0x80 | ((cp >> 6) & 0x3f));
        out += (char)(0x80 | (cp & 0x3f));
    }
}

class Json {
  public:
    Json(const uint8_t *text, size_t len) : t_(text), n_(len) {}

    JValue document() {
        skip();
        JValue v = value(0);
        skip();
        if (pos_ != n_) throw err("text after the value");
        return v;
    }

  private:
    static constexpr size_t MAX_DEPTH = 128;
    const uint8_t *t_;
    size_t n_, pos_ = 0;

    JsonError err(const char *m) const { return JsonError{pos_, m}; }
    int peek() const { return pos_ < n_ ? t_[pos_] : -1; }
    void skip() {
        while (pos_ < n_ && (t_[pos_] == ' ' || t_[pos_] == '\t' || t_[pos_] == '\n' || t_[pos_] == '\r')) pos_++;
    }
    void word(const char *w) {
        const size_t len = strlen(w);
        if (n_ - pos_ < len || memcmp(t_ + pos_, w, len) != 0) throw err("unknown word");
        pos_ += len;
    }
    JValue value(size_t depth) {
        if (depth >= MAX_DEPTH) throw err("nested too deeply");
        JValue v;
        switch (peek()) {
        case -1: throw err("unexpected end");
        case 'n': word("null"); return v;
        case 't': word("true"); v.kind = JValue::Bool; v.b = true; return v;
        case 'f': word("false"); v.kind = JValue::Bool; return v;
        case '"': v.kind = JValue::String; v.text = string(); return v;
        case '[': return array(depth);
        case '{': return object(depth);
        default:
            if (peek() == '-' || (peek() >= '0' && peek() <= '9')) return number();
            throw err("unexpected character");
        }
    }
    JValue array(size_t depth) {
        pos_++;
        JValue v;
        v.kind = JValue::Array;
        skip();
        if (peek() == ']') {
            pos_++;
            return v;
        }
        for (;;) {
            skip();
            v.items.push_back(value(depth + 1));
            skip();
            if (peek() == ',') {
                pos_++;
            } else if (peek() == ']') {
                pos_++;
                return v;
            } else {
                throw err("expected , or ]");
            }
        }
    }
    JValue object(size_t depth) {
        pos_++;
        JValue v;
        v.kind = JValue::Object;
        skip();
        if (peek() == '}') {
            pos_++;
            return v;
        }
        for (;;) {
            skip();
            if (peek() != '"') throw err("expected a string key");
            std::string key = string();
            skip();
            if (peek() != ':') throw err("expected :");
            pos_++;
            skip();
            JValue item = value(depth + 1);
            v.members.emplace_back(std::move(key), std::move(item));
            skip();
            if (peek() == ',') {
                pos_++;
            } else if (peek() == '}') {
                pos_++;
                break;
            } else {
                throw err("expected , or }");
            }
        }
        std::vector<const std::string *> keys;
        for (const auto &m : v.members) keys.push_back(&m.first);
        std::sort(keys.begin(), keys.end(), [](const std::string *a, const std::string *b) { return *a < *b; });
        for (size_t i = 1; i < keys.size(); i++)
            if (*keys[i] == *keys[i - 1]) throw err("duplicate key");
        return v;
    }
    void digits() {
        while (peek() >= '0' && peek() <= '9') pos_++;
    }
    JValue number() {
        const size_t start = pos_;
        if (peek() == '-') pos_++;
        if (peek() == '0')
            pos_++;
        else if (peek() >= '1' && peek() <= '9')
            digits();
        else
            throw err("expected a digit");
        if (peek() == '.') {
            pos_++;
            if (!(peek() >= '0' && peek() <= '9')) throw err("expected a digit after .");
            digits();
        }
        if (peek() == 'e' || peek() == 'E') {
            pos_++;
            if (peek() == '+' || peek() == '-') pos_++;
            if (!(peek() >= '0' && peek() <= '9')) throw err("expected a digit in the exponent");
            digits();
        }
        JValue v;
        v.kind = JValue::Number;
        v.text.assign(reinterpret_cast<const char *>(t_ + start), pos_ - start);
        return v;
    }
    uint32_t hex4() {
        if (n_ - pos_ < 4) throw err("expected four hex digits");
        uint32_t v = 0;
        for (int i = 0; i < 4; i++) {
            const int c = t_[pos_ + i];
            int d;
            if (c >= '0' && c <= '9')
                d = c - '0';
            else if (c >= 'a' && c <= 'f')
                d = c - 'a' + 10;
            else if (c >= 'A' && c <= 'F')
                d = c - 'A' + 10;
            else
                throw err("expected four hex digits");
            v = v * 16 + (uint32_t)d;
        }
        pos_ += 4;
        return v;
    }
    std::string string() {
        pos_++;
        std::string out;
        for (;;) {
            const size_t run = pos_;
            while (pos_ < n_ && t_[pos_] != '"' && t_[pos_] != '\\' && t_[pos_] >= 0x20) pos_++;
            out.append(reinterpret_cast<const char *>(t_ + run), pos_ - run);
            const int c = peek();
            if (c == -1) throw err("unterminated string");
            if (c == '"') {
                pos_++;
                break;
            }
            if (c != '\\') throw err("control character in a string");
            pos_++;
            const int e = peek();
            if (e == -1) throw err("unterminated escape");
            pos_++;
            switch (e) {
            case '"': out += '"'; break;
            case '\\': out += '\\'; break;
            case '/': out += '/'; break;
            case 'b': out += '\x08'; break;
            case 'f': out += '\x0c'; break;
            case 'n': out += '\n'; break;
            case 'r': out += '\r'; break;
            case 't': out += '\t'; break;
            case 'u': {
                const uint32_t first = hex4();
                uint32_t code = first;
                if (first >= 0xd800 && first < 0xdc00) {
                    if (n_ - pos_ < 2 || t_[pos_] != '\\' || t_[pos_ + 1] != 'u') throw err("unpaired surrogate");
                    pos_ += 2;
                    const uint32_t second = hex4();
                    if (second < 0xdc00 || second >= 0xe000) throw err("unpaired surrogate");
                    code = 0x10000 + ((first - 0xd800) << 10) + (second - 0xdc00);
                } else if (first >= 0xdc00 && first < 0xe000) {
                    throw err("unpaired surrogate");
                }
                put_utf8(out, code);
                break;
            }
            default: throw err("unknown escape");
            }
        }
        if (!valid_utf8(out)) throw err("invalid UTF-8 in a string");
        return out;
    }
};

// ---------------------------------------------------------------------------- the pack

constexpr size_t PREFIX = 16, TRAILER = 24, ALIGN = 64;
constexpr uint64_t MAX_INDEX = 64ull << 20;
constexpr uint32_t VERSION = 1;

const char *const PRECISION_NAMES[] = {"f32", "f16", "bf16", "int8", "q8_0"};  // src/quant.rs:41-49

}  // namespace

struct tg_pack {
    const uint8_t *data = nullptr;
    size_t len = 0;
    bool mapped = false;
    std::vector<uint8_t> copy;  // when not mapped
    std::string model;
    std::vector<std::pair<std::string, std::string>> metadata;
    struct Item {
        std::string name;
        uint32_t type = 0, precision = 0;
        size_t n = 0, k = 0, rank = 0, shape[8] = {0};
        size_t offset = 0, bytes = 0, scales_offset = 0, scales_bytes = 0;
        bool has_scales = false;
    };
    std::vector<Item> items;
    std::map<std::string, size_t> by_name;

    ~tg_pack() {
        if (mapped && data) munmap(const_cast<uint8_t *>(data), len);
    }
};

namespace {

int bad(const std::string &message) { return pack_fail(TG_ERR_ARG, "The pack file isn't usable. " + message); }

// Pack::parse (src/pack.rs:98-259).
int parse(tg_pack &p) {
    const uint8_t *d = p.data;
    const size_t len = p.len;
    if (len < PREFIX + TRAILER || memcmp(d, "TELMOPAK", 8) != 0) return bad("It isn't a pack.");
    uint32_t version;
    memcpy(&version, d + 8, 4);
    if (version != VERSION)
        return pack_fail(TG_ERR_ARG, "The pack has format version " + std::to_string(version) +
                                         ", and this version of the engine reads " + std::to_string(VERSION) +
                                         ". Convert the model again.");
    const uint8_t *trailer = d + len - TRAILER;
    if (memcmp(trailer + 16, "TELMOIDX", 8) != 0) return bad("Its index is missing, so the file may be cut short.");
    uint64_t index_at, index_len;
    memcpy(&index_at, trailer, 8);
    memcpy(&index_len, trailer + 8, 8);
    if (index_len > MAX_INDEX || index_at < PREFIX || index_at > UINT64_MAX - index_len ||
        index_at + index_len != (uint64_t)(len - TRAILER))
        return bad("Its index is out of place.");
    JValue root;
    try {
        root = Json(d + index_at, (size_t)index_len).document();
    } catch (const JsonError &e) {
        return pack_fail(TG_ERR_ARG, std::string("JSON error at byte ") + std::to_string(e.offset) + ": " + e.message);
    }
    const JValue *model = root.get("model");
    if (!model || model->kind != JValue::String) return bad("The index names no model.");
    p.model = model->text;
    if (const JValue *meta = root.get("metadata"); meta && meta->kind == JValue::Object) {
        for (const auto &m : meta->members) {
            if (m.second.kind != JValue::String) return bad("A metadata value isn't a string.");
            p.metadata.emplace_back(m.first, m.second.text);
        }
    }
    const JValue *list = root.get("entries");
    if (!list || list->kind != JValue::Array) return bad("The index lists no entries.");
    std::vector<std::pair<size_t, size_t>> ranges;
    for (const JValue &item : list->items) {
        const JValue *nm = item.get("name");
        if (!nm || nm->kind != JValue::String) return bad("An entry has no name.");
        tg_pack::Item e;
        e.name = nm->text;
        auto num = [&](const char *key, size_t &out) -> int {
            uint64_t v;
            const JValue *x = item.get(key);
            if (!x || !x->as_u64(v) || v >= (1ull << 40))
                return bad("Entry " + e.name + " has no valid " + key + ".");
            out = (size_t)v;
            return TG_OK;
        };
        const JValue *type = item.get("type");
        const std::string ty = type && type->kind == JValue::String ? type->text : "";
        int rc;
        if (ty == "matrix") {
            e.type = TG_ENTRY_MATRIX;
            const JValue *prec = item.get("precision");
            int found = -1;
            if (prec && prec->kind == JValue::String)
                for (int i = 0; i < 5; i++)
                    if (prec->text == PRECISION_NAMES[i]) found = i;
            if (found < 0) return bad("Entry " + e.name + " has an unknown precision.");
            e.precision = (uint32_t)found;
            if ((rc = num("n", e.n)) || (rc = num("k", e.k))) return rc;
            if (e.n == 0 || e.k == 0 || e.n > (1u << 24) || e.k > (1u << 24) || !tg_fits(e.precision, e.k))
                return bad("Entry " + e.name + " has an impossible shape.");
        } else if (ty == "f32") {
            e.type = TG_ENTRY_F32;
            const JValue *shape = item.get("shape");
            bool ok = shape && shape->kind == JValue::Array && shape->items.size() <= 8;
            if (ok) {
                e.rank = shape->items.size();
                for (size_t i = 0; i < e.rank && ok; i++) {
                    uint64_t v;
                    ok = shape->items[i].as_u64(v);
                    e.shape[i] = (size_t)v;
                }
            }
            if (!ok) return bad("Entry " + e.name + " has no valid shape.");
        } else if (ty == "bytes") {
            e.type = TG_ENTRY_BYTES;
        } else {
            return bad("Entry " + e.name + " has an unknown type.");
        }
        if ((rc = num("offset", e.offset)) || (rc = num("bytes", e.bytes))) return rc;
        bool size_ok;
        if (e.type == TG_ENTRY_MATRIX) {
            size_ok = tg_panel_bytes(e.precision, e.n, e.k) == e.bytes;
        } else if (e.type == TG_ENTRY_F32) {
            size_t expect = 4;
            bool overflow = false;
            for (size_t i = 0; i < e.rank; i++) {
                if (e.shape[i] != 0 && expect > SIZE_MAX / e.shape[i]) overflow = true;
                expect *= e.shape[i];
            }
            size_ok = !overflow && expect == e.bytes;
        } else {
            size_ok = true;
        }
        if (!size_ok) return bad("Entry " + e.name + " has the wrong size.");
        auto check_range = [&](size_t offset, size_t bytes) -> int {
            if (offset < PREFIX || offset % ALIGN != 0 || offset > SIZE_MAX - bytes || offset + bytes > index_at)
                return bad("Entry " + e.name + " is out of place.");
            ranges.emplace_back(offset, offset + bytes);
            return TG_OK;
        };
        if ((rc = check_range(e.offset, e.bytes))) return rc;
        if (e.type == TG_ENTRY_MATRIX && tg_scale_count(e.precision, e.n, e.k) > 0) {
            if ((rc = num("scales_bytes", e.scales_bytes))) return rc;
            if (e.scales_bytes != tg_scale_count(e.precision, e.n, e.k) * 4)
                return bad("Entry " + e.name + " has the wrong number of scales.");
            if ((rc = num("scales_offset", e.scales_offset))) return rc;
            if ((rc = check_range(e.scales_offset, e.scales_bytes))) return rc;
            e.has_scales = true;
        }
        if (!p.by_name.emplace(e.name, p.items.size()).second)
            return bad("Two entries are named " + e.name + ".");
        p.items.push_back(std::move(e));
    }
    std::sort(ranges.begin(), ranges.end());
    for (size_t i = 1; i < ranges.size(); i++)
        if (ranges[i].first < ranges[i - 1].second) return bad("Two entries overlap.");
    return TG_OK;
}

void fill(const tg_pack &p, const tg_pack::Item &e, tg_pack_entry *out) {
    memset(out, 0, sizeof(*out));
    out->name = e.name.c_str();
    out->type = e.type;
    out->precision = e.precision;
    out->n = e.n;
    out->k = e.k;
    out->rank = e.rank;
    for (size_t i = 0; i < 8; i++) out->shape[i] = e.shape[i];
    out->data = p.data + e.offset;
    out->bytes = e.bytes;
    out->scales = e.has_scales ? reinterpret_cast<const float *>(p.data + e.scales_offset) : nullptr;
    out->n_scales = e.has_scales ? e.scales_bytes / 4 : 0;
}

int finish(std::unique_ptr<tg_pack> &p, tg_pack **out) {
    const int rc = parse(*p);
    if (rc) return rc;
    *out = p.release();
    g_pack_error.clear();
    return TG_OK;
}

}  // namespace

extern "C" {

const char *tg_pack_last_error(void) { return g_pack_error.c_str(); }

int tg_pack_open(const char *path, tg_pack **out) {
    if (!path || !out) return pack_fail(TG_ERR_NULL, "null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return pack_fail(TG_ERR_ARG, std::string("Cannot open ") + path + ": " + strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return pack_fail(TG_ERR_ARG, std::string("Cannot read ") + path + ": " + strerror(errno));
    }
    const size_t len = (size_t)st.st_size;
    auto p = std::make_unique<tg_pack>();
    if (len < PREFIX + TRAILER) {
        close(fd);
        return bad("The file is too short.");
    }
    void *m = mmap(nullptr, len, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m != MAP_FAILED) {
        p->data = static_cast<const uint8_t *>(m);
        p->mapped = true;
    } else {
        // No mapping: read the file into memory (64-byte aligned once the vector's start is).
        p->copy.resize(len + ALIGN);
        uint8_t *base = p->copy.data();
        uint8_t *aligned = base + (ALIGN - reinterpret_cast<uintptr_t>(base) % ALIGN) % ALIGN;
        size_t got = 0;
        while (got < len) {
            const ssize_t r = pread(fd, aligned + got, len - got, (off_t)got);
            if (r <= 0) {
                close(fd);
                return pack_fail(TG_ERR_ARG, std::string("Cannot read ") + path);
            }
            got += (size_t)r;
        }
        p->data = aligned;
    }
    p->len = len;
    close(fd);
    return finish(p, out);
}

int tg_pack_from_bytes(const void *data, size_t len, tg_pack **out) {
    if (!out || (!data && len)) return pack_fail(TG_ERR_NULL, "null argument");
    *out = nullptr;
    auto p = std::make_unique<tg_pack>();
    p->copy.resize(len + ALIGN);
    uint8_t *base = p->copy.data();
    uint8_t *aligned = base + (ALIGN - reinterpret_cast<uintptr_t>(base) % ALIGN) % ALIGN;
    if (len) memcpy(aligned, data, len);
    p->data = aligned;
    p->len = len;
    return finish(p, out);
}

void tg_pack_close(tg_pack *pack) { delete pack; }

int tg_pack_is_mapped(const tg_pack *pack) { return pack && pack->mapped; }

const char *tg_pack_model(const tg_pack *pack) { return pack ? pack->model.c_str() : ""; }

const char *tg_pack_meta(const tg_pack *pack, const char *key) {
    if (!pack || !key) return nullptr;
    for (const auto &m : pack->metadata)
        if (m.first == key) return m.second.c_str();
    return nullptr;
}

size_t tg_pack_meta_count(const tg_pack *pack) { return pack ? pack->metadata.size() : 0; }

int tg_pack_meta_at(const tg_pack *pack, size_t i, const char **key, const char **value) {
    if (!pack || !key || !value) return TG_ERR_NULL;
    if (i >= pack->metadata.size()) return TG_ERR_ARG;
    *key = pack->metadata[i].first.c_str();
    *value = pack->metadata[i].second.c_str();
    return TG_OK;
}

size_t tg_pack_entry_count(const tg_pack *pack) { return pack ? pack->items.size() : 0; }

int tg_pack_entry_at(const tg_pack *pack, size_t i, tg_pack_entry *out) {
    if (!pack || !out) return pack_fail(TG_ERR_NULL, "null argument");
    if (i >= pack->items.size()) return pack_fail(TG_ERR_ARG, "no such entry");
    fill(*pack, pack->items[i], out);
    return TG_OK;
}

int tg_pack_find(const tg_pack *pack, const char *name, tg_pack_entry *out) {
    if (!pack || !name || !out) return pack_fail(TG_ERR_NULL, "null argument");
    const auto it = pack->by_name.find(name);
    if (it == pack->by_name.end()) return bad(std::string("Entry ") + name + " is missing.");
    fill(*pack, pack->items[it->second], out);
    return TG_OK;
}

}  // extern "C"
