// Weight readers: `.pth` ZIP + data-only pickle (src/weights/{zip,pickle}.rs), `ZJM1` / `ZJB1` /
// `ZJB2` packed files (src/weights/packed.rs). Host C++, no device code.

#include "checkpoint.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>

#include "../../include/zjai_hip.h"

namespace zjai {

namespace {

constexpr uint32_t kVersion = 1;
constexpr size_t kAlign = 64;
constexpr uint32_t kMaxEntries = 1u << 20;  // table sizes, against hostile inputs
constexpr size_t kMaxRank = 8;

[[noreturn]] void model_error(const std::string& m) { throw Error(ZJAI_E_MODEL, m); }
[[noreturn]] void limit_error(const std::string& m) { throw Error(ZJAI_E_LIMIT, m); }

size_t round_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

bool mul_ok(uint64_t a, uint64_t b, uint64_t* r) { return !__builtin_mul_overflow(a, b, r); }

// Bounds-checked little-endian cursor over a byte range.
struct Cursor {
    const uint8_t* p;
    size_t n, pos = 0;
    const char* what;
    const uint8_t* take(size_t k) {
        if (k > n - pos) model_error(std::string(what) + ": truncated");
        const uint8_t* r = p + pos;
        pos += k;
        return r;
    }
    uint64_t le(size_t k) {
        const uint8_t* b = take(k);
        uint64_t v = 0;
        for (size_t i = 0; i < k; ++i) v |= (uint64_t)b[i] << (8 * i);
        return v;
    }
    uint8_t u8() { return (uint8_t)le(1); }
    uint16_t u16() { return (uint16_t)le(2); }
    uint32_t u32() { return (uint32_t)le(4); }
    uint64_t u64() { return le(8); }
    std::string str(size_t k) {
        const uint8_t* b = take(k);
        return std::string((const char*)b, k);
    }
};

uint64_t le_at(const uint8_t* d, size_t n, size_t pos, size_t k, const char* what) {
    if (pos > n || k > n - pos) model_error(what);
    uint64_t v = 0;
    for (size_t i = 0; i < k; ++i) v |= (uint64_t)d[pos + i] << (8 * i);
    return v;
}

bool valid_utf8(const std::string& s) {
    size_t i = 0;
    while (i < s.size()) {
        const uint8_t c = (uint8_t)s[i];
        int extra;
        uint32_t cp;
        if (c < 0x80) {
            ++i;
            continue;
        } else if ((c & 0xe0) == 0xc0) {
            extra = 1;
            cp = c & 0x1f;
        } else if ((c & 0xf0) == 0xe0) {
            extra = 2;
            cp = c & 0x0f;
        } else if ((c & 0xf8) == 0xf0) {
            extra = 3;
            cp = c & 0x07;
        } else {
            return false;
        }
        if (i + extra >= s.size()) return false;
        for (int k = 1; k <= extra; ++k) {
            const uint8_t cc = (uint8_t)s[i + k];
            if ((cc & 0xc0) != 0x80) return false;
            cp = (cp << 6) | (cc & 0x3f);
        }
        static const uint32_t min_cp[4] = {0, 0x80, 0x800, 0x10000};
        if (cp < min_cp[extra] || cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff)) return false;
        i += extra + 1;
    }
    return true;
}

void put_le(std::vector<uint8_t>& out, uint64_t v, size_t k) {
    for (size_t i = 0; i < k; ++i) out.push_back((uint8_t)(v >> (8 * i)));
}

void put_name(std::vector<uint8_t>& out, const std::string& s, const char* what) {
    if (s.size() > 0xffff) model_error(std::string(what) + ": name too long");
    put_le(out, s.size(), 2);
    out.insert(out.end(), s.begin(), s.end());
}

void pad_to_align(std::vector<uint8_t>& out) { out.resize(round_up(out.size()), 0); }

// Cursor past a packed header: magic, then the u32 version.
Cursor packed_header(const uint8_t* d, size_t n, const char* magic) {
    Cursor c{d, n, 0, "packed model"};
    if (n < 4 || std::memcmp(c.take(4), magic, 4) != 0) model_error("packed model: bad magic");
    if (c.u32() != kVersion) model_error("packed model: unsupported version");
    return c;
}

// ------------------------------------------------------------------------------------ ZIP
// The uncompressed archives torch.save writes (src/weights/zip.rs): central directory (ZIP64
// aware), stored members only; payload ranges are located through each local header, whose
// extra field torch pads so payloads are 64-byte aligned.
constexpr uint32_t kEocd = 0x06054b50, kEocd64Locator = 0x07064b50, kEocd64 = 0x06064b50,
                   kCentral = 0x02014b50, kLocal = 0x04034b50;

std::vector<std::pair<std::string, std::pair<size_t, size_t>>> zip_members(const uint8_t* d, size_t n) {
    auto u16 = [&](size_t p) { return le_at(d, n, p, 2, "zip: truncated"); };
    auto u32 = [&](size_t p) { return le_at(d, n, p, 4, "zip: truncated"); };
    auto u64 = [&](size_t p) { return le_at(d, n, p, 8, "zip: truncated"); };
    if (n < 22) model_error("zip: file too small");
    // End-of-central-directory record: search back over the (<= 64 KiB) archive comment.
    size_t eocd = SIZE_MAX;
    const size_t lo = n >= 22 + 65535 ? n - 22 - 65535 : 0;
    for (size_t p = n - 22 + 1; p-- > lo;)
        if (u32(p) == kEocd) {
            eocd = p;
            break;
        }
    if (eocd == SIZE_MAX) model_error("zip: end of central directory not found");
    uint64_t count = u16(eocd + 10), cd_size = u32(eocd + 12), cd_off = u32(eocd + 16);
    if (eocd >= 20 && u32(eocd - 20) == kEocd64Locator) {
        const uint64_t rec = u64(eocd - 20 + 8);
        if (rec > n || u32((size_t)rec) != kEocd64) model_error("zip: bad zip64 record");
        count = u64((size_t)rec + 32);
        cd_size = u64((size_t)rec + 40);
        cd_off = u64((size_t)rec + 48);
    }
    if (count > 1000000) model_error("zip: implausible entry count");
    if (cd_off > n || cd_size > n - cd_off) model_error("zip: central directory out of bounds");
    const size_t cd_end = (size_t)(cd_off + cd_size);
    std::vector<std::pair<std::string, std::pair<size_t, size_t>>> out;
    size_t p = (size_t)cd_off;
    for (uint64_t i = 0; i < count; ++i) {
        if (p + 46 > cd_end || u32(p) != kCentral) model_error("zip: bad central directory entry");
        const uint64_t method = u16(p + 10);
        uint64_t csize = u32(p + 20), usize = u32(p + 24), local = u32(p + 42);
        const size_t name_len = u16(p + 28), extra_len = u16(p + 30), comment_len = u16(p + 32);
        if (p + 46 + name_len + extra_len > n) model_error("zip: truncated entry");
        std::string name((const char*)d + p + 46, name_len);
        if (!valid_utf8(name)) model_error("zip: entry name is not UTF-8");
        // ZIP64 extended information (id 1): 64-bit values for the saturated fields only, in the
        // order uncompressed size, compressed size, local header offset.
        size_t e = p + 46 + name_len;
        const size_t e_end = e + extra_len;
        while (e + 4 <= e_end) {
            const uint64_t id = u16(e), len = u16(e + 2);
            if (e + 4 + len > e_end) model_error("zip: truncated extra field");
            if (id == 1) {
                size_t q = e + 4;
                for (uint64_t* f : {&usize, &csize, &local})
                    if (*f == 0xffffffffull) {
                        if (q + 8 > e + 4 + len) model_error("zip: truncated zip64 field");
                        *f = u64(q);
                        q += 8;
                    }
            }
            e += 4 + len;
        }
        if (method != 0 || csize != usize)
            model_error("zip: entry `" + name + "` is compressed; torch checkpoints are stored");
        if (local > n || u32((size_t)local) != kLocal) model_error("zip: bad local header");
        const size_t start = (size_t)local + 30 + u16((size_t)local + 26) + u16((size_t)local + 28);
        if (start > n || usize > n - start) model_error("zip: entry data out of bounds");
        out.push_back({name, {start, (size_t)usize}});
        p += 46 + name_len + extra_len + comment_len;
    }
    return out;
}

// --------------------------------------------------------------------------------- pickle
// A data-only interpreter for the opcodes torch.save emits (protocol 2, plus the framing and
// memo opcodes of protocols 4 / 5): GLOBAL only records a name, and REDUCE builds a value from
// three known constructors (OrderedDict, _rebuild_tensor_v2, _rebuild_parameter); anything else
// becomes an opaque object. Containers are shared between the stack and the memo, as in Python.
// Values live in one arena per parse and refer to each other by plain pointers, so a pickle
// that nests or cycles its containers neither leaks nor recurses when released.
struct PVal;
using PV = PVal*;
struct PVal {
    enum Kind { NONE, BOOL, INT, FLOAT, STR, BYTES, TUPLE, LIST, DICT, GLOBAL, STORAGE, TENSOR, OBJECT, MARK } k;
    int64_t i = 0;
    double f = 0;
    std::string s, s2;          // STR / BYTES / storage key; GLOBAL module and name
    std::vector<PV> items;      // TUPLE / LIST; OBJECT (callable, args)
    std::vector<std::pair<PV, PV>> dict;
    CkTensor t;                 // TENSOR; STORAGE uses t.dtype
    explicit PVal(Kind kind) : k(kind) {}
};
struct Arena {
    std::vector<std::unique_ptr<PVal>> vals;
};
thread_local Arena* t_arena = nullptr;
PV mk(PVal::Kind k) {
    t_arena->vals.emplace_back(new PVal(k));
    return t_arena->vals.back().get();
}
PV mk_int(int64_t v) {
    PV p = mk(PVal::INT);
    p->i = v;
    return p;
}
PV mk_str(PVal::Kind k, std::string s) {
    PV p = mk(k);
    p->s = std::move(s);
    return p;
}

constexpr size_t kMaxStack = 1u << 20, kMaxMemo = 1u << 22;

[[noreturn]] void bad_pickle(const std::string& m) { model_error("pickle: " + m); }

int storage_dtype(const std::string& cls) {
    static const std::map<std::string, int> m = {
        {"DoubleStorage", CK_F64}, {"FloatStorage", CK_F32}, {"HalfStorage", CK_F16},
        {"LongStorage", CK_I64},   {"IntStorage", CK_I32},   {"ShortStorage", CK_I16},
        {"CharStorage", CK_I8},    {"ByteStorage", CK_U8},   {"BoolStorage", CK_BOOL}};
    auto it = m.find(cls);
    if (it == m.end()) model_error("pickle: unsupported storage class `" + cls + "`");
    return it->second;
}

uint64_t as_index(const PV& v) {
    if (v->k != PVal::INT || v->i < 0) bad_pickle("expected a non-negative integer");
    return (uint64_t)v->i;
}

std::vector<uint64_t> as_index_list(const PV& v) {
    if (v->k != PVal::TUPLE && v->k != PVal::LIST) bad_pickle("expected a tuple of integers");
    std::vector<uint64_t> r;
    for (const PV& x : v->items) r.push_back(as_index(x));
    return r;
}

// REDUCE / NEWOBJ over the allow-list (src/weights/pickle.rs:150-177).
PV reduce(const PV& callable, const PV& args) {
    if (callable->k == PVal::GLOBAL && args->k == PVal::TUPLE) {
        const std::string& mod = callable->s;
        const std::string& nm = callable->s2;
        const auto& a = args->items;
        if (mod == "collections" && nm == "OrderedDict" && a.empty()) return mk(PVal::DICT);
        if (mod == "torch._utils" && nm == "_rebuild_tensor_v2" && a.size() >= 4) {
            if (a[0]->k != PVal::STORAGE) bad_pickle("tensor without a storage");
            PV t = mk(PVal::TENSOR);
            t->t.storage = a[0]->s;
            t->t.dtype = a[0]->t.dtype;
            t->t.offset = as_index(a[1]);
            t->t.shape = as_index_list(a[2]);
            t->t.stride = as_index_list(a[3]);
            return t;
        }
        if (mod == "torch._utils" && nm == "_rebuild_parameter" && !a.empty()) return a[0];
    }
    PV o = mk(PVal::OBJECT);
    o->items = {callable, args};
    return o;
}

// BINPERSID: ('storage', <StorageClass>, key, location, numel) (src/weights/pickle.rs:179-203).
PV persistent_load(const PV& pid) {
    if (pid->k != PVal::TUPLE) bad_pickle("persistent id is not a tuple");
    const auto& a = pid->items;
    if (a.size() < 3 || a[0]->k != PVal::STR || a[0]->s != "storage" || a[1]->k != PVal::GLOBAL ||
        a[2]->k != PVal::STR)
        bad_pickle("unrecognised persistent id");
    PV s = mk(PVal::STORAGE);
    s->s = a[2]->s;
    s->t.dtype = storage_dtype(a[1]->s2);
    return s;
}

int64_t long_le(const uint8_t* b, size_t n) {
    if (n > 8) bad_pickle("integer wider than 64 bits");
    if (n == 0) return 0;
    uint64_t v = (b[n - 1] & 0x80) ? ~0ull : 0ull;
    for (size_t i = 0; i < n; ++i) {
        v &= ~(0xffull << (8 * i));
        v |= (uint64_t)b[i] << (8 * i);
    }
    return (int64_t)v;
}

PV unpickle(const uint8_t* data, size_t len, Arena& arena) {
    struct Use {
        Arena* prev;
        explicit Use(Arena& a) : prev(t_arena) { t_arena = &a; }
        ~Use() { t_arena = prev; }
    } use(arena);
    Cursor r{data, len, 0, "pickle"};
    std::vector<PV> stack;
    std::vector<PV> memo;
    auto pop = [&]() {
        if (stack.empty()) bad_pickle("stack underflow");
        PV v = stack.back();
        stack.pop_back();
        return v;
    };
    auto pop_mark = [&]() {
        size_t m = stack.size();
        while (m > 0 && stack[m - 1]->k != PVal::MARK) --m;
        if (m == 0) bad_pickle("missing MARK");
        std::vector<PV> items(stack.begin() + m, stack.end());
        stack.resize(m - 1);
        return items;
    };
    auto top = [&]() -> PV& {
        if (stack.empty()) bad_pickle("empty stack");
        return stack.back();
    };
    auto memo_put = [&](size_t idx) {
        if (idx >= kMaxMemo) bad_pickle("memo index too large");
        if (idx >= memo.size()) memo.resize(idx + 1);
        memo[idx] = top();
    };
    auto memo_get = [&](size_t idx) {
        if (idx >= memo.size() || !memo[idx]) bad_pickle("memo miss");
        stack.push_back(memo[idx]);
    };
    auto line = [&]() {
        const size_t start = r.pos;
        while (r.pos < r.n && r.p[r.pos] != '\n') ++r.pos;
        if (r.pos >= r.n) bad_pickle("unterminated line");
        std::string s((const char*)r.p + start, r.pos - start);
        ++r.pos;
        return s;
    };
    auto text = [&](size_t n) {
        std::string s = r.str(n);
        if (!valid_utf8(s)) bad_pickle("string is not UTF-8");
        return s;
    };
    auto size_of = [&](uint64_t n) {
        if (n > r.n - r.pos) bad_pickle("length beyond the data");
        return (size_t)n;
    };
    auto set_items = [&](PV& target, std::vector<PV>& kv, const char* op) {
        if (target->k == PVal::DICT) {
            for (size_t i = 0; i + 1 < kv.size(); i += 2) target->dict.push_back({kv[i], kv[i + 1]});
        } else if (target->k != PVal::OBJECT) {
            bad_pickle(std::string(op) + " target is not a dict");
        }
    };
    for (;;) {
        if (stack.size() > kMaxStack) bad_pickle("stack too deep");
        const uint8_t op = r.u8();
        switch (op) {
            case 0x80:  // PROTO
                if (r.u8() > 5) bad_pickle("unsupported protocol");
                break;
            case 0x95: r.u64(); break;  // FRAME: a length hint
            case '.': return pop();     // STOP
            case '(': stack.push_back(mk(PVal::MARK)); break;
            case 'N': stack.push_back(mk(PVal::NONE)); break;
            case 0x88:
            case 0x89: {
                PV b = mk(PVal::BOOL);
                b->i = op == 0x88;
                stack.push_back(b);
                break;
            }
            case 'J': stack.push_back(mk_int((int32_t)r.u32())); break;
            case 'K': stack.push_back(mk_int(r.u8())); break;
            case 'M': stack.push_back(mk_int(r.u16())); break;
            case 0x8a: {  // LONG1
                const size_t n = r.u8();
                stack.push_back(mk_int(long_le(r.take(n), n)));
                break;
            }
            case 0x8b: {  // LONG4
                const size_t n = size_of(r.u32());
                stack.push_back(mk_int(long_le(r.take(n), n)));
                break;
            }
            case 'G': {  // BINFLOAT, big-endian
                const uint8_t* b = r.take(8);
                uint64_t bits = 0;
                for (int i = 0; i < 8; ++i) bits = (bits << 8) | b[i];
                PV f = mk(PVal::FLOAT);
                std::memcpy(&f->f, &bits, 8);
                stack.push_back(f);
                break;
            }
            case 'X': stack.push_back(mk_str(PVal::STR, text(size_of(r.u32())))); break;
            case 0x8c: stack.push_back(mk_str(PVal::STR, text(r.u8()))); break;
            case 0x8d: stack.push_back(mk_str(PVal::STR, text(size_of(r.u64())))); break;
            case 'U':
            case 'C': stack.push_back(mk_str(PVal::BYTES, r.str(r.u8()))); break;
            case 'T':
            case 'B': stack.push_back(mk_str(PVal::BYTES, r.str(size_of(r.u32())))); break;
            case 0x8e:
            case 0x96: stack.push_back(mk_str(PVal::BYTES, r.str(size_of(r.u64())))); break;
            case 'c': {  // GLOBAL "module\nname\n"
                PV g = mk(PVal::GLOBAL);
                g->s = line();
                g->s2 = line();
                stack.push_back(g);
                break;
            }
            case 0x93: {  // STACK_GLOBAL
                PV name = pop(), mod = pop();
                if (mod->k != PVal::STR || name->k != PVal::STR) bad_pickle("STACK_GLOBAL operands are not strings");
                PV g = mk(PVal::GLOBAL);
                g->s = mod->s;
                g->s2 = name->s;
                stack.push_back(g);
                break;
            }
            case ')': stack.push_back(mk(PVal::TUPLE)); break;
            case 't': {
                PV t = mk(PVal::TUPLE);
                t->items = pop_mark();
                stack.push_back(t);
                break;
            }
            case 0x85:
            case 0x86:
            case 0x87: {  // TUPLE1..3
                const size_t n = op - 0x84;
                if (stack.size() < n) bad_pickle("stack underflow");
                PV t = mk(PVal::TUPLE);
                t->items.assign(stack.end() - n, stack.end());
                stack.resize(stack.size() - n);
                stack.push_back(t);
                break;
            }
            case ']': stack.push_back(mk(PVal::LIST)); break;
            case 0x8f: stack.push_back(mk(PVal::LIST)); break;  // EMPTY_SET, kept as a list
            case 'l': {
                PV l = mk(PVal::LIST);
                l->items = pop_mark();
                stack.push_back(l);
                break;
            }
            case 0x91: {  // FROZENSET
                PV l = mk(PVal::LIST);
                l->items = pop_mark();
                stack.push_back(l);
                break;
            }
            case 'a': {
                PV v = pop();
                if (top()->k != PVal::LIST) bad_pickle("APPEND target is not a list");
                top()->items.push_back(v);
                break;
            }
            case 'e':
            case 0x90: {  // APPENDS, ADDITEMS
                std::vector<PV> items = pop_mark();
                if (top()->k != PVal::LIST) bad_pickle("APPENDS target is not a list");
                top()->items.insert(top()->items.end(), items.begin(), items.end());
                break;
            }
            case '}': stack.push_back(mk(PVal::DICT)); break;
            case 'd': {
                std::vector<PV> kv = pop_mark();
                PV d = mk(PVal::DICT);
                set_items(d, kv, "DICT");
                stack.push_back(d);
                break;
            }
            case 's': {
                PV v = pop(), k = pop();
                std::vector<PV> kv = {k, v};
                set_items(top(), kv, "SETITEM");
                break;
            }
            case 'u': {
                std::vector<PV> kv = pop_mark();
                set_items(top(), kv, "SETITEMS");
                break;
            }
            case 'R':
            case 0x81: {  // REDUCE, NEWOBJ
                PV args = pop(), callable = pop();
                stack.push_back(reduce(callable, args));
                break;
            }
            case 0x92: {  // NEWOBJ_EX (cls, args, kwargs)
                pop();
                PV args = pop(), cls = pop();
                stack.push_back(reduce(cls, args));
                break;
            }
            case 'b':  // BUILD: object state (OrderedDict._metadata); carries no tensor data
                pop();
                if (stack.empty()) bad_pickle("BUILD without an object");
                break;
            case 'Q': {
                PV pid = pop();
                stack.push_back(persistent_load(pid));
                break;
            }
            case 'q': memo_put(r.u8()); break;
            case 'r': memo_put(r.u32()); break;
            case 0x94: memo_put(memo.size()); break;  // MEMOIZE
            case 'h': memo_get(r.u8()); break;
            case 'j': memo_get(r.u32()); break;
            case '0': pop(); break;
            case '1': pop_mark(); break;
            case '2': stack.push_back(top()); break;
            default: {
                char buf[64];
                std::snprintf(buf, sizeof buf, "unsupported opcode 0x%02x at byte %zu", op, r.pos - 1);
                bad_pickle(buf);
            }
        }
    }
}

// Nested dicts of a state dict, flattened to dotted names up to three levels: tensor leaves
// and lists of numbers (src/weights/mod.rs:78-126).
void flatten(const std::string& prefix, const PV& d, int depth, std::vector<CkTensor>& tensors,
             std::vector<std::pair<std::string, std::vector<double>>>& lists) {
    if (depth >= 3) return;
    for (const auto& kv : d->dict) {
        if (kv.first->k != PVal::STR) continue;
        const std::string name = prefix + "." + kv.first->s;
        const PV& v = kv.second;
        if (v->k == PVal::TENSOR) {
            CkTensor t = v->t;
            t.name = name;
            tensors.push_back(t);
        } else if (v->k == PVal::DICT) {
            flatten(name, v, depth + 1, tensors, lists);
        } else if (v->k == PVal::LIST) {
            std::vector<double> xs;
            bool numeric = true;
            for (const PV& x : v->items) {
                if (x->k == PVal::FLOAT) xs.push_back(x->f);
                else if (x->k == PVal::INT) xs.push_back((double)x->i);
                else {
                    numeric = false;
                    break;
                }
            }
            if (numeric) lists.push_back({name, xs});
        }
    }
}

}  // namespace

size_t ck_dtype_size(int dtype) {
    switch (dtype) {
        case CK_F64:
        case CK_I64: return 8;
        case CK_F32:
        case CK_I32: return 4;
        case CK_F16:
        case CK_I16: return 2;
        default: return 1;
    }
}

uint16_t f32_to_f16_bits(float v) {
    uint32_t b;
    std::memcpy(&b, &v, 4);
    const uint16_t sign = (uint16_t)((b >> 16) & 0x8000);
    const int exp = (int)((b >> 23) & 0xff);
    const uint32_t mant = b & 0x007fffff;
    if (exp == 255) {
        const uint16_t payload = (uint16_t)((mant >> 13) | 0x200);
        return (uint16_t)(sign | 0x7c00 | (mant ? payload : 0));
    }
    const int e = exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) {
        if (e < -10) return sign;
        const uint32_t m = mant | 0x00800000;
        const uint32_t shift = (uint32_t)(14 - e);
        const uint32_t dropped = m & ((1u << shift) - 1);
        const uint32_t half = 1u << (shift - 1);
        uint32_t r = m >> shift;
        if (dropped > half || (dropped == half && (r & 1))) r += 1;
        return (uint16_t)(sign | r);
    }
    const uint32_t dropped = mant & 0x1fff;
    uint32_t r = mant >> 13;
    if (dropped > 0x1000 || (dropped == 0x1000 && (r & 1))) r += 1;
    return (uint16_t)(sign | (((uint32_t)e << 10) + r));
}

float f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t bits;
    if (e == 0) {
        const float sub = (float)m * 5.9604644775390625e-8f;  // m * 2^-24, exact
        std::memcpy(&bits, &sub, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint64_t CkTensor::numel() const {
    uint64_t n = 1;
    for (uint64_t d : shape)
        if (!mul_ok(n, d, &n)) model_error("tensor `" + name + "`: size overflow");
    return n;
}

std::unique_ptr<Checkpoint> Checkpoint::parse(const uint8_t* data, size_t len) {
    if (!data && len) throw Error(ZJAI_E_INVALID_ARGUMENT, "checkpoint: null data");
    std::unique_ptr<Checkpoint> ck(new Checkpoint());
    ck->file_.assign(data, data + len);
    if (len >= 4 && std::memcmp(data, "ZJM1", 4) == 0) ck->parse_zjm();
    else ck->parse_pth();
    return ck;
}

// `parse_zjm` (src/weights/packed.rs:150-205).
void Checkpoint::parse_zjm() {
    packed_ = true;
    const uint8_t* d = file_.data();
    const size_t n = file_.size();
    Cursor c = packed_header(d, n, "ZJM1");
    const uint32_t nt = c.u32(), ni = c.u32();
    if (nt > kMaxEntries || ni > kMaxEntries) limit_error("packed model: too many entries");
    for (uint32_t i = 0; i < nt; ++i) {
        CkTensor t;
        t.name = c.str(c.u16());
        if (!valid_utf8(t.name)) model_error("packed model: name is not UTF-8");
        t.dtype = c.u8();
        if (t.dtype >= CK_NDTYPES) model_error("packed model: unknown dtype code");
        const size_t rank = c.u8();
        if (rank > kMaxRank) model_error("packed model: tensor rank above 8");
        for (size_t k = 0; k < rank; ++k) t.shape.push_back(c.u64());
        const uint64_t off = c.u64(), len = c.u64();
        const size_t es = ck_dtype_size(t.dtype);
        uint64_t bytes = 1;
        bool ok = true;
        for (uint64_t dim : t.shape) ok = ok && mul_ok(bytes, dim, &bytes);
        ok = ok && mul_ok(bytes, es, &bytes);
        if (!ok || bytes != len || off % kAlign != 0 || off > n || len > n - off)
            model_error("packed model: tensor `" + t.name + "` has an invalid extent");
        t.offset = off / es;
        t.stride.assign(rank, 1);
        for (size_t k = rank; k-- > 1;) t.stride[k - 1] = t.stride[k] * t.shape[k];
        tensors_.push_back(std::move(t));
    }
    for (uint32_t i = 0; i < ni; ++i) {
        std::string name = c.str(c.u16());
        if (!valid_utf8(name)) model_error("packed model: name is not UTF-8");
        ints_.push_back({name, (int64_t)c.u64()});
    }
}

void Checkpoint::parse_pth() {
    members_ = zip_members(file_.data(), file_.size());
    const std::pair<std::string, std::pair<size_t, size_t>>* pkl = nullptr;
    for (const auto& m : members_) {
        const std::string& nm = m.first;
        if (nm == "data.pkl" || (nm.size() > 9 && nm.compare(nm.size() - 9, 9, "/data.pkl") == 0)) {
            pkl = &m;
            break;
        }
    }
    if (!pkl) model_error("checkpoint has no data.pkl");
    prefix_ = pkl->first.substr(0, pkl->first.size() - 8);
    Arena arena;
    const PV root = unpickle(file_.data() + pkl->second.first, pkl->second.second, arena);
    std::sort(members_.begin(), members_.end());
    if (root->k != PVal::DICT) model_error("checkpoint root is not a state dict");
    for (const auto& kv : root->dict) {
        if (kv.first->k != PVal::STR) continue;
        const PV& v = kv.second;
        if (v->k == PVal::TENSOR) {
            CkTensor t = v->t;
            t.name = kv.first->s;
            tensors_.push_back(t);
        } else if (v->k == PVal::INT) {
            ints_.push_back({kv.first->s, v->i});
        } else if (v->k == PVal::DICT) {
            flatten(kv.first->s, v, 0, tensors_, lists_);
        }
    }
}

const CkTensor* Checkpoint::find(const std::string& name) const {
    for (const CkTensor& t : tensors_)
        if (t.name == name) return &t;
    return nullptr;
}

std::pair<const uint8_t*, size_t> Checkpoint::storage(const CkTensor& t) const {
    if (packed_) return {file_.data(), file_.size()};
    const std::string key = prefix_ + "data/" + t.storage;
    auto it = std::lower_bound(members_.begin(), members_.end(), key,
                               [](const auto& m, const std::string& k) { return m.first < k; });
    if (it == members_.end() || it->first != key)
        model_error("tensor `" + t.name + "`: storage `" + t.storage + "` missing");
    return {file_.data() + it->second.first, it->second.second};
}

std::vector<uint8_t> Checkpoint::bytes(const CkTensor& t) const {
    if (t.shape.size() != t.stride.size()) model_error("tensor `" + t.name + "`: shape/stride rank mismatch");
    const auto st = storage(t);
    const size_t es = ck_dtype_size(t.dtype);
    const uint64_t numel = t.numel();
    uint64_t total;
    if (!mul_ok(numel, es, &total)) model_error("tensor `" + t.name + "`: size overflow");
    const uint64_t storage_elems = st.second / es;
    bool contiguous = true;
    uint64_t expect = 1;
    for (size_t k = t.shape.size(); k-- > 0;) {
        if (t.shape[k] != 1 && t.stride[k] != expect) contiguous = false;
        expect *= t.shape[k];
    }
    std::vector<uint8_t> out;
    if (numel == 0) return out;
    if (contiguous) {
        uint64_t start;
        if (!mul_ok(t.offset, es, &start) || start > st.second || total > st.second - start)
            model_error("tensor `" + t.name + "` exceeds its storage");
        out.assign(st.first + start, st.first + start + total);
        return out;
    }
    // Strided view: the farthest element must lie inside the storage, then gather row-major.
    uint64_t last = t.offset;
    for (size_t k = 0; k < t.shape.size(); ++k) {
        uint64_t span;
        if (!mul_ok(t.shape[k] - 1, t.stride[k], &span) || __builtin_add_overflow(last, span, &last))
            model_error("tensor `" + t.name + "`: stride overflow");
    }
    if (last >= storage_elems) model_error("tensor `" + t.name + "` exceeds its storage");
    out.resize(total);
    std::vector<uint64_t> idx(t.shape.size(), 0);
    for (uint64_t i = 0; i < numel; ++i) {
        uint64_t e = t.offset;
        for (size_t k = 0; k < idx.size(); ++k) e += idx[k] * t.stride[k];
        std::memcpy(out.data() + i * es, st.first + e * es, es);
        for (size_t k = idx.size(); k-- > 0;) {
            if (++idx[k] < t.shape[k]) break;
            idx[k] = 0;
        }
    }
    return out;
}

std::vector<float> Checkpoint::f32(const CkTensor& t) const {
    if (t.dtype != CK_F32 && t.dtype != CK_F16)
        model_error("tensor `" + t.name + "` is not f32 (or f16)");
    const std::vector<uint8_t> b = bytes(t);
    std::vector<float> out(b.size() / ck_dtype_size(t.dtype));
    if (t.dtype == CK_F32) {
        if (!b.empty()) std::memcpy(out.data(), b.data(), b.size());
    } else {
        for (size_t i = 0; i < out.size(); ++i) out[i] = f16_bits_to_f32((uint16_t)(b[2 * i] | (b[2 * i + 1] << 8)));
    }
    return out;
}

std::vector<uint8_t> write_zjm(const Checkpoint& ck, const std::vector<std::string>& names, bool f16) {
    struct Payload {
        int dtype;
        const std::vector<uint64_t>* shape;
        std::vector<uint8_t> bytes;
    };
    std::vector<Payload> pl;
    for (const std::string& nm : names) {
        const CkTensor* t = ck.find(nm);
        if (!t) model_error("tensor `" + nm + "` not found");
        if (t->shape.size() > kMaxRank) model_error("packed model: tensor rank above 8");
        Payload p{t->dtype, &t->shape, ck.bytes(*t)};
        if (f16 && t->dtype == CK_F32 && nm != "vr_vec.c") {
            std::vector<uint8_t> half(p.bytes.size() / 2);
            for (size_t i = 0; i < half.size() / 2; ++i) {
                float v;
                std::memcpy(&v, p.bytes.data() + 4 * i, 4);
                const uint16_t h = f32_to_f16_bits(v);
                half[2 * i] = (uint8_t)h;
                half[2 * i + 1] = (uint8_t)(h >> 8);
            }
            p.dtype = CK_F16;
            p.bytes = std::move(half);
        }
        pl.push_back(std::move(p));
    }
    size_t table = 16;
    for (size_t i = 0; i < names.size(); ++i) table += 2 + names[i].size() + 2 + 8 * pl[i].shape->size() + 16;
    for (const auto& iv : ck.ints()) table += 2 + iv.first.size() + 8;
    std::vector<uint8_t> out;
    out.insert(out.end(), {'Z', 'J', 'M', '1'});
    put_le(out, kVersion, 4);
    put_le(out, names.size(), 4);
    put_le(out, ck.ints().size(), 4);
    size_t offset = round_up(table);
    for (size_t i = 0; i < names.size(); ++i) {
        put_name(out, names[i], "packed model");
        out.push_back((uint8_t)pl[i].dtype);
        out.push_back((uint8_t)pl[i].shape->size());
        for (uint64_t dim : *pl[i].shape) put_le(out, dim, 8);
        put_le(out, offset, 8);
        put_le(out, pl[i].bytes.size(), 8);
        offset = round_up(offset + pl[i].bytes.size());
    }
    for (const auto& iv : ck.ints()) {
        put_name(out, iv.first, "packed model");
        put_le(out, (uint64_t)iv.second, 8);
    }
    pad_to_align(out);
    for (const Payload& p : pl) {
        out.insert(out.end(), p.bytes.begin(), p.bytes.end());
        pad_to_align(out);
    }
    return out;
}

// `PackedBundle::add` (src/weights/packed.rs:307-345).
void Bundle::add(const uint8_t* data, size_t len) {
    if (!data && len) throw Error(ZJAI_E_INVALID_ARGUMENT, "bundle: null data");
    const char* magic = nullptr;
    if (len >= 4 && std::memcmp(data, "ZJB1", 4) == 0) magic = "ZJB1";
    else if (len >= 4 && std::memcmp(data, "ZJB2", 4) == 0) magic = "ZJB2";
    else model_error("packed model: bad magic");
    Part part;
    part.data.assign(data, data + len);
    const uint8_t* d = part.data.data();
    Cursor c = packed_header(d, len, magic);
    const uint32_t count = c.u32();
    if (count > kMaxEntries) limit_error("bundle: too many files");
    part.notice_len = c.u32();
    part.notice_at = c.pos;
    if (!valid_utf8(c.str(part.notice_len))) model_error("bundle: notice is not UTF-8");
    for (uint32_t i = 0; i < count; ++i) {
        std::string rel = c.str(c.u16());
        if (!valid_utf8(rel)) model_error("packed model: name is not UTF-8");
        const uint64_t off = c.u64(), n = c.u64();
        if (off > len || n > len - off || off % kAlign != 0)
            model_error("bundle: `" + rel + "` has an invalid extent");
        part.files.push_back({rel, {(size_t)off, (size_t)n}});
    }
    std::sort(part.files.begin(), part.files.end());
    parts_.push_back(std::move(part));
}

std::vector<std::string> Bundle::paths() const {
    std::vector<std::string> out;
    for (const Part& p : parts_)
        for (const auto& f : p.files) out.push_back(f.first);
    return out;
}

std::pair<const uint8_t*, size_t> Bundle::get(const std::string& rel) const {
    for (const Part& p : parts_) {
        auto it = std::lower_bound(p.files.begin(), p.files.end(), rel,
                                   [](const auto& f, const std::string& k) { return f.first < k; });
        if (it != p.files.end() && it->first == rel) return {p.data.data() + it->second.first, it->second.second};
    }
    return {nullptr, 0};
}

std::string Bundle::notice() const {
    if (parts_.empty()) return "";
    const Part& p = parts_.front();
    return std::string((const char*)p.data.data() + p.notice_at, p.notice_len);
}

std::vector<uint8_t> write_bundle(const std::vector<std::pair<std::string, std::vector<uint8_t>>>& files,
                                  const std::string& notice, bool f16) {
    if (notice.size() > 0xffffffffull) model_error("bundle: notice too long");
    size_t table = 16 + notice.size();
    for (const auto& f : files) table += 2 + f.first.size() + 16;
    std::vector<uint8_t> out;
    const char* magic = f16 ? "ZJB2" : "ZJB1";
    out.insert(out.end(), magic, magic + 4);
    put_le(out, kVersion, 4);
    put_le(out, files.size(), 4);
    put_le(out, notice.size(), 4);
    out.insert(out.end(), notice.begin(), notice.end());
    size_t offset = round_up(table);
    for (const auto& f : files) {
        put_name(out, f.first, "bundle");
        put_le(out, offset, 8);
        put_le(out, f.second.size(), 8);
        offset = round_up(offset + f.second.size());
    }
    pad_to_align(out);
    for (const auto& f : files) {
        out.insert(out.end(), f.second.begin(), f.second.end());
        pad_to_align(out);
    }
    return out;
}

}  // namespace zjai
