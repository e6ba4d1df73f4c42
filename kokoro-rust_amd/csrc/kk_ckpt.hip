// kk_ckpt.hip -- host reader of PyTorch zip checkpoints (the model file and the voice packs) and
// the weight_norm resolution of hydration.  Host code only.
//
// Replaces the reference's native reader (src/torchpt.rs) and the host-side weight_norm
// (src/ops.rs:9-23).  The archive is read, never executed: a zip directory walk (STORED entries,
// the way torch.save writes them) and a small pickle machine that accepts exactly what torch.save
// emits for float32 tensors inside (ordered) dicts and refuses everything else.
#include "kk_ckpt.h"

#include <cmath>
#include <cstring>
#include <fstream>
#include <memory>
#include <stdexcept>

namespace kk {
namespace {

[[noreturn]] void bad(const std::string& m) { throw std::runtime_error(m); }

std::vector<uint8_t> read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    if (!f) bad("cannot open " + path);
    const std::streamsize n = f.tellg();
    if (n < 0) bad("cannot size " + path);
    std::vector<uint8_t> b((size_t)n);
    f.seekg(0);
    if (n > 0 && !f.read((char*)b.data(), n)) bad("cannot read " + path);
    return b;
}

// ------------------------------------------------------------------ zip directory
struct Archive {
    const std::vector<uint8_t>& bytes;
    std::map<std::string, std::pair<size_t, size_t>> entries;  // name -> (data offset, size)

    uint32_t u16(size_t o) const {
        if (o + 2 > bytes.size()) bad("zip: truncated");
        return (uint32_t)bytes[o] | ((uint32_t)bytes[o + 1] << 8);
    }
    uint32_t u32(size_t o) const {
        if (o + 4 > bytes.size()) bad("zip: truncated");
        return (uint32_t)bytes[o] | ((uint32_t)bytes[o + 1] << 8) | ((uint32_t)bytes[o + 2] << 16) |
               ((uint32_t)bytes[o + 3] << 24);
    }

    explicit Archive(const std::vector<uint8_t>& b) : bytes(b) {
        if (b.size() < 22) bad("not a zip archive");
        // the end-of-central-directory record: its signature within the last 22 + 65535 bytes
        size_t eocd = SIZE_MAX;
        const size_t lo = b.size() >= 22 + 65535 ? b.size() - 22 - 65535 : 0;
        for (size_t i = b.size() - 22 + 1; i-- > lo;)
            if (u32(i) == 0x06054b50u) {
                eocd = i;
                break;
            }
        if (eocd == SIZE_MAX) bad("zip: no end-of-central-directory record");
        const uint32_t n = u16(eocd + 10), cd = u32(eocd + 16);
        if (n == 0xffffu || cd == 0xffffffffu) bad("zip64 archives are not supported");
        size_t p = cd;
        for (uint32_t e = 0; e < n; e++) {
            if (u32(p) != 0x02014b50u) bad("zip: bad central directory entry");
            const uint32_t method = u16(p + 10), csize = u32(p + 20), usize = u32(p + 24);
            const uint32_t nlen = u16(p + 28), xlen = u16(p + 30), clen = u16(p + 32), lho = u32(p + 42);
            if (p + 46 + nlen > b.size()) bad("zip: truncated");
            const std::string name((const char*)&b[p + 46], nlen);
            if (method != 0) bad("zip entry " + name + " is compressed (method " + std::to_string(method) + "); only STORED entries are read");
            if (csize != usize || csize == 0xffffffffu) bad("zip entry " + name + ": unsupported sizes");
            if (u32(lho) != 0x04034b50u) bad("zip: bad local header of " + name);
            const size_t data = (size_t)lho + 30 + u16(lho + 26) + u16(lho + 28);
            if (data + csize > b.size()) bad("zip entry " + name + " runs past the end of the file");
            entries[name] = {data, csize};
            p += 46 + (size_t)nlen + xlen + clen;
        }
    }
    bool has(const std::string& name) const { return entries.count(name) != 0; }
    std::pair<const uint8_t*, size_t> get(const std::string& name) const {
        auto it = entries.find(name);
        if (it == entries.end()) bad("zip entry " + name + " missing");
        return {bytes.data() + it->second.first, it->second.second};
    }
};

// ------------------------------------------------------------------ pickle values
struct Val;
using VP = std::shared_ptr<Val>;
enum Kind { K_NONE, K_BOOL, K_INT, K_STR, K_TUPLE, K_DICT, K_GLOBAL, K_STORAGE, K_TENSOR, K_MARK };
struct Val {
    Kind kind = K_NONE;
    int64_t i = 0;
    std::string s;                        // string, global name, storage key
    std::vector<VP> items;                // tuple
    std::vector<std::pair<VP, VP>> dict;  // dict entries in insertion order
    int64_t offset = 0;                   // tensor view
    std::vector<int64_t> shape, stride;
};
VP mk(Kind k) {
    auto v = std::make_shared<Val>();
    v->kind = k;
    return v;
}

std::vector<int64_t> int_tuple(const VP& v, const char* what) {
    if (v->kind != K_TUPLE) bad(std::string("pickle: ") + what + " is not a tuple");
    std::vector<int64_t> r;
    for (auto& x : v->items) {
        if (x->kind != K_INT || x->i < 0) bad(std::string("pickle: ") + what + " holds a non-index");
        r.push_back(x->i);
    }
    return r;
}

// Interprets the pickle program; returns the root object.
VP unpickle(const uint8_t* d, size_t n) {
    std::vector<VP> st;
    std::map<uint32_t, VP> memo;
    size_t i = 0;
    auto take = [&](size_t k) -> const uint8_t* {
        if (i + k > n) bad("pickle: truncated");
        const uint8_t* p = d + i;
        i += k;
        return p;
    };
    auto le = [](const uint8_t* p, int k) {
        uint64_t v = 0;
        for (int j = k - 1; j >= 0; j--) v = (v << 8) | p[j];
        return v;
    };
    auto pop = [&]() {
        if (st.empty()) bad("pickle: stack underflow");
        VP v = st.back();
        st.pop_back();
        return v;
    };
    auto pop_to_mark = [&]() {
        size_t m = st.size();
        while (m > 0 && st[m - 1]->kind != K_MARK) m--;
        if (m == 0) bad("pickle: MARK not found");
        std::vector<VP> items(st.begin() + m, st.end());
        st.resize(m - 1);
        return items;
    };
    auto top_dict = [&]() -> Val& {
        if (st.empty() || st.back()->kind != K_DICT) bad("pickle: SETITEM(S) on a non-dict");
        return *st.back();
    };
    for (;;) {
        const uint8_t op = *take(1);
        switch (op) {
            case 0x80: take(1); break;  // PROTO
            case '}': st.push_back(mk(K_DICT)); break;
            case ')': case ']': st.push_back(mk(K_TUPLE)); break;  // EMPTY_TUPLE, EMPTY_LIST
            case 'N': st.push_back(mk(K_NONE)); break;
            case 0x88: case 0x89: {  // NEWTRUE, NEWFALSE
                VP v = mk(K_BOOL);
                v->i = op == 0x88;
                st.push_back(v);
                break;
            }
            case '(': st.push_back(mk(K_MARK)); break;
            case 'X': {  // BINUNICODE
                const uint64_t len = le(take(4), 4);
                VP v = mk(K_STR);
                v->s.assign((const char*)take(len), len);
                st.push_back(v);
                break;
            }
            case 0x8c: {  // SHORT_BINUNICODE
                const uint64_t len = *take(1);
                VP v = mk(K_STR);
                v->s.assign((const char*)take(len), len);
                st.push_back(v);
                break;
            }
            case 'J': case 'K': case 'M': {  // BININT, BININT1, BININT2
                VP v = mk(K_INT);
                v->i = op == 'J' ? (int64_t)(int32_t)(uint32_t)le(take(4), 4) : (int64_t)le(take(op == 'K' ? 1 : 2), op == 'K' ? 1 : 2);
                st.push_back(v);
                break;
            }
            case 0x8a: {  // LONG1: little-endian two's complement of up to 8 bytes
                const int len = *take(1);
                if (len > 8) bad("pickle: integer wider than 64 bits");
                const uint8_t* p = take(len);
                uint64_t u = le(p, len);
                if (len > 0 && len < 8 && (p[len - 1] & 0x80)) u |= ~0ull << (8 * len);
                VP v = mk(K_INT);
                v->i = (int64_t)u;
                st.push_back(v);
                break;
            }
            case 'q': case 'r': {  // BINPUT, LONG_BINPUT
                const uint32_t k = (uint32_t)le(take(op == 'q' ? 1 : 4), op == 'q' ? 1 : 4);
                if (st.empty()) bad("pickle: BINPUT on an empty stack");
                memo[k] = st.back();
                break;
            }
            case 'h': case 'j': {  // BINGET, LONG_BINGET
                const uint32_t k = (uint32_t)le(take(op == 'h' ? 1 : 4), op == 'h' ? 1 : 4);
                auto it = memo.find(k);
                if (it == memo.end()) bad("pickle: BINGET of an unset memo slot");
                st.push_back(it->second);
                break;
            }
            case 'c': {  // GLOBAL "module\nname\n"
                auto line = [&]() {
                    const size_t b = i;
                    while (i < n && d[i] != '\n') i++;
                    if (i >= n) bad("pickle: bad GLOBAL");
                    std::string s((const char*)d + b, i - b);
                    i++;
                    return s;
                };
                const std::string mod = line(), name = line();
                const std::string g = mod + "." + name;
                if (g != "collections.OrderedDict" && g != "torch._utils._rebuild_tensor_v2" && g != "torch.FloatStorage")
                    bad("pickle: refusing global " + g + " (only float32 tensors in dicts are read)");
                VP v = mk(K_GLOBAL);
                v->s = g;
                st.push_back(v);
                break;
            }
            case 't': {
                VP v = mk(K_TUPLE);
                v->items = pop_to_mark();
                st.push_back(v);
                break;
            }
            case 0x85: case 0x86: case 0x87: {  // TUPLE1..3
                const size_t k = op - 0x84;
                if (st.size() < k) bad("pickle: stack underflow");
                VP v = mk(K_TUPLE);
                v->items.assign(st.end() - k, st.end());
                st.resize(st.size() - k);
                st.push_back(v);
                break;
            }
            case 'Q': {  // BINPERSID: ("storage", torch.FloatStorage, key, location, numel)
                VP pid = pop();
                if (pid->kind != K_TUPLE || pid->items.size() != 5 || pid->items[0]->kind != K_STR ||
                    pid->items[0]->s != "storage" || pid->items[1]->kind != K_GLOBAL ||
                    pid->items[1]->s != "torch.FloatStorage" || pid->items[2]->kind != K_STR)
                    bad("pickle: unsupported persistent id (only float32 storages are read)");
                VP v = mk(K_STORAGE);
                v->s = pid->items[2]->s;
                st.push_back(v);
                break;
            }
            case 'R': {  // REDUCE
                VP args = pop(), f = pop();
                if (f->kind != K_GLOBAL || args->kind != K_TUPLE) bad("pickle: unsupported REDUCE");
                if (f->s == "collections.OrderedDict") {
                    st.push_back(mk(K_DICT));
                } else if (f->s == "torch._utils._rebuild_tensor_v2") {
                    const auto& a = args->items;
                    if (a.size() < 4 || a[0]->kind != K_STORAGE || a[1]->kind != K_INT || a[1]->i < 0)
                        bad("pickle: bad _rebuild_tensor_v2 arguments");
                    VP v = mk(K_TENSOR);
                    v->s = a[0]->s;
                    v->offset = a[1]->i;
                    v->shape = int_tuple(a[2], "tensor shape");
                    v->stride = int_tuple(a[3], "tensor stride");
                    if (v->shape.size() != v->stride.size()) bad("pickle: shape and stride ranks differ");
                    st.push_back(v);
                } else {
                    bad("pickle: REDUCE of " + f->s);
                }
                break;
            }
            case 'b': pop(); break;  // BUILD: the state (OrderedDict metadata) is not needed
            case 's': {              // SETITEM
                VP v = pop(), k = pop();
                top_dict().dict.emplace_back(k, v);
                break;
            }
            case 'u': {  // SETITEMS
                auto items = pop_to_mark();
                if (items.size() % 2) bad("pickle: SETITEMS with an odd count");
                Val& dd = top_dict();
                for (size_t j = 0; j < items.size(); j += 2) dd.dict.emplace_back(items[j], items[j + 1]);
                break;
            }
            case '.': return pop();  // STOP
            default: {
                char buf[64];
                std::snprintf(buf, sizeof(buf), "pickle: unsupported opcode 0x%02x at %zu", op, i - 1);
                bad(buf);
            }
        }
    }
}

struct Loader {
    std::vector<uint8_t> bytes;
    std::unique_ptr<Archive> zip;
    std::string prefix;  // "<archive name>/"
    VP root;

    // path: the file's name in messages (the archive is `data`, read from it or handed over)
    Loader(std::vector<uint8_t> data, const std::string& path) : bytes(std::move(data)) {
        zip = std::make_unique<Archive>(bytes);
        std::string pkl;
        for (auto& e : zip->entries) {
            const std::string& nm = e.first;
            if (nm.size() >= 9 && nm.compare(nm.size() - 9, 9, "/data.pkl") == 0) {
                pkl = nm;
                break;
            }
        }
        if (pkl.empty()) bad(path + ": no data.pkl (not a torch.save archive)");
        prefix = pkl.substr(0, pkl.size() - 8);
        if (zip->has(prefix + "byteorder")) {
            auto bo = zip->get(prefix + "byteorder");
            if (std::string((const char*)bo.first, bo.second) != "little") bad(path + ": big-endian storages are not read");
        }
        auto p = zip->get(pkl);
        root = unpickle(p.first, p.second);
    }

    // A tensor view as a contiguous row-major copy of its storage.
    HostTensor tensor(const VP& v) const {
        if (v->kind != K_TENSOR) bad("expected a tensor");
        auto raw = zip->get(prefix + "data/" + v->s);
        if (raw.second % 4) bad("storage " + v->s + ": size not a multiple of 4");
        const int64_t total = (int64_t)(raw.second / 4);
        HostTensor t;
        t.shape = v->shape;
        // The view's extent, overflow-checked: with a non-negative offset, sizes and strides, every
        // element's offset lies in [offset, last], so last < total bounds every read below.
        if (v->stride.size() != v->shape.size() || v->offset < 0) bad("tensor view of " + v->s + ": bad offset or rank");
        int64_t numel = 1, last = v->offset;
        for (size_t d = 0; d < v->shape.size(); d++) {
            const int64_t n = v->shape[d], st = v->stride[d];
            if (n < 0 || st < 0) bad("tensor view of " + v->s + ": negative size or stride");
            int64_t span = 0;
            if (__builtin_mul_overflow(numel, n, &numel) ||
                (n > 0 && (__builtin_mul_overflow(n - 1, st, &span) || __builtin_add_overflow(last, span, &last))))
                bad("tensor view of " + v->s + ": size overflows");
        }
        if (numel > ((int64_t)1 << 28)) bad("tensor view of " + v->s + ": more than 2^28 elements");
        if (numel > 0 && last >= total) bad("tensor view runs past storage " + v->s);
        t.data.resize((size_t)numel);
        auto at = [&](int64_t k) {
            float f;
            std::memcpy(&f, raw.first + 4 * k, 4);
            return f;
        };
        // row-major contiguous: one range of the storage
        bool contiguous = true;
        int64_t expect = 1;
        for (int d = (int)v->shape.size() - 1; d >= 0; d--) {
            if (v->shape[d] != 1 && v->stride[d] != expect) contiguous = false;
            expect *= v->shape[d];
        }
        if (contiguous) {
            if (numel) std::memcpy(t.data.data(), raw.first + 4 * v->offset, 4 * (size_t)numel);
            return t;
        }
        const int nd = (int)v->shape.size();
        std::vector<int64_t> idx(nd, 0);
        for (int64_t k = 0; k < numel; k++) {
            int64_t off = v->offset;
            for (int d = 0; d < nd; d++) off += idx[d] * v->stride[d];
            t.data[(size_t)k] = at(off);
            for (int d = nd - 1; d >= 0; d--) {
                if (++idx[d] < v->shape[d]) break;
                idx[d] = 0;
            }
        }
        return t;
    }
};

const std::string& key_str(const VP& k) {
    if (k->kind != K_STR) bad("checkpoint: non-string dictionary key");
    return k->s;
}

}  // namespace

std::map<std::string, HostTensor> read_model_checkpoint_bytes(std::vector<uint8_t> data, const std::string& path) {
    Loader ld(std::move(data), path);
    if (ld.root->kind != K_DICT) bad(path + ": the root object is not a dict of state dicts");
    std::map<std::string, HostTensor> out;
    for (auto& kv : ld.root->dict) {
        const std::string& sub = key_str(kv.first);
        if (kv.second->kind != K_DICT) bad(path + ": " + sub + " is not a state dict");
        for (auto& pv : kv.second->dict) {
            std::string name = key_str(pv.first);
            if (name.compare(0, 7, "module.") == 0) name = name.substr(7);
            out[sub + "." + name] = ld.tensor(pv.second);
        }
    }
    return out;
}

std::map<std::string, HostTensor> read_model_checkpoint(const std::string& path) {
    return read_model_checkpoint_bytes(read_file(path), path);
}

HostTensor read_voice_pack_bytes(std::vector<uint8_t> data, const std::string& path) {
    Loader ld(std::move(data), path);
    HostTensor t = ld.tensor(ld.root);
    if (t.shape.size() != 3 || t.shape[1] != 1 || t.shape[2] != 256) {
        std::string s;
        for (auto d : t.shape) s += (s.empty() ? "" : ", ") + std::to_string(d);
        bad(path + ": voice pack of shape [" + s + "], expected [rows, 1, 256]");
    }
    return t;
}

HostTensor read_voice_pack(const std::string& path) { return read_voice_pack_bytes(read_file(path), path); }

void weight_norm(const float* v, const float* g, int64_t rows, int64_t per_row, float* w) {
    for (int64_t r = 0; r < rows; r++) {
        const float* vr = v + r * per_row;
        double ss = 0.0;
        for (int64_t j = 0; j < per_row; j++) ss += (double)vr[j] * (double)vr[j];
        const float norm = (float)std::sqrt(ss);
        const float scale = g[r] / norm;
        for (int64_t j = 0; j < per_row; j++) w[r * per_row + j] = vr[j] * scale;
    }
}

}  // namespace kk
