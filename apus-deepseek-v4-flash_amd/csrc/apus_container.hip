/*
 * apus_container.hip — index of the routed-expert slabs of an apus model
 * container (host code; no device use).
 *
 * Container format (c/st.h:1-31, tools/convert.py): a shard is an 8-byte
 * little-endian header length N, N bytes of JSON {"name": {"dtype", "shape",
 * "data_offsets": [a, b]}, ...}, then the payloads (offsets relative to the
 * end of the header). model.safetensors.index.json maps every tensor name to
 * its shard under "weight_map".
 *
 * The slab rules follow apus_store_open (c/cache.h:1030-1110) and
 * apus_store_derive_slab (:431-509): expert names are matched exactly
 * (canonical decimal numbers, kind "weight" or "scale"); MTP block K maps to
 * store layer n_main + K; every expert needs all six tensors in one shard,
 * tiling one contiguous byte range; weights are I8 [O, K/2], scales F8_E8M0
 * [O, K/32]; every slab has the same size. Beyond the reference, a slab must
 * also lie inside its shard file.
 */
#include "apus_container.h"

#include <stdio.h>
#include <string.h>
#include <sys/stat.h>

#include <algorithm>
#include <map>
#include <memory>

namespace {

/* ------------------------------------------------------------- JSON */

/* A small JSON reader for index and shard headers: objects keep their keys
 * in file order, numbers are kept as doubles (tensor offsets in shards stay
 * below 2^53). */
struct JNode {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    double num = 0;
    std::string str;
    std::vector<JNode> items;                        /* ARR elements, OBJ values */
    std::vector<std::string> keys;                   /* OBJ keys */
    const JNode *get(const char *k) const {
        if (kind != OBJ) return nullptr;
        for (size_t i = 0; i < keys.size(); i++)
            if (keys[i] == k) return &items[i];
        return nullptr;
    }
};

struct JParser {
    const char *p, *end;
    std::string err;

    void ws() {
        while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
    }
    bool fail(const char *what) {
        if (err.empty()) err = what;
        return false;
    }
    bool hex4(unsigned &v) {
        if (end - p < 4) return fail("short \\u escape");
        v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = *p++;
            v <<= 4;
            if (c >= '0' && c <= '9') v |= c - '0';
            else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
            else return fail("bad \\u escape");
        }
        return true;
    }
    void utf8(std::string &s, unsigned cp) {
        if (cp < 0x80) s += (char)cp;
        else if (cp < 0x800) { s += (char)(0xc0 | (cp >> 6)); s += (char)(0x80 | (cp & 0x3f)); }
        else if (cp < 0x10000) {
            s += (char)(0xe0 | (cp >> 12)); s += (char)(0x80 | ((cp >> 6) & 0x3f));
            s += (char)(0x80 | (cp & 0x3f));
        } else {
            s += (char)(0xf0 | (cp >> 18)); s += (char)(0x80 | ((cp >> 12) & 0x3f));
            s += (char)(0x80 | ((cp >> 6) & 0x3f)); s += (char)(0x80 | (cp & 0x3f));
        }
    }
    bool string(std::string &s) {
        if (p >= end || *p != '"') return fail("expected string");
        p++;
        while (p < end && *p != '"') {
            if (*p != '\\') { s += *p++; continue; }
            if (++p >= end) break;
            const char c = *p++;
            switch (c) {
            case '"': s += '"'; break;
            case '\\': s += '\\'; break;
            case '/': s += '/'; break;
            case 'b': s += '\b'; break;
            case 'f': s += '\f'; break;
            case 'n': s += '\n'; break;
            case 'r': s += '\r'; break;
            case 't': s += '\t'; break;
            case 'u': {
                unsigned cp;
                if (!hex4(cp)) return false;
                if (cp >= 0xd800 && cp < 0xdc00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
                    p += 2;
                    unsigned lo;
                    if (!hex4(lo)) return false;
                    cp = 0x10000 + ((cp - 0xd800) << 10) + (lo - 0xdc00);
                }
                utf8(s, cp);
                break;
            }
            default: return fail("bad escape");
            }
        }
        if (p >= end) return fail("unterminated string");
        p++;
        return true;
    }
    bool value(JNode &n, int depth) {
        if (depth > 64) return fail("nesting too deep");
        ws();
        if (p >= end) return fail("unexpected end");
        const char c = *p;
        if (c == '{') {
            n.kind = JNode::OBJ;
            p++;
            ws();
            if (p < end && *p == '}') { p++; return true; }
            for (;;) {
                ws();
                std::string k;
                if (!string(k)) return false;
                ws();
                if (p >= end || *p != ':') return fail("expected ':'");
                p++;
                n.keys.push_back(std::move(k));
                n.items.emplace_back();
                if (!value(n.items.back(), depth + 1)) return false;
                ws();
                if (p < end && *p == ',') { p++; continue; }
                if (p < end && *p == '}') { p++; return true; }
                return fail("expected ',' or '}'");
            }
        }
        if (c == '[') {
            n.kind = JNode::ARR;
            p++;
            ws();
            if (p < end && *p == ']') { p++; return true; }
            for (;;) {
                n.items.emplace_back();
                if (!value(n.items.back(), depth + 1)) return false;
                ws();
                if (p < end && *p == ',') { p++; continue; }
                if (p < end && *p == ']') { p++; return true; }
                return fail("expected ',' or ']'");
            }
        }
        if (c == '"') { n.kind = JNode::STR; return string(n.str); }
        if (end - p >= 4 && !strncmp(p, "true", 4)) { n.kind = JNode::BOOL; n.num = 1; p += 4; return true; }
        if (end - p >= 5 && !strncmp(p, "false", 5)) { n.kind = JNode::BOOL; p += 5; return true; }
        if (end - p >= 4 && !strncmp(p, "null", 4)) { n.kind = JNode::NUL; p += 4; return true; }
        /* number */
        const char *q = p;
        if (q < end && (*q == '-' || *q == '+')) q++;
        while (q < end && ((*q >= '0' && *q <= '9') || *q == '.' || *q == 'e' || *q == 'E' ||
                           *q == '-' || *q == '+'))
            q++;
        if (q == p) return fail("unexpected character");
        n.kind = JNode::NUM;
        n.num = strtod(std::string(p, q).c_str(), nullptr);
        p = q;
        return true;
    }
};

bool parse_json(const char *buf, size_t n, JNode &out, std::string &err) {
    JParser jp{buf, buf + n, {}};
    if (!jp.value(out, 0)) { err = jp.err; return false; }
    jp.ws();
    if (jp.p != jp.end) { err = "trailing characters"; return false; }
    return true;
}

bool read_file(const std::string &path, std::string &out) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) return false;
    char buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, n);
    const bool ok = !ferror(f);
    fclose(f);
    return ok;
}

bool file_exists(const std::string &path) {
    struct stat sb;
    return stat(path.c_str(), &sb) == 0 && S_ISREG(sb.st_mode);
}

/* ------------------------------------------------------ shard headers */

enum Dtype { DT_I8, DT_U8, DT_F8_E8M0, DT_F8_E4M3, DT_BF16, DT_F16, DT_F32, DT_I32, DT_I64, DT_OTHER };

Dtype dtype_of(const std::string &s) {
    static const std::pair<const char *, Dtype> tab[] = {
        {"I8", DT_I8}, {"U8", DT_U8}, {"F8_E8M0", DT_F8_E8M0}, {"F8_E4M3", DT_F8_E4M3},
        {"BF16", DT_BF16}, {"F16", DT_F16}, {"F32", DT_F32}, {"I32", DT_I32}, {"I64", DT_I64}};
    for (const auto &t : tab)
        if (s == t.first) return t.second;
    return DT_OTHER;
}

struct ShardTensor {
    Dtype dtype = DT_OTHER;
    std::vector<int64_t> shape;
    uint64_t file_off = 0, nbytes = 0;
};

struct Shard {
    uint64_t file_size = 0;
    std::map<std::string, ShardTensor> tensors;
};

bool read_shard_header(const std::string &path, Shard &sh, std::string &err) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) { err = "cannot open shard " + path; return false; }
    uint8_t lenb[8];
    if (fread(lenb, 1, 8, f) != 8) { fclose(f); err = "short shard " + path; return false; }
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | lenb[i];
    struct stat sb;
    if (fstat(fileno(f), &sb) != 0 || hlen > (1ull << 28) || 8 + hlen > (uint64_t)sb.st_size) {
        fclose(f);
        err = "bad header in " + path;
        return false;
    }
    sh.file_size = (uint64_t)sb.st_size;
    std::string hbuf(hlen, '\0');
    const bool got = fread(&hbuf[0], 1, hlen, f) == hlen;
    fclose(f);
    if (!got) { err = "header read failed " + path; return false; }
    JNode hdr;
    std::string jerr;
    if (!parse_json(hbuf.data(), hbuf.size(), hdr, jerr) || hdr.kind != JNode::OBJ) {
        err = "header JSON of " + path + ": " + (jerr.empty() ? "not an object" : jerr);
        return false;
    }
    const uint64_t base = 8 + hlen;
    for (size_t i = 0; i < hdr.keys.size(); i++) {
        if (hdr.keys[i] == "__metadata__") continue;
        const JNode &m = hdr.items[i];
        ShardTensor t;
        const JNode *dt = m.get("dtype");
        t.dtype = dtype_of(dt && dt->kind == JNode::STR ? dt->str : "");
        const JNode *shp = m.get("shape");
        if (shp && shp->kind == JNode::ARR)
            for (const JNode &d : shp->items) t.shape.push_back((int64_t)d.num);
        const JNode *off = m.get("data_offsets");
        if (!off || off->kind != JNode::ARR || off->items.size() != 2 ||
            off->items[1].num < off->items[0].num) {
            err = "bad data_offsets for " + hdr.keys[i] + " in " + path;
            return false;
        }
        t.file_off = base + (uint64_t)off->items[0].num;
        t.nbytes = (uint64_t)off->items[1].num - (uint64_t)off->items[0].num;
        sh.tensors[hdr.keys[i]] = std::move(t);
    }
    return true;
}

/* ------------------------------------------------------ expert names */

/* "<prefix>.<L>.ffn.experts.<E>.w<W>.<weight|scale>" with canonical decimal
 * numbers (no sign, no leading zeros): the names tools/convert.py writes and
 * c/cache.h:381-407 accepts */
bool parse_uint(const char *&s, int &v) {
    if (*s < '0' || *s > '9') return false;
    if (*s == '0' && s[1] >= '0' && s[1] <= '9') return false;
    long long x = 0;
    while (*s >= '0' && *s <= '9') {
        x = x * 10 + (*s++ - '0');
        if (x > 0x7fffffff) return false;
    }
    v = (int)x;
    return true;
}

bool expect(const char *&s, const char *lit) {
    const size_t n = strlen(lit);
    if (strncmp(s, lit, n)) return false;
    s += n;
    return true;
}

bool parse_expert_name(const std::string &name, int &layer, int &eid, int &w, int &is_scale,
                       int &is_mtp) {
    const char *s = name.c_str();
    if (expect(s, "layers.")) is_mtp = 0;
    else if (expect(s, "mtp.")) is_mtp = 1;
    else return false;
    if (!parse_uint(s, layer) || !expect(s, ".ffn.experts.") || !parse_uint(s, eid) ||
        !expect(s, ".w") || !parse_uint(s, w) || w < 1 || w > 3 || !expect(s, "."))
        return false;
    if (!strcmp(s, "weight")) is_scale = 0;
    else if (!strcmp(s, "scale")) is_scale = 1;
    else return false;
    return true;
}

struct Ref {
    int layer, eid, w, is_scale, is_mtp;
    std::string shard;
};

std::string member_name(const ApusHipContainer &c, const Ref &r) {
    char buf[200];
    const int n_main = c.n_layers - c.n_mtp;
    snprintf(buf, sizeof buf, "%s.%d.ffn.experts.%d.w%d.%s", r.is_mtp ? "mtp" : "layers",
             r.is_mtp ? r.layer - n_main : r.layer, r.eid, r.w, r.is_scale ? "scale" : "weight");
    return buf;
}

}  // namespace

ApusHipContainer *apus_container_index(const char *model_dir, int n_layers, int n_mtp, int E,
                                       std::string &err) {
    char msg[512];
    if (!model_dir || n_layers <= 0 || E <= 0 || n_mtp < 0 || n_mtp > n_layers) {
        err = "container: n_layers/n_experts required";
        return nullptr;
    }
    std::unique_ptr<ApusHipContainer> c(new ApusHipContainer());
    c->n_layers = n_layers; c->n_mtp = n_mtp; c->E = E;
    const std::string md(model_dir);
    c->dir = file_exists(md + "/model.safetensors.index.json") ? md : md + "/weights";
    const std::string ipath = c->dir + "/model.safetensors.index.json";
    std::string ibuf;
    if (!read_file(ipath, ibuf)) { err = "container: cannot read " + ipath; return nullptr; }
    JNode idx;
    std::string jerr;
    if (!parse_json(ibuf.data(), ibuf.size(), idx, jerr)) {
        err = "container: " + ipath + ": " + jerr;
        return nullptr;
    }
    const JNode *wm = idx.get("weight_map");
    if (!wm || wm->kind != JNode::OBJ) { err = "container: no weight_map in " + ipath; return nullptr; }

    const int n_main = n_layers - n_mtp;
    std::vector<Ref> refs;
    std::vector<int> have((size_t)n_layers * E, 0);
    for (size_t i = 0; i < wm->keys.size(); i++) {
        Ref r;
        if (!parse_expert_name(wm->keys[i], r.layer, r.eid, r.w, r.is_scale, r.is_mtp)) continue;
        if (r.is_mtp) {
            if (r.layer >= n_mtp) continue;
            r.layer += n_main;
        } else if (r.layer >= n_main) {
            continue;
        }
        if (r.layer >= n_layers || r.eid >= E) continue;
        if (wm->items[i].kind != JNode::STR) {
            err = "container: weight_map entry of " + wm->keys[i] + " is not a string";
            return nullptr;
        }
        r.shard = wm->items[i].str;
        refs.push_back(std::move(r));
        have[(size_t)refs.back().layer * E + refs.back().eid]++;
    }
    for (int i = 0; i < n_layers * E; i++)
        if (have[i] != 6) {
            snprintf(msg, sizeof msg, "container: expert %d.%d has %d/6 tensors in weight_map",
                     i / E, i % E, have[i]);
            err = msg;
            return nullptr;
        }
    std::sort(refs.begin(), refs.end(), [](const Ref &a, const Ref &b) {
        if (a.layer != b.layer) return a.layer < b.layer;
        if (a.eid != b.eid) return a.eid < b.eid;
        if (a.w != b.w) return a.w < b.w;
        return a.is_scale < b.is_scale;
    });

    std::map<std::string, int> shard_id;
    std::vector<Shard> shards;
    auto shard_of = [&](const std::string &name) -> int {
        auto it = shard_id.find(name);
        if (it != shard_id.end()) return it->second;
        Shard sh;
        if (!read_shard_header(c->dir + "/" + name, sh, err)) return -1;
        shards.push_back(std::move(sh));
        c->shards.push_back(name);
        const int id = (int)shards.size() - 1;
        shard_id[name] = id;
        return id;
    };

    c->recs.resize((size_t)n_layers * E);
    for (size_t i = 0; i < refs.size(); i += 6) {
        const Ref *m6 = &refs[i];
        const int layer = m6[0].layer, eid = m6[0].eid;
        /* duplicates in the weight map would leave a member out */
        for (int j = 0; j < 6; j++)
            if (m6[j].layer != layer || m6[j].eid != eid || m6[j].w != 1 + j / 2 ||
                m6[j].is_scale != (j & 1)) {
                snprintf(msg, sizeof msg, "container: expert %d.%d has a duplicate member", layer, eid);
                err = msg;
                return nullptr;
            }
        const int sid = shard_of(m6[0].shard);
        if (sid < 0) return nullptr;
        const ShardTensor *mem[6];
        for (int j = 0; j < 6; j++) {
            if (m6[j].shard != m6[0].shard) {
                snprintf(msg, sizeof msg, "container: expert %d.%d split across shards", layer, eid);
                err = msg;
                return nullptr;
            }
            const std::string tn = member_name(*c, m6[j]);
            auto it = shards[sid].tensors.find(tn);
            if (it == shards[sid].tensors.end()) {
                err = "container: missing tensor " + tn;
                return nullptr;
            }
            mem[j] = &it->second;
        }
        int ord[6] = {0, 1, 2, 3, 4, 5};
        std::sort(ord, ord + 6, [&](int a, int b) { return mem[a]->file_off < mem[b]->file_off; });
        const uint64_t base = mem[ord[0]]->file_off;
        uint64_t cur = base;
        for (int j = 0; j < 6; j++) {
            if (mem[ord[j]]->file_off != cur) {
                snprintf(msg, sizeof msg,
                         "container: expert %d.%d slab not contiguous (gap at member %d)", layer,
                         eid, ord[j]);
                err = msg;
                return nullptr;
            }
            cur += mem[ord[j]]->nbytes;
        }
        ApusHipSlabRec &rec = c->recs[(size_t)layer * E + eid];
        rec.shard = sid;
        rec.off = base;
        rec.len = cur - base;
        if (cur > shards[sid].file_size) {
            snprintf(msg, sizeof msg, "container: expert %d.%d slab runs past the end of %s", layer,
                     eid, m6[0].shard.c_str());
            err = msg;
            return nullptr;
        }
        for (int j = 0; j < 6; j++) rec.rel[j] = (uint32_t)(mem[j]->file_off - base);
        for (int t = 0; t < 3; t++) {
            const ShardTensor *wt = mem[2 * t], *sc = mem[2 * t + 1];
            if (wt->dtype != DT_I8 || sc->dtype != DT_F8_E8M0 || wt->shape.size() != 2 ||
                sc->shape.size() != 2 || wt->shape[0] != sc->shape[0] ||
                wt->shape[1] * 2 != sc->shape[1] * 32 ||
                wt->nbytes != (uint64_t)(wt->shape[0] * wt->shape[1]) ||
                sc->nbytes != (uint64_t)(sc->shape[0] * sc->shape[1])) {
                snprintf(msg, sizeof msg, "container: expert %d.%d w%d shape/dtype mismatch",
                         layer, eid, t + 1);
                err = msg;
                return nullptr;
            }
            rec.O[t] = wt->shape[0];
            rec.K[t] = wt->shape[1] * 2;
        }
        if (c->slab_bytes == 0) c->slab_bytes = rec.len;
        if (rec.len != c->slab_bytes) {
            snprintf(msg, sizeof msg, "container: expert %d.%d slab %llu != slab_bytes %llu", layer,
                     eid, (unsigned long long)rec.len, (unsigned long long)c->slab_bytes);
            err = msg;
            return nullptr;
        }
    }
    return c.release();
}

extern "C" {

ApusHipContainer *apus_hip_container_open(const char *model_dir, int n_layers, int n_mtp,
                                          int n_experts, char *err, size_t errcap) {
    std::string e;
    ApusHipContainer *c = apus_container_index(model_dir, n_layers, n_mtp, n_experts, e);
    if (!c && err && errcap) snprintf(err, errcap, "%s", e.c_str());
    return c;
}

void apus_hip_container_close(ApusHipContainer *c) { delete c; }

int apus_hip_container_slab(const ApusHipContainer *c, int layer, int eid, ApusHipSlabRec *out) {
    if (!c || !out || layer < 0 || layer >= c->n_layers || eid < 0 || eid >= c->E) return 1;
    *out = c->recs[(size_t)layer * c->E + eid];
    return 0;
}

const char *apus_hip_container_shard(const ApusHipContainer *c, int i) {
    if (!c || i < 0 || i >= (int)c->shards.size()) return nullptr;
    return c->shards[i].c_str();
}

}  // extern "C"
