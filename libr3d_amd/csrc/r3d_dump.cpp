/* r3d_dump.cpp -- env-gated capture of row launches for offline replay (the reference's
 * R3D_DUMP, src/r3d_dump.h:1-35, src/r3d_dump.hip:149-302).
 *
 * With R3D_DUMP=<dir> set, the first R3D_DUMP_MAX (default 2) launches of every row whose
 * name contains one of the comma-separated R3D_DUMP_OPS substrings (default: every row of
 * this library) are captured: the byte span each operand's view covers, before and after
 * the launch, the launch scratch likewise, every parameter and tunable.  A capture is
 * <dir>/<seq>_<row>/ holding manifest.tsv, pre.bin and post.bin (the operands' spans, in
 * operand order, then the scratch span); tests/replay_dump.py rebuilds the launch from it
 * and diffs what the GPU wrote against the oracle, or re-launches it on the device.
 *
 * manifest.tsv lines (tab-separated), as the reference writes them plus two of this
 * library's own:
 *   H  row  rc  n_t  n_p
 *   P  kind  key  ival  ihi  sval|-  dval
 *   T  index  dtype  rank  shape...  stride...  bytes  truncated  null  address
 *   V  name  value                             (one per engine tunable)
 *   X  scratch_bytes  captured_bytes  truncated (the launch scratch, when given)
 *
 * A span is what a strided view touches: 1 + sum (shape - 1) * stride elements from the
 * data pointer; FP4 counts nibbles, so its span is ceil(elements / 2) bytes.  Spans over
 * R3D_DUMP_CAP bytes (default 32 MiB) are cut there and flagged.  This is a debug path: a
 * captured launch synchronises its stream and copies through the host, which no production
 * launch may do -- hence the gate; unset, a wrapped entry costs one branch.
 */
#include "r3d_dump.h"

#include <hip/hip_runtime_api.h>

#include <sys/stat.h>
#include <sys/types.h>

#include <mutex>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <string>
#include <vector>

namespace r3d {
namespace {

struct DumpConfig {
    bool on = false;
    std::string dir;
    std::vector<std::string> ops;
    int per_row = 2;
    size_t cap = (size_t)32 << 20;
};

const DumpConfig& config() {
    static const DumpConfig c = [] {
        DumpConfig x;
        const char* d = getenv("R3D_DUMP");
        if (!d || !*d) return x;
        x.on = true;
        x.dir = d;
        const char* o = getenv("R3D_DUMP_OPS");
        std::string ops =
            o && *o ? o : "gemm_nt_q,quant_act_fp8,gated_quant_fp8,rmsnorm_quant_fp8,logits_gemm";
        size_t p = 0;
        while (p <= ops.size()) {
            const size_t e = ops.find(',', p);
            const std::string tok = ops.substr(p, e == std::string::npos ? std::string::npos : e - p);
            if (!tok.empty()) x.ops.push_back(tok);
            if (e == std::string::npos) break;
            p = e + 1;
        }
        if (const char* n = getenv("R3D_DUMP_MAX")) {
            const int v = atoi(n);
            if (v >= 0) x.per_row = v;
        }
        if (const char* n = getenv("R3D_DUMP_CAP")) {
            const long long v = atoll(n);
            if (v > 0) x.cap = (size_t)v;
        }
        return x;
    }();
    return c;
}

/* bytes of the span a view covers (see the header comment) */
size_t span_bytes(const RadTensor& t) {
    if (!t.data) return 0;
    long long els = 1;
    for (uint32_t r = 0; r < t.rank && r < RAD_MAX_RANK; ++r) {
        long long step = 0;
        if (t.shape[r] <= 0 || t.stride[r] < 0 ||
            __builtin_mul_overflow((long long)(t.shape[r] - 1), (long long)t.stride[r], &step) ||
            __builtin_add_overflow(els, step, &els) || els > (1LL << 40))
            return 0;                                     /* no span a capture could copy */
    }
    switch (t.dtype) {
        case RAD_FP4E2M1: return (size_t)((els + 1) / 2);
        case RAD_F32: case RAD_I32: case RAD_U32: return (size_t)els * 4;
        case RAD_I64: return (size_t)els * 8;
        case RAD_BF16: case RAD_F16: case RAD_I16: return (size_t)els * 2;
        default: return (size_t)els;                      /* the one-byte formats */
    }
}

bool to_host(std::vector<uint8_t>& out, const void* dev, size_t n) {
    out.resize(n);
    return n == 0 || hipMemcpy(out.data(), dev, n, hipMemcpyDeviceToHost) == hipSuccess;
}

void make_dirs(const std::string& path) {
    for (size_t i = 1; i <= path.size(); ++i)
        if (i == path.size() || path[i] == '/') mkdir(path.substr(0, i).c_str(), 0777);
}

std::mutex g_mu;
std::vector<std::pair<std::string, int>> g_counts;    /* captures taken per row */

struct Capture {
    std::string row;
    int seq = 0;
    std::vector<std::vector<uint8_t>> pre, post;
    std::vector<size_t> bytes;
    std::vector<int> trunc;
    std::vector<uint8_t> spre, spost;                 /* launch scratch */
    size_t sbytes = 0;
    int strunc = 0;
};

}  // namespace

bool dump_wanted(const char* row) {
    const DumpConfig& c = config();
    if (!c.on) return false;
    for (const std::string& t : c.ops)
        if (strstr(row, t.c_str())) return true;
    return false;
}

void* dump_begin(const char* row, const RadArgs* a, RadStream s) {
    const DumpConfig& c = config();
    if (!a) return nullptr;
    int seq = 0;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        auto it = g_counts.begin();
        for (; it != g_counts.end() && it->first != row; ++it) {}
        if (it == g_counts.end()) {
            g_counts.emplace_back(row, 0);
            it = g_counts.end() - 1;
        }
        if (it->second >= c.per_row) return nullptr;
        seq = it->second++;
    }
    if (hipStreamSynchronize((hipStream_t)s) != hipSuccess) return nullptr;
    Capture* cp = new Capture();
    cp->row = row;
    cp->seq = seq;
    cp->pre.resize(a->n_t);
    cp->post.resize(a->n_t);
    cp->bytes.assign(a->n_t, 0);
    cp->trunc.assign(a->n_t, 0);
    for (int i = 0; i < a->n_t; ++i) {
        size_t nb = span_bytes(a->t[i]);
        if (nb > c.cap) { nb = c.cap; cp->trunc[i] = 1; }
        cp->bytes[i] = nb;
        if (!to_host(cp->pre[i], a->t[i].data, nb)) { delete cp; return nullptr; }
    }
    if (a->scratch && a->scratch_bytes > 0) {
        size_t nb = (size_t)a->scratch_bytes;
        if (nb > c.cap) { nb = c.cap; cp->strunc = 1; }
        cp->sbytes = nb;
        if (!to_host(cp->spre, a->scratch, nb)) { delete cp; return nullptr; }
    }
    return cp;
}

void dump_end(void* handle, const RadArgs* a, RadStream s, int rc) {
    Capture* cp = static_cast<Capture*>(handle);
    if (!cp) return;
    bool ok = true;
    if (rc == RAD_OK) {
        ok = hipStreamSynchronize((hipStream_t)s) == hipSuccess;
        for (int i = 0; ok && i < a->n_t; ++i) ok = to_host(cp->post[i], a->t[i].data, cp->bytes[i]);
        if (ok && cp->sbytes) ok = to_host(cp->spost, a->scratch, cp->sbytes);
    }
    if (!ok) {
        fprintf(stderr, "libr3d_gfx950: R3D_DUMP: post-state copy of %s failed\n", cp->row.c_str());
        delete cp;
        return;
    }
    char sub[64];
    snprintf(sub, sizeof sub, "/%04d_", cp->seq);
    const std::string dir = config().dir + sub + cp->row;
    make_dirs(dir);
    if (FILE* f = fopen((dir + "/manifest.tsv").c_str(), "w")) {
        fprintf(f, "H\t%s\t%d\t%d\t%d\n", cp->row.c_str(), rc, a->n_t, a->n_p);
        for (int i = 0; i < a->n_p; ++i) {
            const RadParam& p = a->p[i];
            fprintf(f, "P\t%d\t%s\t%lld\t%lld\t%s\t%.17g\n", p.kind, p.key ? p.key : "-", p.ival,
                    p.ihi, p.kind == RAD_P_STR && p.sval && *p.sval ? p.sval : "-", p.dval);
        }
        for (int i = 0; i < a->n_t; ++i) {
            const RadTensor& t = a->t[i];
            const uint32_t rank = t.data ? (t.rank < RAD_MAX_RANK ? t.rank : RAD_MAX_RANK) : 0;
            fprintf(f, "T\t%d\t%u\t%u", i, t.dtype, rank);
            for (uint32_t r = 0; r < rank; ++r) fprintf(f, "\t%lld", (long long)t.shape[r]);
            for (uint32_t r = 0; r < rank; ++r) fprintf(f, "\t%lld", (long long)t.stride[r]);
            fprintf(f, "\t%zu\t%d\t%d\t0x%llx\n", cp->bytes[i], cp->trunc[i], t.data == nullptr,
                    (unsigned long long)(uintptr_t)t.data);
        }
        for (int i = 0; a->tv && i < a->n_tv; ++i)
            fprintf(f, "V\t%s\t%lld\n", a->tv[i].name ? a->tv[i].name : "-", a->tv[i].value);
        if (a->scratch && a->scratch_bytes > 0)
            fprintf(f, "X\t%lld\t%zu\t%d\n", (long long)a->scratch_bytes, cp->sbytes, cp->strunc);
        fclose(f);
    }
    for (int pass = 0; pass < 2; ++pass) {
        if (pass == 1 && rc != RAD_OK) break;             /* a refused launch wrote nothing */
        FILE* g = fopen((dir + (pass ? "/post.bin" : "/pre.bin")).c_str(), "wb");
        if (!g) continue;
        for (int i = 0; i < a->n_t; ++i) {
            const std::vector<uint8_t>& v = pass ? cp->post[i] : cp->pre[i];
            if (!v.empty()) fwrite(v.data(), 1, v.size(), g);
        }
        const std::vector<uint8_t>& sv = pass ? cp->spost : cp->spre;
        if (!sv.empty()) fwrite(sv.data(), 1, sv.size(), g);
        fclose(g);
    }
    delete cp;
}

}  // namespace r3d
