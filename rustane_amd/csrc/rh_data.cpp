// rh_data.cpp -- the on-disk formats on either side of the forward, behind
// include/rustane_hip.h:
//   * RSTK v1 checkpoints (crates/engine/src/bin/train.rs:238-345): a 28-byte
//     little-endian header then every tensor as fp32, in the order the
//     weight upload takes them;
//   * token files (crates/engine/src/data.rs:11-44): flat little-endian uint16
//     ids, memory-mapped; token_bytes (data.rs:46-71): int32 byte length per id;
//   * the validation loop (bin/train.rs:196-236) and compute_bpb
//     (data.rs:75-91), with the reference's f32 accumulation order.
// Checkpoint tensors are uploaded straight from the mapping (no host copy of
// a multi-GB file); saving streams one tensor at a time from the device.
#include "../../include/rustane_hip.h"
#include "rh_internal.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <vector>

namespace {

thread_local std::string t_err;

int fail_tls(int code, const std::string& m) {
    t_err = m;
    return code;
}

// A read-only mapping of a whole file (empty files map to nothing).
struct Mapped {
    const uint8_t* p = nullptr;
    size_t n = 0;
    int open(const char* path) {
        const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
        if (fd < 0) return fail_tls(RH_EIO, std::string("cannot open ") + path + ": " + std::strerror(errno));
        struct stat sb;
        if (fstat(fd, &sb) != 0) {
            ::close(fd);
            return fail_tls(RH_EIO, std::string("cannot stat ") + path);
        }
        n = (size_t)sb.st_size;
        if (n > 0) {
            void* m = mmap(nullptr, n, PROT_READ, MAP_PRIVATE, fd, 0);
            if (m == MAP_FAILED) {
                ::close(fd);
                return fail_tls(RH_EIO, std::string("cannot map ") + path + ": " + std::strerror(errno));
            }
            p = (const uint8_t*)m;
        }
        ::close(fd);
        return RH_OK;
    }
    ~Mapped() {
        if (p) munmap((void*)p, n);
    }
};

uint32_t le32(const uint8_t* b) { return (uint32_t)b[0] | (uint32_t)b[1] << 8 | (uint32_t)b[2] << 16 | (uint32_t)b[3] << 24; }
void put32(uint8_t* b, uint32_t v) {
    b[0] = (uint8_t)v; b[1] = (uint8_t)(v >> 8); b[2] = (uint8_t)(v >> 16); b[3] = (uint8_t)(v >> 24);
}

constexpr size_t RSTK_HEADER = 28;  // "RSTK" + 6 x u32 (train.rs:249-256, :300)

int parse_header(const Mapped& m, const char* path, rh_ckpt_info* out) {
    if (m.n < RSTK_HEADER || std::memcmp(m.p, "RSTK", 4) != 0)
        return fail_tls(RH_EIO, std::string(path) + ": not an RSTK checkpoint (bad magic or short header)");
    out->version = le32(m.p + 4);
    out->step = le32(m.p + 8);
    out->dim = le32(m.p + 12);
    out->nlayers = le32(m.p + 16);
    out->vocab = le32(m.p + 20);
    out->seq = le32(m.p + 24);
    out->file_bytes = m.n;
    return RH_OK;
}

// fp32 elements of every tensor, in file order, for an MHA config
// (q_dim = kv_dim = dim).
std::vector<size_t> tensor_sizes(const rh_config& c) {
    const size_t D = c.dim, F = c.hidden, V = c.vocab;
    std::vector<size_t> s{V * D, D};
    for (int l = 0; l < c.nlayers; ++l)
        for (size_t e : {D * D, D * D, D * D, D * D, D * F, D * F, D * F, D, D}) s.push_back(e);
    return s;
}

}  // namespace

const char* rh_internal_tls_error() { return t_err.c_str(); }

struct rh_tokens {
    Mapped map;
    int64_t n = 0;
};

extern "C" {

int rh_checkpoint_info(const char* path, rh_ckpt_info* out) {
    if (!path || !out) return fail_tls(RH_EINVAL, "null argument");
    Mapped m;
    int rc = m.open(path);
    if (rc) return rc;
    return parse_header(m, path, out);
}

int rh_load_checkpoint(rh_ctx* ctx, const char* path, uint32_t* step_out) {
    if (!ctx || !path) return rh_internal_fail(ctx, RH_EINVAL, "null argument");
    rh_config c;
    int max_batch = 0, max_ctx = 0;
    int rc = rh_context_info(ctx, &c, &max_batch, &max_ctx);
    if (rc) return rc;
    Mapped m;
    rh_ckpt_info h;
    if ((rc = m.open(path)) || (rc = parse_header(m, path, &h))) return rh_internal_fail(ctx, rc, t_err);
    // load_checkpoint takes hidden and heads from the model preset and the
    // shapes below from the file's header (train.rs:296-345)
    if (h.dim != (uint32_t)c.dim || h.nlayers != (uint32_t)c.nlayers || h.vocab != (uint32_t)c.vocab)
        return rh_internal_fail(ctx, RH_EINVAL,
                                std::string(path) + ": checkpoint is dim " + std::to_string(h.dim) + ", " +
                                    std::to_string(h.nlayers) + " layers, vocab " + std::to_string(h.vocab) +
                                    "; the context is dim " + std::to_string(c.dim) + ", " +
                                    std::to_string(c.nlayers) + " layers, vocab " + std::to_string(c.vocab));
    const std::vector<size_t> sz = tensor_sizes(c);
    size_t need = RSTK_HEADER;
    for (size_t e : sz) need += 4 * e;
    if (m.n != need)
        return rh_internal_fail(ctx, RH_EIO,
                                std::string(path) + ": " + std::to_string(m.n) + " bytes, expected " +
                                    std::to_string(need) + " for this config (hidden " +
                                    std::to_string(c.hidden) + ")");
    // fp32 tensors start at byte 28: 4-byte aligned in the page-aligned mapping
    std::vector<const float*> ptr(sz.size());
    size_t off = RSTK_HEADER;
    for (size_t i = 0; i < sz.size(); ++i) {
        ptr[i] = (const float*)(m.p + off);
        off += 4 * sz[i];
    }
    rc = rh_load_weights_f32(ctx, ptr[0], ptr[1], ptr.data() + 2);
    if (rc) return rc;
    if (step_out) *step_out = h.step;
    return RH_OK;
}

int rh_save_checkpoint(rh_ctx* ctx, const char* path, uint32_t step) {
    if (!ctx || !path) return rh_internal_fail(ctx, RH_EINVAL, "null argument");
    rh_config c;
    int max_batch = 0, max_ctx = 0;
    int rc = rh_context_info(ctx, &c, &max_batch, &max_ctx);
    if (rc) return rc;
    const std::vector<size_t> sz = tensor_sizes(c);
    size_t biggest = 0;
    for (size_t e : sz) biggest = e > biggest ? e : biggest;
    std::vector<float> buf;
    try {
        buf.resize(biggest);
    } catch (const std::bad_alloc&) {
        return rh_internal_fail(ctx, RH_ENOMEM, "host buffer for checkpoint tensors");
    }
    const std::string tmp = std::string(path) + ".tmp";
    FILE* f = std::fopen(tmp.c_str(), "wb");
    if (!f) return rh_internal_fail(ctx, RH_EIO, "cannot create " + tmp + ": " + std::strerror(errno));
    uint8_t hdr[RSTK_HEADER];
    std::memcpy(hdr, "RSTK", 4);
    put32(hdr + 4, 1);  // version
    put32(hdr + 8, step);
    put32(hdr + 12, (uint32_t)c.dim);
    put32(hdr + 16, (uint32_t)c.nlayers);
    put32(hdr + 20, (uint32_t)c.vocab);
    put32(hdr + 24, (uint32_t)c.seq);
    bool ok = std::fwrite(hdr, 1, RSTK_HEADER, f) == RSTK_HEADER;
    std::vector<float*> lt((size_t)9 * c.nlayers, nullptr);
    for (size_t i = 0; ok && i < sz.size(); ++i) {
        // one tensor per download: only its pointer is set
        if (i == 0) rc = rh_read_weights_f32(ctx, buf.data(), nullptr, nullptr);
        else if (i == 1) rc = rh_read_weights_f32(ctx, nullptr, buf.data(), nullptr);
        else {
            lt[i - 2] = buf.data();
            rc = rh_read_weights_f32(ctx, nullptr, nullptr, lt.data());
            lt[i - 2] = nullptr;
        }
        if (rc) break;
        // little-endian host: the fp32 bytes are the file bytes
        ok = std::fwrite(buf.data(), sizeof(float), sz[i], f) == sz[i];
    }
    ok = (std::fclose(f) == 0) && ok;
    if (rc || !ok) {
        std::remove(tmp.c_str());
        return rc ? rc : rh_internal_fail(ctx, RH_EIO, "write failed: " + tmp);
    }
    if (std::rename(tmp.c_str(), path) != 0) {
        std::remove(tmp.c_str());
        return rh_internal_fail(ctx, RH_EIO, std::string("cannot rename to ") + path);
    }
    return RH_OK;
}

int rh_tokens_open(const char* path, rh_tokens** out) {
    if (!path || !out) return fail_tls(RH_EINVAL, "null argument");
    *out = nullptr;
    rh_tokens* t = new (std::nothrow) rh_tokens;
    if (!t) return fail_tls(RH_ENOMEM, "out of host memory");
    const int rc = t->map.open(path);
    if (rc) {
        delete t;
        return rc;
    }
    t->n = (int64_t)(t->map.n / 2);  // a trailing odd byte is ignored (data.rs:23)
    *out = t;
    return RH_OK;
}

void rh_tokens_close(rh_tokens* t) { delete t; }

int64_t rh_tokens_len(const rh_tokens* t) { return t ? t->n : 0; }

int rh_tokens_read(const rh_tokens* t, int64_t start, int len, uint32_t* out) {
    if (!t || (!out && len > 0) || len < 0 || start < 0) return fail_tls(RH_EINVAL, "bad argument");
    if (start + len > t->n)
        return fail_tls(RH_ERANGE, "token range [" + std::to_string(start) + ", " + std::to_string(start + len) +
                                       ") past the file's " + std::to_string(t->n) + " tokens");
    const uint8_t* b = t->map.p + 2 * start;
    for (int i = 0; i < len; ++i) out[i] = (uint32_t)b[2 * i] | (uint32_t)b[2 * i + 1] << 8;
    return RH_OK;
}

int rh_compute_bpb(const float* losses, const uint32_t* targets, int64_t n, const int32_t* token_bytes,
                   int vocab, float* bpb_out, float* total_nats_out, int64_t* total_bytes_out) {
    if ((n > 0 && (!losses || !targets)) || !token_bytes || vocab <= 0 || n < 0)
        return fail_tls(RH_EINVAL, "bad argument");
    float nats = 0.0f;
    int64_t bytes = 0;
    for (int64_t i = 0; i < n; ++i) {
        if (targets[i] >= (uint32_t)vocab) return fail_tls(RH_ERANGE, "target id >= vocab");
        const int32_t bl = token_bytes[targets[i]];
        if (bl > 0) {
            nats += losses[i];
            bytes += bl;
        }
    }
    const float ln2 = 0.693147180559945309f;
    if (bpb_out) *bpb_out = bytes > 0 ? nats / (ln2 * (float)bytes) : 0.0f;
    if (total_nats_out) *total_nats_out = nats;
    if (total_bytes_out) *total_bytes_out = bytes;
    return RH_OK;
}

int rh_validate(rh_ctx* ctx, const rh_tokens* val, const int32_t* token_bytes, int steps, float* avg_loss_out,
                float* bpb_out) {
    if (!ctx || !val || steps <= 0) return rh_internal_fail(ctx, RH_EINVAL, "bad argument");
    rh_config c;
    int max_batch = 0, max_ctx = 0;
    int rc = rh_context_info(ctx, &c, &max_batch, &max_ctx);
    if (rc) return rc;
    const int S = c.seq;
    if (val->n < (int64_t)S + 2)
        return rh_internal_fail(ctx, RH_ERANGE, "validation file shorter than seq + 2 tokens");
    const int64_t max_pos = val->n - S - 1;
    const int B = max_batch;
    std::vector<uint32_t> tok((size_t)B * S), tgt((size_t)B * (S + 1));
    std::vector<float> losses((size_t)B * S);
    std::vector<float> all_losses;
    std::vector<uint32_t> all_targets;
    if (token_bytes) {
        all_losses.reserve((size_t)steps * S);
        all_targets.reserve((size_t)steps * S);
    }
    float total_loss = 0.0f;
    int64_t total_tokens = 0;
    for (int v0 = 0; v0 < steps; v0 += B) {
        const int nb = steps - v0 < B ? steps - v0 : B;
        for (int b = 0; b < nb; ++b) {
            const int64_t pos = ((int64_t)(v0 + b) * S) % max_pos;
            // input = tokens(pos, seq), target = tokens(pos + 1, seq): one read of seq + 1
            if ((rc = rh_tokens_read(val, pos, S + 1, &tgt[(size_t)b * (S + 1)])))
                return rh_internal_fail(ctx, rc, t_err);
            std::memcpy(&tok[(size_t)b * S], &tgt[(size_t)b * (S + 1)], (size_t)S * sizeof(uint32_t));
            std::memmove(&tgt[(size_t)b * S], &tgt[(size_t)b * (S + 1) + 1], (size_t)S * sizeof(uint32_t));
        }
        // compact targets: row b now sits at [b*S, (b+1)*S) (rows are moved in order)
        if ((rc = rh_forward(ctx, tok.data(), tgt.data(), nb, S, nullptr, losses.data(), nullptr))) return rc;
        for (int b = 0; b < nb; ++b) {
            float s = 0.0f;  // losses.iter().sum::<f32>() of one window
            for (int i = 0; i < S; ++i) s += losses[(size_t)b * S + i];
            total_loss += s;
            total_tokens += S;
            if (token_bytes) {
                all_losses.insert(all_losses.end(), &losses[(size_t)b * S], &losses[(size_t)(b + 1) * S]);
                all_targets.insert(all_targets.end(), &tgt[(size_t)b * S], &tgt[(size_t)(b + 1) * S]);
            }
        }
    }
    if (avg_loss_out) *avg_loss_out = total_loss / (float)total_tokens;
    if (bpb_out) {
        *bpb_out = 0.0f;
        if (token_bytes &&
            (rc = rh_compute_bpb(all_losses.data(), all_targets.data(), (int64_t)all_losses.size(), token_bytes,
                                 c.vocab, bpb_out, nullptr, nullptr)))
            return rh_internal_fail(ctx, rc, t_err);
    }
    return RH_OK;
}

}  // extern "C"
