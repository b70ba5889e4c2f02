// nexus_amd/csrc/kv_session.cpp -- the KV session formats of include/nexus_hip_kv.h
// (NXKVCACH, NXKVLYR1 of src/model/kvcache.h:352-551) read into and written from
// device-resident caches.
//
// Every call first computes the complete plan -- header fields, which layers carry data,
// the byte offset of every K/V block, the total size -- and checks it against the buffer
// or file and the device capacities; only then does it copy.  Each head's rows
// [0, n_tokens) are contiguous in the device layout [n_kv][row_stride][hd] and contiguous
// in the file, so every block is one DMA copy (memory forms) or a run of staged chunks
// (file forms).
#include "nexus_hip_kv.h"

#include <hip/hip_runtime.h>

#include <sys/stat.h>

#include <algorithm>
#include <climits>
#include <cstdio>
#include <cstring>
#include <vector>

#include "capi_status.h"

using nxa::capi_fail;
using nxa::capi_ok;

namespace {

constexpr char kCacheMagic[8] = {'N', 'X', 'K', 'V', 'C', 'A', 'C', 'H'};
constexpr char kLayerMagic[8] = {'N', 'X', 'K', 'V', 'L', 'Y', 'R', '1'};
constexpr size_t kHeaderBytes = 8 + 4 * sizeof(int32_t);
constexpr size_t kStageBytes = 16u << 20;              // per pinned staging buffer (file forms)

// One K or V block of one head: device rows [0, n_tokens) <-> file bytes at `off`.
struct Block {
    uint16_t* dev;                                     // nullptr: zeros on save
    size_t off;
    size_t bytes;
};

struct Plan {
    int32_t hdr[4];
    size_t total = 0;                                  // bytes the image occupies
    std::vector<Block> blocks;                         // in file order
};

size_t block_bytes(const nexus_kv_layer_view& v, int n_tokens)
{
    return (size_t)n_tokens * (size_t)v.head_dim * sizeof(uint16_t);
}

int check_view(const nexus_kv_layer_view& v, int l)
{
    if (v.n_kv_heads < 0) return capi_fail(NEXUS_E_INVALID, "layer %d: n_kv_heads=%d", l, v.n_kv_heads);
    if (v.n_kv_heads > 0 && v.head_dim <= 0) return capi_fail(NEXUS_E_INVALID, "layer %d: head_dim=%d", l, v.head_dim);
    if (v.row_stride < 0) return capi_fail(NEXUS_E_INVALID, "layer %d: row_stride=%lld", l, (long long)v.row_stride);
    return NEXUS_OK;
}

int check_views(const nexus_kv_layer_view* views, int n_layers)
{
    if (!views || n_layers <= 0) return capi_fail(NEXUS_E_INVALID, "views=%p n_layers=%d", (const void*)views, n_layers);
    for (int l = 0; l < n_layers; ++l) {
        const int rc = check_view(views[l], l);
        if (rc != NEXUS_OK) return rc;
    }
    return NEXUS_OK;
}

// Capacity and pointers of a layer that is going to receive n_tokens rows, or give them.
int check_rows(const nexus_kv_layer_view& v, int l, int n_tokens, bool load)
{
    if (v.n_kv_heads == 0) return NEXUS_OK;
    if ((int64_t)n_tokens > v.row_stride)
        return capi_fail(NEXUS_E_INVALID, "layer %d: %d tokens exceed row_stride=%lld", l, n_tokens,
                         (long long)v.row_stride);
    if (load && (!v.k || !v.v)) return capi_fail(NEXUS_E_INVALID, "layer %d: null k/v for a load", l);
    if (!load && (!v.k) != (!v.v)) return capi_fail(NEXUS_E_INVALID, "layer %d: only one of k/v is null", l);
    return NEXUS_OK;
}

// Header geometry of a cache image: the largest head count and head dim over the layers
// (KVCache::init_per_layer, kvcache.h:88-109; equal to the global geometry for a uniform cache).
void header_geometry(const nexus_kv_layer_view* views, int n_layers, int32_t* nh, int32_t* hd)
{
    *nh = 0;
    *hd = 0;
    for (int l = 0; l < n_layers; ++l) {
        *nh = std::max(*nh, views[l].n_kv_heads);
        *hd = std::max(*hd, views[l].head_dim);
    }
}

void add_layer_blocks(Plan& p, const nexus_kv_layer_view& v, int n_tokens, size_t& off)
{
    const size_t bb = block_bytes(v, n_tokens);
    for (int h = 0; h < v.n_kv_heads; ++h) {
        const size_t row0 = (size_t)h * (size_t)v.row_stride * (size_t)v.head_dim;
        p.blocks.push_back({v.k ? v.k + row0 : nullptr, off, bb});
        off += bb;
        p.blocks.push_back({v.v ? v.v + row0 : nullptr, off, bb});
        off += bb;
    }
}

// NXKVCACH as written (save_to_buffer, kvcache.h:427-449).
Plan cache_plan(const nexus_kv_layer_view* views, int n_layers, int n_tokens)
{
    Plan p;
    int32_t nh, hd;
    header_geometry(views, n_layers, &nh, &hd);
    p.hdr[0] = n_layers;
    p.hdr[1] = nh;
    p.hdr[2] = hd;
    p.hdr[3] = n_tokens;
    size_t off = kHeaderBytes;
    for (int l = 0; l < n_layers; ++l) add_layer_blocks(p, views[l], n_tokens, off);
    p.total = off;
    return p;
}

// expected_bytes (kvcache.h:455-463): the image size now, or in the legacy layout where
// every layer had the header geometry.
size_t expected_bytes(const nexus_kv_layer_view* views, int n_layers, int n_tokens, bool legacy, int32_t fh1,
                      int32_t fh2)
{
    size_t total = kHeaderBytes;
    for (int l = 0; l < n_layers; ++l) {
        const size_t hd = legacy ? (size_t)fh2 : (size_t)views[l].head_dim;
        const size_t nh = legacy ? (size_t)fh1 : (size_t)views[l].n_kv_heads;
        if (nh) total += nh * (size_t)n_tokens * hd * sizeof(uint16_t) * 2;
    }
    return total;
}

// NXKVCACH as read (load_from_buffer / load, kvcache.h:476-551) from a header and the image
// size; fails (status set) on a mismatch.
int cache_load_plan(const int32_t hdr[4], size_t image_bytes, const nexus_kv_layer_view* views, int n_layers,
                    Plan& p)
{
    int32_t nh, hd;
    header_geometry(views, n_layers, &nh, &hd);
    if (hdr[0] != n_layers || hdr[1] != nh || hdr[2] != hd)
        return capi_fail(NEXUS_E_INVALID, "model mismatch: file {%d layers, %d heads, dim %d}, cache {%d, %d, %d}",
                         hdr[0], hdr[1], hdr[2], n_layers, nh, hd);
    const int n_tokens = hdr[3];
    if (n_tokens < 0) return capi_fail(NEXUS_E_INVALID, "n_tokens=%d in the header", n_tokens);
    const size_t cur = expected_bytes(views, n_layers, n_tokens, false, nh, hd);
    const size_t old = expected_bytes(views, n_layers, n_tokens, true, nh, hd);
    const bool legacy = old != cur && image_bytes == old;            // is_legacy_layout (kvcache.h:464-469)
    if (!legacy && image_bytes < cur)
        return capi_fail(NEXUS_E_INVALID, "image of %zu bytes is shorter than the %zu its header implies",
                         image_bytes, cur);
    for (int l = 0; l < n_layers; ++l) {
        const int rc = check_rows(views[l], l, n_tokens, true);
        if (rc != NEXUS_OK) return rc;
    }
    p.hdr[0] = hdr[0];
    p.hdr[1] = hdr[1];
    p.hdr[2] = hdr[2];
    p.hdr[3] = hdr[3];
    size_t off = kHeaderBytes;
    for (int l = 0; l < n_layers; ++l) {
        if (legacy && views[l].n_kv_heads == 0) {
            off += (size_t)nh * (size_t)n_tokens * (size_t)hd * sizeof(uint16_t) * 2;   // zero blocks, skipped
            continue;
        }
        add_layer_blocks(p, views[l], n_tokens, off);
    }
    if (off > image_bytes)                               // a legacy image whose KV layers differ
        return capi_fail(NEXUS_E_INVALID, "image of %zu bytes is shorter than the %zu its layers need", image_bytes, off);
    p.total = off;
    return NEXUS_OK;
}

int copy_err(const char* what, hipError_t e)
{
    (void)hipGetLastError();
    return capi_fail(NEXUS_E_LAUNCH, "%s: %s", what, hipGetErrorString(e));
}

// Memory image <-> device, one DMA copy per block, then wait.
int run_blocks(const Plan& p, uint8_t* image, bool to_device, hipStream_t s)
{
    for (const Block& b : p.blocks) {
        if (b.bytes == 0) continue;
        hipError_t e;
        if (to_device) {
            e = hipMemcpyAsync(b.dev, image + b.off, b.bytes, hipMemcpyHostToDevice, s);
        } else if (b.dev) {
            e = hipMemcpyAsync(image + b.off, b.dev, b.bytes, hipMemcpyDeviceToHost, s);
        } else {
            std::memset(image + b.off, 0, b.bytes);
            continue;
        }
        if (e != hipSuccess) return copy_err("block copy", e);
    }
    const hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return copy_err("stream synchronize", e);
    return capi_ok();
}

void put_header(uint8_t* dst, const char magic[8], const int32_t hdr[4])
{
    std::memcpy(dst, magic, 8);
    std::memcpy(dst + 8, hdr, 4 * sizeof(int32_t));
}

// Two pinned buffers for the file forms.
struct Staging {
    void* buf[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool ok = false;
    Staging()
    {
        ok = hipHostMalloc(&buf[0], kStageBytes, hipHostMallocDefault) == hipSuccess &&
             hipHostMalloc(&buf[1], kStageBytes, hipHostMallocDefault) == hipSuccess &&
             hipEventCreateWithFlags(&ev[0], hipEventDisableTiming) == hipSuccess &&
             hipEventCreateWithFlags(&ev[1], hipEventDisableTiming) == hipSuccess;
        if (!ok) (void)hipGetLastError();
    }
    ~Staging()
    {
        for (int i = 0; i < 2; ++i) {
            if (ev[i]) {
                (void)hipEventSynchronize(ev[i]);
                (void)hipEventDestroy(ev[i]);
            }
            if (buf[i]) (void)hipHostFree(buf[i]);
        }
    }
};

// Device -> file: chunk c is copied into buffer c&1 while chunk c-1 is written out.
int stream_save(const Plan& p, FILE* f, hipStream_t s)
{
    Staging st;
    if (!st.ok) return capi_fail(NEXUS_E_LAUNCH, "pinned staging allocation failed");
    struct Pending {
        int slot;
        size_t bytes;
        bool zeros;
    };
    std::vector<uint8_t> zeros;
    int chunk = 0;
    bool have = false;
    Pending prev{0, 0, false};
    auto flush = [&](const Pending& q) -> int {
        if (q.zeros) {
            if (zeros.size() < q.bytes) zeros.assign(q.bytes, 0);
            if (fwrite(zeros.data(), 1, q.bytes, f) != q.bytes) return capi_fail(NEXUS_E_IO, "write failed");
            return NEXUS_OK;
        }
        const hipError_t e = hipEventSynchronize(st.ev[q.slot]);
        if (e != hipSuccess) return copy_err("staging wait", e);
        if (fwrite(st.buf[q.slot], 1, q.bytes, f) != q.bytes) return capi_fail(NEXUS_E_IO, "write failed");
        return NEXUS_OK;
    };
    for (const Block& b : p.blocks) {
        for (size_t done = 0; done < b.bytes;) {
            const size_t n = std::min(kStageBytes, b.bytes - done);
            Pending cur{chunk & 1, n, b.dev == nullptr};
            if (!cur.zeros) {
                // buffer cur.slot held chunk - 2, already written out during the previous chunk
                hipError_t e = hipMemcpyAsync(st.buf[cur.slot], (const uint8_t*)b.dev + done, n,
                                              hipMemcpyDeviceToHost, s);
                if (e == hipSuccess) e = hipEventRecord(st.ev[cur.slot], s);
                if (e != hipSuccess) return copy_err("staged copy", e);
            }
            if (have) {
                const int rc = flush(prev);
                if (rc != NEXUS_OK) return rc;
            }
            prev = cur;
            have = true;
            ++chunk;
            done += n;
        }
    }
    if (have) {
        const int rc = flush(prev);
        if (rc != NEXUS_OK) return rc;
    }
    return NEXUS_OK;
}

// File -> device: chunk c is read into buffer c&1 (after the copy out of it, two chunks
// back, has finished) while chunk c-1 is still on its way to the device.
int stream_load(const Plan& p, FILE* f, hipStream_t s)
{
    Staging st;
    if (!st.ok) return capi_fail(NEXUS_E_LAUNCH, "pinned staging allocation failed");
    int chunk = 0;
    size_t pos = kHeaderBytes;
    for (const Block& b : p.blocks) {
        if (pos != b.off) {                              // legacy zero blocks are skipped
            if (fseeko(f, (off_t)b.off, SEEK_SET) != 0) return capi_fail(NEXUS_E_IO, "seek failed");
            pos = b.off;
        }
        for (size_t done = 0; done < b.bytes;) {
            const size_t n = std::min(kStageBytes, b.bytes - done);
            const int slot = chunk & 1;
            hipError_t e = hipEventSynchronize(st.ev[slot]);
            if (e != hipSuccess) return copy_err("staging wait", e);
            if (fread(st.buf[slot], 1, n, f) != n) return capi_fail(NEXUS_E_IO, "read failed or file truncated");
            e = hipMemcpyAsync((uint8_t*)b.dev + done, st.buf[slot], n, hipMemcpyHostToDevice, s);
            if (e == hipSuccess) e = hipEventRecord(st.ev[slot], s);
            if (e != hipSuccess) return copy_err("staged copy", e);
            ++chunk;
            done += n;
            pos += n;
        }
    }
    const hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return copy_err("stream synchronize", e);
    return NEXUS_OK;
}

}  // namespace

extern "C" {

size_t nexus_hip_kv_layer_bytes(const nexus_kv_layer_view* view, int n_tokens)
{
    if (!view || n_tokens < 0 || check_view(*view, 0) != NEXUS_OK) return 0;
    if (view->n_kv_heads == 0) return 0;
    return kHeaderBytes + 2 * (size_t)view->n_kv_heads * block_bytes(*view, n_tokens);
}

size_t nexus_hip_kv_cache_bytes(const nexus_kv_layer_view* views, int n_layers, int n_tokens)
{
    if (n_tokens < 0 || check_views(views, n_layers) != NEXUS_OK) return 0;
    return cache_plan(views, n_layers, n_tokens).total;
}

int nexus_hip_kv_layer_save(int layer, const nexus_kv_layer_view* view, int n_tokens, void* buf, size_t buf_bytes,
                            nexus_stream_t stream)
{
    if (!view) return capi_fail(NEXUS_E_INVALID, "view is NULL");
    int rc = check_view(*view, layer);
    if (rc != NEXUS_OK) return rc;
    if (layer < 0 || n_tokens < 0) return capi_fail(NEXUS_E_INVALID, "layer=%d n_tokens=%d", layer, n_tokens);
    if (view->n_kv_heads == 0) return capi_ok();           // no KV: an empty record
    rc = check_rows(*view, layer, n_tokens, false);
    if (rc != NEXUS_OK) return rc;
    Plan p;
    p.hdr[0] = layer;
    p.hdr[1] = view->n_kv_heads;
    p.hdr[2] = view->head_dim;
    p.hdr[3] = n_tokens;
    size_t off = kHeaderBytes;
    add_layer_blocks(p, *view, n_tokens, off);
    p.total = off;
    if (!buf || buf_bytes < p.total)
        return capi_fail(NEXUS_E_INVALID, "buffer of %zu bytes, the record needs %zu", buf_bytes, p.total);
    put_header((uint8_t*)buf, kLayerMagic, p.hdr);
    return run_blocks(p, (uint8_t*)buf, false, (hipStream_t)stream);
}

int nexus_hip_kv_layer_load(const void* buf, size_t buf_bytes, const nexus_kv_layer_view* views, int n_layers,
                            int* layer_out, int* n_tokens_out, nexus_stream_t stream)
{
    int rc = check_views(views, n_layers);
    if (rc != NEXUS_OK) return rc;
    if (!buf || buf_bytes < kHeaderBytes || std::memcmp(buf, kLayerMagic, 8) != 0)
        return capi_fail(NEXUS_E_INVALID, "not an NXKVLYR1 record");
    int32_t hdr[4];
    std::memcpy(hdr, (const uint8_t*)buf + 8, sizeof(hdr));
    const int l = hdr[0];
    if (l < 0 || l >= n_layers) return capi_fail(NEXUS_E_INVALID, "record for layer %d of %d", l, n_layers);
    const nexus_kv_layer_view& v = views[l];
    if (hdr[1] != v.n_kv_heads || hdr[2] != v.head_dim)
        return capi_fail(NEXUS_E_INVALID, "layer %d geometry mismatch: record {%d heads, dim %d}, cache {%d, %d}", l,
                         hdr[1], hdr[2], v.n_kv_heads, v.head_dim);
    if (hdr[3] < 0) return capi_fail(NEXUS_E_INVALID, "n_tokens=%d in the record", hdr[3]);
    rc = check_rows(v, l, hdr[3], true);
    if (rc != NEXUS_OK) return rc;
    Plan p;
    size_t off = kHeaderBytes;
    add_layer_blocks(p, v, hdr[3], off);
    if (buf_bytes < off)
        return capi_fail(NEXUS_E_INVALID, "record of %zu bytes, its header implies %zu", buf_bytes, off);
    rc = run_blocks(p, (uint8_t*)buf, true, (hipStream_t)stream);
    if (rc != NEXUS_OK) return rc;
    if (layer_out) *layer_out = l;
    if (n_tokens_out) *n_tokens_out = hdr[3];
    return capi_ok();
}

int nexus_hip_kv_cache_save(const nexus_kv_layer_view* views, int n_layers, int n_tokens, void* buf, size_t buf_bytes,
                            nexus_stream_t stream)
{
    int rc = check_views(views, n_layers);
    if (rc != NEXUS_OK) return rc;
    if (n_tokens < 0) return capi_fail(NEXUS_E_INVALID, "n_tokens=%d", n_tokens);
    for (int l = 0; l < n_layers; ++l)
        if ((rc = check_rows(views[l], l, n_tokens, false)) != NEXUS_OK) return rc;
    const Plan p = cache_plan(views, n_layers, n_tokens);
    if (!buf || buf_bytes < p.total)
        return capi_fail(NEXUS_E_INVALID, "buffer of %zu bytes, the image needs %zu", buf_bytes, p.total);
    put_header((uint8_t*)buf, kCacheMagic, p.hdr);
    return run_blocks(p, (uint8_t*)buf, false, (hipStream_t)stream);
}

int nexus_hip_kv_cache_load(const void* buf, size_t buf_bytes, const nexus_kv_layer_view* views, int n_layers,
                            int* n_tokens_out, nexus_stream_t stream)
{
    int rc = check_views(views, n_layers);
    if (rc != NEXUS_OK) return rc;
    if (!buf || buf_bytes < kHeaderBytes || std::memcmp(buf, kCacheMagic, 8) != 0)
        return capi_fail(NEXUS_E_INVALID, "not an NXKVCACH image");
    int32_t hdr[4];
    std::memcpy(hdr, (const uint8_t*)buf + 8, sizeof(hdr));
    Plan p;
    if ((rc = cache_load_plan(hdr, buf_bytes, views, n_layers, p)) != NEXUS_OK) return rc;
    rc = run_blocks(p, (uint8_t*)buf, true, (hipStream_t)stream);
    if (rc != NEXUS_OK) return rc;
    if (n_tokens_out) *n_tokens_out = hdr[3];
    return capi_ok();
}

int nexus_hip_kv_cache_save_file(const char* path, const nexus_kv_layer_view* views, int n_layers, int n_tokens,
                                 nexus_stream_t stream)
{
    int rc = check_views(views, n_layers);
    if (rc != NEXUS_OK) return rc;
    if (!path) return capi_fail(NEXUS_E_INVALID, "path is NULL");
    if (n_tokens < 0) return capi_fail(NEXUS_E_INVALID, "n_tokens=%d", n_tokens);
    for (int l = 0; l < n_layers; ++l)
        if ((rc = check_rows(views[l], l, n_tokens, false)) != NEXUS_OK) return rc;
    const Plan p = cache_plan(views, n_layers, n_tokens);
    FILE* f = fopen(path, "wb");
    if (!f) return capi_fail(NEXUS_E_IO, "cannot open %s for writing", path);
    uint8_t head[kHeaderBytes];
    put_header(head, kCacheMagic, p.hdr);
    rc = fwrite(head, 1, kHeaderBytes, f) == kHeaderBytes ? stream_save(p, f, (hipStream_t)stream)
                                                          : capi_fail(NEXUS_E_IO, "write failed");
    if (fclose(f) != 0 && rc == NEXUS_OK) rc = capi_fail(NEXUS_E_IO, "close of %s failed", path);
    return rc == NEXUS_OK ? capi_ok() : rc;
}

int nexus_hip_kv_cache_load_file(const char* path, const nexus_kv_layer_view* views, int n_layers, int* n_tokens_out,
                                 nexus_stream_t stream)
{
    int rc = check_views(views, n_layers);
    if (rc != NEXUS_OK) return rc;
    if (!path) return capi_fail(NEXUS_E_INVALID, "path is NULL");
    FILE* f = fopen(path, "rb");
    if (!f) return capi_fail(NEXUS_E_IO, "cannot open %s", path);
    struct stat sb;
    char magic[8];
    int32_t hdr[4];
    Plan p;
    if (fstat(fileno(f), &sb) != 0) {
        rc = capi_fail(NEXUS_E_IO, "cannot stat %s", path);
    } else if (fread(magic, 1, 8, f) != 8 || std::memcmp(magic, kCacheMagic, 8) != 0) {
        rc = capi_fail(NEXUS_E_INVALID, "%s is not an NXKVCACH file", path);
    } else if (fread(hdr, sizeof(int32_t), 4, f) != 4) {
        rc = capi_fail(NEXUS_E_INVALID, "%s: header truncated", path);
    } else {
        rc = cache_load_plan(hdr, (size_t)sb.st_size, views, n_layers, p);
        if (rc == NEXUS_OK) rc = stream_load(p, f, (hipStream_t)stream);
    }
    fclose(f);
    if (rc != NEXUS_OK) return rc;
    if (n_tokens_out) *n_tokens_out = hdr[3];
    return capi_ok();
}

}  // extern "C"
