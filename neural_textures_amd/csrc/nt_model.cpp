// nt_model.cpp — the model container: nt_model_bytes / nt_model_save / nt_model_load.
//
// The reference keeps trained latents and weights only in device memory and writes PNG
// renders (main.cpp:855-904); this file image is what carries a trained (or half-trained)
// neural texture between processes. Host code only: it formats and checks host buffers.
//
// Image layout (little-endian):
//   [0, 64)        Header
//   [64, 192)      description: 32 int32 (contents, num_grids, channels, width[4],
//                  height[4], num_mips[4], num_layers, sizes[7], used_outputs, step, 0...)
//   [192, ...)     section table, one 32-byte Entry per section, in the fixed order
//                  plan_sections() gives
//   data           sections at 256-byte aligned offsets, zero padding between them
// Checksums are CRC-32C (Castagnoli): one per section, one over description + table.
#include <cstring>

#include "nt_internal.hpp"

static_assert(__BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__, "the model image is little-endian");

namespace {

constexpr char kMagic[8] = {'N', 'T', 'M', 'O', 'D', 'E', 'L', '\0'};
constexpr int kDescInts = 32;
constexpr uint64_t kSectionAlign = 256;
constexpr int kMaxSections = NT_MAX_GRIDS * 7 + NT_MAX_LAYERS * 6;
constexpr int kMaxSize = 1024;     // network widths
constexpr int kMaxExtent = 1 << 16; // grid widths / heights

enum Section : uint32_t {
    kCodec = 1,
    kWeights = 2,
    kBiases = 3,
    kLatents = 4,
    kLatentM1 = 5,
    kLatentM2 = 6,
    kWeightM1 = 7,
    kWeightM2 = 8,
    kBiasM1 = 9,
    kBiasM2 = 10,
    kBlocks = 11,
    kBlockM1 = 12,
    kBlockM2 = 13,
};

const char *section_name(uint32_t t)
{
    static const char *names[] = {"?",              "codec",         "weights",        "biases",
                                  "latents",        "latent_moment1", "latent_moment2", "weight_moment1",
                                  "weight_moment2", "bias_moment1",  "bias_moment2",   "block_params",
                                  "block_moment1",  "block_moment2"};
    return t <= kBlockM2 ? names[t] : "?";
}

struct Header {
    char magic[8];
    uint32_t version;
    uint32_t header_bytes;
    uint32_t num_sections;
    uint32_t contents;
    uint64_t image_bytes;
    uint32_t meta_crc; // over the description and the section table
    uint32_t reserved[7];
};
static_assert(sizeof(Header) == 64, "header is 64 bytes");

struct Entry {
    uint32_t type, index;
    uint64_t offset, bytes;
    uint32_t crc, reserved;
};
static_assert(sizeof(Entry) == 32, "section entry is 32 bytes");

constexpr uint64_t kDescOff = sizeof(Header);
constexpr uint64_t kTableOff = kDescOff + kDescInts * 4;

// CRC-32C, reflected polynomial 0x82F63B78, eight bytes per step through eight tables
// (table k = the CRC of a byte followed by k zero bytes). Check value of "123456789":
// 0xE3069283.
struct Crc32c {
    uint32_t t[8][256];
    Crc32c()
    {
        for (uint32_t i = 0; i < 256; ++i) {
            uint32_t c = i;
            for (int k = 0; k < 8; ++k)
                c = (c >> 1) ^ (0x82F63B78u & (0u - (c & 1u)));
            t[0][i] = c;
        }
        for (uint32_t i = 0; i < 256; ++i)
            for (int k = 1; k < 8; ++k)
                t[k][i] = (t[k - 1][i] >> 8) ^ t[0][t[k - 1][i] & 0xffu];
    }
    uint32_t update(uint32_t crc, const void *data, size_t n) const
    {
        const uint8_t *p = (const uint8_t *)data;
        crc = ~crc;
        while (n && ((uintptr_t)p & 7u)) {
            crc = (crc >> 8) ^ t[0][(crc ^ *p++) & 0xffu];
            --n;
        }
        for (; n >= 8; n -= 8, p += 8) {
            uint64_t v;
            std::memcpy(&v, p, 8);
            v ^= crc;
            crc = t[7][v & 0xffu] ^ t[6][(v >> 8) & 0xffu] ^ t[5][(v >> 16) & 0xffu] ^
                  t[4][(v >> 24) & 0xffu] ^ t[3][(v >> 32) & 0xffu] ^ t[2][(v >> 40) & 0xffu] ^
                  t[1][(v >> 48) & 0xffu] ^ t[0][v >> 56];
        }
        while (n--)
            crc = (crc >> 8) ^ t[0][(crc ^ *p++) & 0xffu];
        return ~crc;
    }
};

uint32_t crc32c(const void *data, size_t n, uint32_t crc = 0)
{
    static const Crc32c tables;
    return tables.update(crc, data, n);
}

uint64_t align_up(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }
uint64_t pad16(int x) { return (uint64_t)((x + 15) / 16 * 16); }

uint64_t chain_blocks(int w, int h, int mips)
{
    uint64_t n = 0;
    for (int m = 0; m < mips; ++m) {
        const int wm = (w >> m) > 0 ? (w >> m) : 1, hm = (h >> m) > 0 ? (h >> m) : 1;
        n += (uint64_t)((wm >> 2) > 0 ? (wm >> 2) : 1) * (uint64_t)((hm >> 2) > 0 ? (hm >> 2) : 1);
    }
    return n;
}

uint64_t chain_texels(int w, int h, int mips)
{
    uint64_t n = 0;
    for (int m = 0; m < mips; ++m) {
        const uint64_t wm = (w >> m) > 0 ? (uint64_t)(w >> m) : 1u;
        const uint64_t hm = (h >> m) > 0 ? (uint64_t)(h >> m) : 1u;
        n += wm * hm;
    }
    return n;
}

void pack_info(const nt_model_info &m, int32_t (&d)[kDescInts])
{
    std::memset(d, 0, sizeof(d));
    int k = 0;
    d[k++] = (int32_t)m.contents;
    d[k++] = m.num_grids;
    d[k++] = m.channels;
    for (int g = 0; g < NT_MAX_GRIDS; ++g)
        d[k++] = g < m.num_grids ? m.width[g] : 0;
    for (int g = 0; g < NT_MAX_GRIDS; ++g)
        d[k++] = g < m.num_grids ? m.height[g] : 0;
    for (int g = 0; g < NT_MAX_GRIDS; ++g)
        d[k++] = g < m.num_grids ? m.num_mips[g] : 0;
    d[k++] = m.num_layers;
    for (int l = 0; l <= NT_MAX_LAYERS; ++l)
        d[k++] = l <= m.num_layers ? m.sizes[l] : 0;
    d[k++] = m.used_outputs;
    d[k++] = m.step;
}

void unpack_info(const int32_t (&d)[kDescInts], nt_model_info *m)
{
    std::memset(m, 0, sizeof(*m));
    int k = 0;
    m->contents = (uint32_t)d[k++];
    m->num_grids = d[k++];
    m->channels = d[k++];
    for (int g = 0; g < NT_MAX_GRIDS; ++g)
        m->width[g] = d[k++];
    for (int g = 0; g < NT_MAX_GRIDS; ++g)
        m->height[g] = d[k++];
    for (int g = 0; g < NT_MAX_GRIDS; ++g)
        m->num_mips[g] = d[k++];
    m->num_layers = d[k++];
    for (int l = 0; l <= NT_MAX_LAYERS; ++l)
        m->sizes[l] = d[k++];
    m->used_outputs = d[k++];
    m->step = d[k++];
}

int check_info(const nt_model_info &m, int status)
{
    const uint32_t all = NT_MODEL_CODEC | NT_MODEL_STATE | NT_MODEL_BLOCKS;
    if (!(m.contents & (NT_MODEL_CODEC | NT_MODEL_STATE)) || (m.contents & ~all))
        return ntk::report(status, "contents 0x%x (need NT_MODEL_CODEC and/or NT_MODEL_STATE)", m.contents);
    if ((m.contents & NT_MODEL_BLOCKS) && !(m.contents & NT_MODEL_STATE))
        return ntk::report(status, "NT_MODEL_BLOCKS needs NT_MODEL_STATE");
    if (m.num_grids < 1 || m.num_grids > NT_MAX_GRIDS)
        return ntk::report(status, "num_grids %d (1..%d)", m.num_grids, NT_MAX_GRIDS);
    if (m.channels < 1 || m.channels > 16)
        return ntk::report(status, "channels %d (1..16)", m.channels);
    if ((m.contents & NT_MODEL_CODEC) && !nt_codec_block_bytes(m.channels))
        return ntk::report(status, "channels %d: the codec needs 4, 8, 12 or 16", m.channels);
    for (int g = 0; g < m.num_grids; ++g) {
        if (m.width[g] < 1 || m.width[g] > kMaxExtent || m.height[g] < 1 || m.height[g] > kMaxExtent)
            return ntk::report(status, "grid %d size %dx%d (1..%d)", g, m.width[g], m.height[g], kMaxExtent);
        if (m.num_mips[g] < 1 || m.num_mips[g] > NT_MAX_MIPS)
            return ntk::report(status, "grid %d num_mips %d (1..%d)", g, m.num_mips[g], NT_MAX_MIPS);
        if ((m.contents & NT_MODEL_BLOCKS) && (((m.width[g] & 3) && m.width[g] > 4) || ((m.height[g] & 3) && m.height[g] > 4)))
            return ntk::report(status, "grid %d: block records need sizes multiple of 4", g);
    }
    if (m.num_layers < 1 || m.num_layers > NT_MAX_LAYERS)
        return ntk::report(status, "num_layers %d (1..%d)", m.num_layers, NT_MAX_LAYERS);
    for (int l = 0; l <= m.num_layers; ++l)
        if (m.sizes[l] < 1 || m.sizes[l] > kMaxSize)
            return ntk::report(status, "sizes[%d] = %d (1..%d)", l, m.sizes[l], kMaxSize);
    if (m.used_outputs < 1 || m.used_outputs > m.sizes[m.num_layers])
        return ntk::report(status, "used_outputs %d (1..%d)", m.used_outputs, m.sizes[m.num_layers]);
    if (m.step < 0 || (m.step && !(m.contents & NT_MODEL_STATE)))
        return ntk::report(status, "step %d (0 without NT_MODEL_STATE)", m.step);
    return NT_OK;
}

struct Plan {
    int n = 0;
    Entry e[kMaxSections];
    uint64_t total = 0;
};

// The sections of a model in image order, with offsets and sizes.
void plan_sections(const nt_model_info &m, Plan *p)
{
    p->n = 0;
    auto add = [&](uint32_t type, int index, uint64_t bytes) {
        Entry &e = p->e[p->n++];
        std::memset(&e, 0, sizeof(e));
        e.type = type;
        e.index = (uint32_t)index;
        e.bytes = bytes;
    };
    if (m.contents & NT_MODEL_CODEC)
        for (int g = 0; g < m.num_grids; ++g) {
            int64_t off[NT_MAX_MIPS];
            add(kCodec, g, nt_codec_mip_chain_layout(m.width[g], m.height[g], m.num_mips[g], m.channels, off));
        }
    for (int l = 0; l < m.num_layers; ++l) {
        add(kWeights, l, pad16(m.sizes[l]) * pad16(m.sizes[l + 1]) * 2);
        add(kBiases, l, (uint64_t)m.sizes[l + 1] * 2);
    }
    if (m.contents & NT_MODEL_STATE) {
        for (int g = 0; g < m.num_grids; ++g) {
            const uint64_t b = chain_texels(m.width[g], m.height[g], m.num_mips[g]) * m.channels * 4;
            add(kLatents, g, b);
            add(kLatentM1, g, b);
            add(kLatentM2, g, b);
        }
        for (int l = 0; l < m.num_layers; ++l) {
            const uint64_t wb = pad16(m.sizes[l]) * pad16(m.sizes[l + 1]) * 4, bb = (uint64_t)m.sizes[l + 1] * 4;
            add(kWeightM1, l, wb);
            add(kWeightM2, l, wb);
            add(kBiasM1, l, bb);
            add(kBiasM2, l, bb);
        }
    }
    if (m.contents & NT_MODEL_BLOCKS)
        for (int g = 0; g < m.num_grids; ++g) {
            const uint64_t nb = chain_blocks(m.width[g], m.height[g], m.num_mips[g]);
            add(kBlocks, g, nb * (4 * m.channels + 18) * 4);
            add(kBlockM1, g, nb * (4 * m.channels + 16) * 4);
            add(kBlockM2, g, nb * (4 * m.channels + 16) * 4);
        }
    uint64_t off = align_up(kTableOff + (uint64_t)p->n * sizeof(Entry), kSectionAlign);
    for (int i = 0; i < p->n; ++i) {
        p->e[i].offset = off;
        off = align_up(off + p->e[i].bytes, kSectionAlign);
    }
    p->total = p->n ? p->e[p->n - 1].offset + p->e[p->n - 1].bytes : off;
}

// The data field of section (type, index).
const void **slot(nt_model_data *d, uint32_t type, uint32_t i)
{
    switch (type) {
    case kCodec:
        return &d->codec[i];
    case kWeights:
        return (const void **)&d->weights[i];
    case kBiases:
        return (const void **)&d->biases[i];
    case kLatents:
        return (const void **)&d->latents[i];
    case kLatentM1:
        return (const void **)&d->latent_moment1[i];
    case kLatentM2:
        return (const void **)&d->latent_moment2[i];
    case kWeightM1:
        return (const void **)&d->weight_moment1[i];
    case kWeightM2:
        return (const void **)&d->weight_moment2[i];
    case kBiasM1:
        return (const void **)&d->bias_moment1[i];
    case kBiasM2:
        return (const void **)&d->bias_moment2[i];
    case kBlocks:
        return (const void **)&d->block_params[i];
    case kBlockM1:
        return (const void **)&d->block_moment1[i];
    default:
        return (const void **)&d->block_moment2[i];
    }
}

} // namespace

extern "C" {

size_t nt_model_bytes(const nt_model_info *info)
{
    if (!info) {
        ntk::report(NT_ERR_NULL_POINTER, "info is NULL");
        return 0;
    }
    if (check_info(*info, NT_ERR_INVALID_ARGUMENT))
        return 0;
    Plan p;
    plan_sections(*info, &p);
    ntk::report(NT_OK, "");
    return (size_t)p.total;
}

int nt_model_save(const nt_model_info *info, const nt_model_data *data, void *out, size_t out_bytes)
{
    if (!info || !data || !out)
        return ntk::report(NT_ERR_NULL_POINTER, "info/data/out is NULL");
    if ((uintptr_t)out & 15u)
        return ntk::report(NT_ERR_MISALIGNED, "out must be 16-byte aligned");
    if (int st = check_info(*info, NT_ERR_INVALID_ARGUMENT))
        return st;
    Plan p;
    plan_sections(*info, &p);
    if (out_bytes < p.total)
        return ntk::report(NT_ERR_INVALID_ARGUMENT, "out_bytes %zu < image bytes %llu", out_bytes,
                           (unsigned long long)p.total);
    nt_model_data src = *data;
    for (int i = 0; i < p.n; ++i)
        if (!*slot(&src, p.e[i].type, p.e[i].index))
            return ntk::report(NT_ERR_NULL_POINTER, "data->%s[%u] is NULL", section_name(p.e[i].type),
                               p.e[i].index);

    uint8_t *img = (uint8_t *)out;
    uint64_t prev_end = kTableOff + (uint64_t)p.n * sizeof(Entry);
    for (int i = 0; i < p.n; ++i) {
        Entry &e = p.e[i];
        std::memset(img + prev_end, 0, e.offset - prev_end);
        const void *s = *slot(&src, e.type, e.index);
        std::memcpy(img + e.offset, s, e.bytes);
        e.crc = crc32c(img + e.offset, e.bytes);
        prev_end = e.offset + e.bytes;
    }
    int32_t desc[kDescInts];
    pack_info(*info, desc);
    std::memcpy(img + kDescOff, desc, sizeof(desc));
    std::memcpy(img + kTableOff, p.e, (size_t)p.n * sizeof(Entry));

    Header h;
    std::memset(&h, 0, sizeof(h));
    std::memcpy(h.magic, kMagic, sizeof(kMagic));
    h.version = NT_MODEL_VERSION;
    h.header_bytes = sizeof(Header);
    h.num_sections = (uint32_t)p.n;
    h.contents = info->contents;
    h.image_bytes = p.total;
    h.meta_crc = crc32c(img + kDescOff, (size_t)(kTableOff - kDescOff) + (size_t)p.n * sizeof(Entry));
    std::memcpy(img, &h, sizeof(h));
    return ntk::report(NT_OK, "");
}

int nt_model_load(const void *in, size_t in_bytes, nt_model_info *info, nt_model_data *data)
{
    if (!in || !info || !data)
        return ntk::report(NT_ERR_NULL_POINTER, "in/info/data is NULL");
    if ((uintptr_t)in & 15u)
        return ntk::report(NT_ERR_MISALIGNED, "in must be 16-byte aligned");
    const uint8_t *img = (const uint8_t *)in;
    if (in_bytes < kTableOff)
        return ntk::report(NT_ERR_FORMAT, "%zu bytes: shorter than a header", in_bytes);
    Header h;
    std::memcpy(&h, img, sizeof(h));
    if (std::memcmp(h.magic, kMagic, sizeof(kMagic)))
        return ntk::report(NT_ERR_FORMAT, "not a model image (magic)");
    if (h.version != NT_MODEL_VERSION)
        return ntk::report(NT_ERR_FORMAT, "image version %u; this library reads version %d", h.version,
                           NT_MODEL_VERSION);
    if (h.header_bytes != sizeof(Header) || h.num_sections > (uint32_t)kMaxSections)
        return ntk::report(NT_ERR_FORMAT, "header bytes %u, %u sections", h.header_bytes, h.num_sections);
    for (uint32_t r : h.reserved)
        if (r)
            return ntk::report(NT_ERR_FORMAT, "reserved header fields are set");
    const uint64_t meta_end = kTableOff + (uint64_t)h.num_sections * sizeof(Entry);
    if (in_bytes < meta_end || in_bytes < h.image_bytes)
        return ntk::report(NT_ERR_FORMAT, "truncated: %zu bytes, the image has %llu", in_bytes,
                           (unsigned long long)(h.image_bytes > meta_end ? h.image_bytes : meta_end));
    if (crc32c(img + kDescOff, (size_t)(meta_end - kDescOff)) != h.meta_crc)
        return ntk::report(NT_ERR_FORMAT, "description / section table checksum mismatch");

    int32_t desc[kDescInts], again[kDescInts];
    std::memcpy(desc, img + kDescOff, sizeof(desc));
    nt_model_info m;
    unpack_info(desc, &m);
    if (int st = check_info(m, NT_ERR_FORMAT))
        return st;
    pack_info(m, again);
    if (std::memcmp(desc, again, sizeof(desc)) || m.contents != h.contents)
        return ntk::report(NT_ERR_FORMAT, "description has fields set beyond its grids / layers");

    Plan p;
    plan_sections(m, &p);
    if ((uint32_t)p.n != h.num_sections || p.total != h.image_bytes)
        return ntk::report(NT_ERR_FORMAT, "%u sections / %llu bytes; the description implies %d / %llu",
                           h.num_sections, (unsigned long long)h.image_bytes, p.n,
                           (unsigned long long)p.total);
    nt_model_data d;
    std::memset(&d, 0, sizeof(d));
    for (int i = 0; i < p.n; ++i) {
        Entry e;
        std::memcpy(&e, img + kTableOff + (uint64_t)i * sizeof(Entry), sizeof(e));
        const Entry &want = p.e[i];
        if (e.type != want.type || e.index != want.index || e.offset != want.offset || e.bytes != want.bytes ||
            e.reserved)
            return ntk::report(NT_ERR_FORMAT, "section %d is %s[%u] at %llu (%llu bytes); expected %s[%u] at %llu (%llu)",
                               i, section_name(e.type), e.index, (unsigned long long)e.offset,
                               (unsigned long long)e.bytes, section_name(want.type), want.index,
                               (unsigned long long)want.offset, (unsigned long long)want.bytes);
        if (crc32c(img + e.offset, e.bytes) != e.crc)
            return ntk::report(NT_ERR_FORMAT, "section %s[%u] checksum mismatch", section_name(e.type), e.index);
        *slot(&d, e.type, e.index) = img + e.offset;
    }
    *info = m;
    *data = d;
    return ntk::report(NT_OK, "");
}

} // extern "C"
