// nt_api.cpp — the extern "C" boundary declared in include/nt/nt.h.
//
// Every entry point validates its arguments completely before enqueueing anything, turns
// the caller's structs into compact kernel descriptors and dispatches to a gfx950 kernel
// instantiated for the network shape. Nothing here allocates device memory.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "nt_internal.hpp"

using namespace ntk;

namespace {

thread_local char g_error[512] = "";
// Test hooks (nt_set_test_hooks): process-wide, read once per train step plan.
std::atomic<int> g_hook_max_workgroups{0};
std::atomic<int> g_hook_no_margins{0};
std::atomic<int> g_hook_sort_random{0};
thread_local hipEvent_t g_prof_start = nullptr;
thread_local hipEvent_t g_prof_stop = nullptr;

// Brackets one kernel launch with the one-shot profiling events, if set.
struct ProfileScope {
    hipStream_t s;
    hipEvent_t stop;
    explicit ProfileScope(hipStream_t stream) : s(stream), stop(g_prof_stop)
    {
        if (g_prof_start && g_prof_stop)
            hipEventRecord(g_prof_start, s);
        else
            stop = nullptr;
        g_prof_start = g_prof_stop = nullptr;
    }
    ~ProfileScope()
    {
        if (stop)
            hipEventRecord(stop, s);
    }
};

int fail(int status, const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return status;
}

int ok()
{
    g_error[0] = '\0';
    return NT_OK;
}

int hip_status(hipError_t e, const char *what)
{
    if (e != hipSuccess)
        return fail(NT_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return ok();
}

constexpr int pad16(int x) { return (x + 15) & ~15; }

// Compute units of the current device (256 on MI355X; also when no device is visible).
int device_cu_count()
{
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return 256;
    }
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) {
            (void)hipGetLastError();
            n = 256;
        }
        cached[dev] = n;
    }
    return cached[dev];
}

int mip_dim_h(int size, int mip)
{
    int d = size >> mip;
    return d > 0 ? d : 1;
}

// Shape of the MLP -> kernel instantiation (see ShapeId). Returns -1 if none is built.
int mlp_shape(const nt_mlp *m)
{
    const int L = m->num_layers;
    if (L < 2 || L > NT_MAX_LAYERS)
        return -1;
    for (int l = 0; l <= L; ++l)
        if (m->sizes[l] < 1)
            return -1;
    if (m->sizes[L] > NT_MAX_OUTPUTS)
        return -1;
    const int k0 = pad16(m->sizes[0]);
    const int h = pad16(m->sizes[1]);
    for (int l = 1; l < L; ++l)
        if (pad16(m->sizes[l]) != h)
            return -1;
    const int nh = L - 1;
    if (k0 == 16 && h == 32 && nh == 2)
        return kShapeRef;
    if (k0 == 16 && h == 16 && nh == 1)
        return kShapeFpt;
    if (k0 == 16 && h == 64 && nh == 2)
        return kShapeC1;
    if (k0 == 32 && h == 64 && nh == 2)
        return kShapeC2;
    if (k0 == 64 && h == 64 && nh == 3)
        return kShapeC4;
    return -1;
}

int shape_channels(int shape)
{
    switch (shape) {
    case kShapeRef:
        return 3;
    case kShapeC1:
        return 8;
    case kShapeC2:
    case kShapeC4:
        return 16;
    default:
        return 0;
    }
}

const char *shape_list()
{
    return "12(16)->32->32->16 C=3; 12(16)->16->16; 8(16)->64->64->16 C=8; 32->64->64->16 C=16; "
           "64->64->64->64->16 C=16";
}

int check_mlp(const nt_mlp *m, bool need_grads, bool need_moments, int *shape)
{
    if (!m)
        return fail(NT_ERR_NULL_POINTER, "mlp is NULL");
    *shape = mlp_shape(m);
    if (*shape < 0)
        return fail(NT_ERR_UNSUPPORTED, "no kernel is built for this MLP shape (built: %s)", shape_list());
    if (m->used_outputs < 0 || m->used_outputs > m->sizes[m->num_layers])
        return fail(NT_ERR_INVALID_ARGUMENT, "used_outputs %d outside [0, %d]", m->used_outputs,
                    m->sizes[m->num_layers]);
    for (int l = 0; l < m->num_layers; ++l) {
        if (!m->weights[l] || !m->biases[l])
            return fail(NT_ERR_NULL_POINTER, "layer %d weights/biases are NULL", l);
        if (need_grads && (!m->weight_grads[l] || !m->bias_grads[l]))
            return fail(NT_ERR_NULL_POINTER, "layer %d gradient buffers are NULL", l);
        if (need_moments && (!m->weight_moment1[l] || !m->weight_moment2[l] ||
                             !m->bias_moment1[l] || !m->bias_moment2[l]))
            return fail(NT_ERR_NULL_POINTER, "layer %d Adam moment buffers are NULL", l);
    }
    return NT_OK;
}

MlpDesc mlp_desc(const nt_mlp *m)
{
    MlpDesc d{};
    d.num_layers = m->num_layers;
    for (int l = 0; l < m->num_layers; ++l) {
        d.W[l] = m->weights[l];
        d.B[l] = m->biases[l];
    }
    for (int l = 0; l <= m->num_layers; ++l)
        d.sizes[l] = m->sizes[l];
    return d;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Validates the latent grids for sampling. unconstrained: values (+ grads) needed;
// otherwise block records.
int check_latents(const nt_latents *lat, int shape, bool need_grads, bool blocks)
{
    if (!lat)
        return fail(NT_ERR_NULL_POINTER, "latents is NULL");
    if (lat->num_grids < 1 || lat->num_grids > NT_MAX_GRIDS)
        return fail(NT_ERR_INVALID_ARGUMENT, "num_grids %d outside [1, %d]", lat->num_grids, NT_MAX_GRIDS);
    const int C = shape_channels(shape);
    if (lat->channels != C)
        return fail(NT_ERR_UNSUPPORTED, "this MLP shape is built for %d channels per grid, got %d", C,
                    lat->channels);
    for (int gi = 0; gi < lat->num_grids; ++gi) {
        const nt_grid &g = lat->grids[gi];
        if (g.width < 1 || g.height < 1 || g.num_mips < 1 || g.num_mips > NT_MAX_MIPS)
            return fail(NT_ERR_INVALID_ARGUMENT, "grid %d: bad size %dx%d or mip count %d", gi, g.width,
                        g.height, g.num_mips);
        if (!blocks) {
            if (!g.values || (need_grads && !g.grads))
                return fail(NT_ERR_NULL_POINTER, "grid %d: values/grads are NULL", gi);
            if ((C % 4 == 0) && !aligned16(g.values))
                return fail(NT_ERR_MISALIGNED, "grid %d: values must be 16-byte aligned", gi);
            for (int m = 0; m < g.num_mips; ++m)
                if (g.mip_offset[m] < 0 || ((C % 4 == 0) && (g.mip_offset[m] * C) % 4))
                    return fail(NT_ERR_MISALIGNED, "grid %d: bad mip_offset[%d]", gi, m);
        } else {
            if (!g.block_params || (need_grads && !g.block_grads))
                return fail(NT_ERR_NULL_POINTER, "grid %d: block_params/block_grads are NULL", gi);
            if ((g.width & 3) && g.width > 4)
                return fail(NT_ERR_INVALID_ARGUMENT, "grid %d: block storage needs a width multiple of 4", gi);
            if ((g.height & 3) && g.height > 4)
                return fail(NT_ERR_INVALID_ARGUMENT, "grid %d: block storage needs a height multiple of 4", gi);
        }
    }
    return NT_OK;
}

GridDesc grid_desc(const nt_grid &g, int C)
{
    GridDesc d{};
    d.values = g.values;
    d.grads = g.grads;
    d.block_params = g.block_params;
    d.block_grads = g.block_grads;
    d.w = g.width;
    d.h = g.height;
    d.num_mips = g.num_mips;
    for (int m = 0; m < NT_MAX_MIPS; ++m) {
        d.mip_off[m] = g.mip_offset[m];
        d.block_off[m] = g.block_offset[m];
    }
    (void)C;
    return d;
}

// Output-channel packing of the reference textures (train.cu:105-157,
// main.cpp:243-258). Returns the number of packed channels or a negative status.
int pack_targets(const nt_texture *tex, int ntex, int8_t *out_tex, int8_t *out_ch, float *out_w,
                 TexDesc *td)
{
    for (int o = 0; o < NT_MAX_OUTPUTS; ++o) {
        out_tex[o] = -1;
        out_ch[o] = 0;
        out_w[o] = 1.f;
    }
    if (ntex < 0 || ntex > NT_MAX_TEXTURES)
        return -fail(NT_ERR_INVALID_ARGUMENT, "num_textures %d outside [0, %d]", ntex, NT_MAX_TEXTURES);
    int oc = 0;
    for (int ti = 0; ti < ntex && oc < NT_MAX_OUTPUTS; ++ti) {
        const nt_texture &t = tex[ti];
        td[ti] = TexDesc{};
        if (!t.texels || t.num_channels <= 0)
            continue;
        if (t.width < 1 || t.height < 1 || t.num_mips < 1 || t.num_mips > NT_MAX_MIPS)
            return -fail(NT_ERR_INVALID_ARGUMENT, "texture %d: bad size or mip count", ti);
        const int nc = t.num_channels == 1 ? 1 : (t.num_channels < 4 ? t.num_channels : 4);
        if (!((t.pitch == 4) || (t.pitch == 1 && nc == 1)))
            return -fail(NT_ERR_INVALID_ARGUMENT, "texture %d: pitch must be 4 (or 1 for one channel)", ti);
        if (t.pitch == 4 && !aligned16(t.texels + t.mip_offset[0] * 4))
            return -fail(NT_ERR_MISALIGNED, "texture %d: texels must be 16-byte aligned", ti);
        td[ti].texels = t.texels + t.mip_offset[0] * t.pitch;
        td[ti].w = t.width;
        td[ti].h = t.height;
        td[ti].pitch = t.pitch;
        td[ti].nch = nc;
        for (int c = 0; c < nc && oc < NT_MAX_OUTPUTS; ++c, ++oc) {
            out_tex[oc] = (int8_t)ti;
            out_ch[oc] = (int8_t)c;
            out_w[oc] = t.loss_weight;
        }
    }
    return oc;
}

// NT_LATENT_TOUCHED keeps its update log in the last kUpdateLogBytes of the workspace (so
// that nt_inference's SSE partials at its start never overlap it); the train step and the
// optimizer both find it there.
size_t touched_bytes(const nt_params *p)
{
    return p->latent_update == NT_LATENT_TOUCHED ? kUpdateLogBytes : 0;
}

UpdateLog *update_log(const nt_params *p)
{
    const size_t lb = touched_bytes(p);
    if (!lb || !p->workspace || p->workspace_bytes < lb)
        return nullptr;
    return (UpdateLog *)((uint8_t *)p->workspace + ((p->workspace_bytes - lb) & ~(size_t)15));
}

// Texel rectangle {x0, x1, y0, y1} of grid g (inclusive, before wrapping: x0 and y0 may
// be negative, x1 and y1 past the grid) that holds every bilinear corner a train step's
// positions reach; the whole grid where the positions are random or span it.
void footprint_rect(const nt_params *p, int width, int height, int (&rect)[4])
{
    if (p->sample_mode == NT_SAMPLES_RANDOM) {
        rect[0] = rect[2] = 0;
        rect[1] = width - 1;
        rect[3] = height - 1;
        return;
    }
    // Positions lie in [off, off + extent] texels of the image (jitter and clamping
    // included); their footprints' corners at floor(pos * r - 0.5) + {0, 1}, with a texel
    // of margin on each side for rounding.
    const int rw = p->region_width > 0 ? p->region_width : NT_DEFAULT_REGION;
    const double rx = (double)width / p->image_width, ry = (double)height / p->image_height;
    const int rows = (int)(((int64_t)p->num_samples + rw - 1) / rw);
    const int x0 = (int)std::floor(p->texel_offset_x * rx - 0.5) - 1;
    const int x1 = (int)std::floor((double)(p->texel_offset_x + rw) * rx - 0.5) + 2;
    const int y0 = (int)std::floor(p->texel_offset_y * ry - 0.5) - 1;
    const int y1 = (int)std::floor((double)(p->texel_offset_y + rows) * ry - 0.5) + 2;
    // Wider than the grid: the whole width (height) of it.
    rect[0] = x1 - x0 + 1 >= width ? 0 : x0;
    rect[1] = x1 - x0 + 1 >= width ? width - 1 : x1;
    rect[2] = y1 - y0 + 1 >= height ? 0 : y0;
    rect[3] = y1 - y0 + 1 >= height ? height - 1 : y1;
}

struct TrainPlan {
    int shape, nwg, chunks_per_wg, tiles_x, P;
    int fp_floats, fp_stride, tile_ok, scatter_mfma, scatter_split, scatter_off, w_rows, union_off;
    int vbox_floats, vbox_off;
    size_t weight_bytes;
    int fp_w[NT_MAX_GRIDS], fp_h[NT_MAX_GRIDS], fp_off[NT_MAX_GRIDS], vb_off[NT_MAX_GRIDS];
    int cb_w[NT_MAX_GRIDS], cb_h[NT_MAX_GRIDS], w_row0[NT_MAX_GRIDS];
    size_t lds, workspace;
    // The 16-channel unconstrained kernel (nt_train16.hip), when it applies.
    int use16, groups, rows;
    Train16Desc t16;
    // Its random-texel sample order (nt_sort.hip): byte offset of the sort buffers in the
    // workspace (0: no sort), the bins a row and the key bits, the digit counts' bytes.
    size_t sort_off, sort_temp;
    int sort_bins_x, sort_key_bits, sort_shift;
    // The BC6 block phase (Bc6PhaseDesc): the rest of the plan is the inner unconstrained
    // step's. Per grid the mips the inner step sees (its chain stops after the last level a
    // sample reaches) and the workspace offsets of the expanded chain and its gradients; per
    // level its grid and mip.
    int bc6;
    Bc6PhaseDesc bc6d;
    int bc6_mips[NT_MAX_GRIDS];
    size_t bc6_values_off[NT_MAX_GRIDS], bc6_grads_off[NT_MAX_GRIDS];
    int bc6_level_grid[2 * NT_MAX_GRIDS], bc6_level_mip[2 * NT_MAX_GRIDS];
};

constexpr size_t kMaxLds = 160 * 1024;

// Plan of the 16-channel kernel (nt_train16.hip): unconstrained latents of 16 channels,
// one to four reference textures of the image size with float4 texels (their channels
// become output rows 4t + ch), and an LDS layout that fits. Sets plan->use16.
// 1/n when n is a power of two (exact in fp32), else 0.
float pow2_reciprocal(int n)
{
    return n > 0 && (n & (n - 1)) == 0 ? 1.f / (float)n : 0.f;
}

void plan16(const nt_params *p, nt_kernel_type type, TrainPlan *plan)
{
    plan->use16 = 0;
    const bool random = p->sample_mode == NT_SAMPLES_RANDOM;
    const int NG = train16_groups(plan->shape, random);
    const int C = p->latents.channels, G = p->latents.num_grids;
    // 16-channel grids, or the reference network's four 3-channel grids.
    const bool c3 = plan->shape == kShapeRef;
    if (type != NT_UNCONSTRAINED || C != (c3 ? 3 : 16) || (c3 && G != 4) || NG == 0 || p->num_textures < 1 ||
        p->num_textures > 4 || p->sample_mip != 0.f)
        return;
    // Random texels: taps are wrapped with one conditional add or subtract (at least four
    // texels a side) and addressed with 32-bit texel indices.
    if (random && (p->image_width < 4 || p->image_height < 4 ||
                   (int64_t)p->image_width * p->image_height >= (1ll << 31)))
        return;
    // The prologue copies the weight matrices with 16-byte loads.
    for (int l = 0; l < p->mlp.num_layers; ++l)
        if (!aligned16(p->mlp.weights[l]))
            return;
    Train16Desc &d = plan->t16;
    d = Train16Desc{};
    // The one-group (config 4) kernel: its single wave per SIMD runs both lane groups' taps
    // in turn (two waves per SIMD cover the imbalance, measured: no gain for them).
    d.split3 = !random && NG == 1 && p->num_textures == 3;
    int prefix = 0;
    bool mapped[NT_MAX_OUTPUTS] = {};
    int8_t row_out[NT_MAX_OUTPUTS];
    for (int r = 0; r < NT_MAX_OUTPUTS; ++r)
        row_out[r] = -1;
    for (int t = 0; t < p->num_textures; ++t) {
        const nt_texture &x = p->textures[t];
        if (!x.texels || x.num_channels < 1 || x.pitch != 4 || x.width != p->image_width ||
            x.height != p->image_height || !aligned16(x.texels + x.mip_offset[0] * 4))
            return;
        const int nch = x.num_channels < 4 ? x.num_channels : 4;
        d.tex[t] = x.texels + x.mip_offset[0] * 4;
        d.tex_nch[t] = nch;
        d.four_channels |= nch == 4;
        d.tex_w[t] = x.loss_weight;
        for (int ch = 0; ch < nch; ++ch) {
            // The third of three textures: channels 0, 1 on rows 8, 9 (lane group 0), 2, 3
            // on rows 12, 13 (lane group 1).
            const int row = d.split3 && t == 2 ? (ch < 2 ? 8 + ch : 12 + ch - 2) : 4 * t + ch;
            row_out[row] = (int8_t)(prefix + ch);
            mapped[prefix + ch] = true;
        }
        prefix += nch;
    }
    for (int t = p->num_textures; t < 4; ++t) {
        d.tex[t] = d.tex[0];
        d.tex_w[t] = 1.f;
    }
    // Rows without a texture channel take the remaining outputs in increasing order.
    int next = 0;
    for (int r = 0; r < NT_MAX_OUTPUTS; ++r) {
        if (row_out[r] < 0) {
            while (mapped[next])
                ++next;
            row_out[r] = (int8_t)next;
            mapped[next] = true;
        }
        d.perm |= (uint64_t)row_out[r] << (4 * r);
    }
    d.ntex = p->num_textures;
    const int rw = p->region_width > 0 ? p->region_width : NT_DEFAULT_REGION;
    const int rows = (int)(((int64_t)p->num_samples + rw - 1) / rw);
    // Region: tiles of 64 x 8NG positions. Random texels: tiles of 512 consecutive samples
    // (of the position-sorted order).
    d.tiles_x = random ? 1 : (rw + 4 * kChunkW - 1) / (4 * kChunkW);
    const int64_t tiles_y = random ? ((int64_t)p->num_samples + 4 * kChunk * NG - 1) / (4 * kChunk * NG)
                                   : (rows + kChunkH * NG - 1) / (kChunkH * NG);
    if ((int64_t)d.tiles_x * tiles_y > (1 << 30))
        return;
    // One workgroup per CU (the kernel's registers and LDS allow no second one); each takes
    // every nwg-th tile, so that fewer, longer-lived workgroups stage the weights and write
    // MLP-gradient partials.
    // A test hook can lower the cap (to give workgroups several tiles at small sizes).
    d.ntiles = d.tiles_x * tiles_y;
    int cap = device_cu_count();
    if (const int hook = g_hook_max_workgroups.load(std::memory_order_relaxed); hook > 0)
        cap = std::min(cap, hook);
    d.nwg = std::min(d.ntiles, cap);
    d.xcd_per = (d.ntiles % 8 == 0 && d.nwg % 8 == 0) ? d.ntiles / 8 : 0;
    // Margin of the chunk cell box beyond the cells positions can reach. A test hook drops
    // it, to drive the scatter's out-of-box path (per-sample global atomics), which
    // positions never take.
    const int cell_margin = g_hook_no_margins.load(std::memory_order_relaxed) ? 0 : 2;
    for (int gi = 0; gi < G; ++gi) {
        const nt_grid &g = p->latents.grids[gi];
        Grid16 &q = d.grid[gi];
        const double rx = (double)g.width / p->image_width, ry = (double)g.height / p->image_height;
        // The kernel addresses a grid's mip 0 with 32-bit offsets.
        if ((int64_t)g.width * g.height * C >= (1ll << 31))
            return;
        q.values = g.values + g.mip_offset[0] * C;
        q.grads = g.grads + g.mip_offset[0] * C;
        q.w = g.width;
        q.h = g.height;
        q.cb_w = (int)std::ceil(kChunkW * rx) + cell_margin;
        q.cb_h = (int)std::ceil(kChunkH * ry) + cell_margin;
        q.ncell = q.cb_w * q.cb_h;
        q.inv_cb_w = 1.f / (float)q.cb_w;
        q.rx = (float)g.width / (float)p->image_width;
        q.ry = (float)g.height / (float)p->image_height;
        if (c3 ? (((uintptr_t)q.values | (uintptr_t)q.grads) & 3) != 0 : !aligned16(q.values) || !aligned16(q.grads))
            return;
    }
    const size_t head = train16_head_bytes(plan->shape);
    // Scatter: dX0 rows, then the weight rows (hi, lo) of the chunk box, or with random texels
    // each wave's corner slots (32 samples x grids x 4 corners x {texel, weight}).
    const size_t dx_rows = (size_t)kChunk * dx_stride(pad16(p->mlp.sizes[0])) * 2;
    d.random_texels = random;
    d.tile_bytes = random ? 0 : d.ntex * kT16TileSlots * 16;
    d.group_off = (int)((head + 15) & ~(size_t)15);
    // The weight-row columns of the grids that take the MFMA reduction, and the LDS that
    // layout needs. A grid whose chunk cell box is large (a grid as fine as the image or
    // nearly: few samples per cell) costs LDS out of proportion to what the reduction saves;
    // while the layout does not fit, the grid with the most cells leaves the reduction and
    // adds its corners with per-sample global atomics instead (an empty cell box sends every
    // footprint down that path).
    auto layout = [&]() {
        int wcols = 0;
        for (int gi = 0; gi < G; ++gi) {
            d.grid[gi].wcol0 = wcols;
            wcols += 16 * ((d.grid[gi].ncell + 15) / 16);
        }
        // Rows of an odd number of 16-byte chunks: each lane clears its own row with 16-byte
        // stores, which then fall in distinct LDS banks. Only the task columns are read (and
        // so cleared), not the padding.
        d.wclear = wcols / 8;
        if (wcols % 16 == 0)
            wcols += 8;
        d.wcols = wcols;
        const size_t scatter = dx_rows + (random ? (size_t)4 * 32 * G * 4 * 8 : 2 * (size_t)kChunk * wcols * 2);
        size_t un = train16_transpose_bytes(plan->shape);
        un = scatter > un ? scatter : un;
        d.group_bytes = (int)((d.tile_bytes + un + 15) & ~(size_t)15);
        return (size_t)d.group_off + (size_t)NG * d.group_bytes;
    };
    // The kernel runs each wave's scatter-reduction tasks (16-cell tiles of the cell boxes)
    // in one pass of two: at most eight (so at most 128 cells per box, and box coordinates
    // below 256).
    auto tasks = [&]() {
        int n = 0;
        for (int gi = 0; gi < G; ++gi)
            n += (d.grid[gi].ncell + 15) / 16;
        return n;
    };
    size_t lds = layout();
    while (!random && (lds > kMaxLds || tasks() > 8)) {
        int big = -1;
        for (int gi = 0; gi < G; ++gi)
            if (d.grid[gi].ncell > 0 && (big < 0 || d.grid[gi].ncell > d.grid[big].ncell))
                big = gi;
        if (big < 0)
            return;
        Grid16 &q = d.grid[big];
        q.cb_w = q.cb_h = q.ncell = 0;
        q.inv_cb_w = 0.f;
        lds = layout();
    }
    // The grids that left the reduction add their corners into LDS boxes over the workgroup
    // tile's footprint (the box of the general kernel: every texel a 64 x 8NG block of
    // positions can touch, plus rounding slack), flushed once per tile, when they fit:
    // per-sample global atomics are performed past the L2, one memory operation per float.
    d.box_lds_off = (int)((lds + 15) & ~(size_t)15);
    d.box_floats = 0;
    d.gather_grids = 0;
    for (int gi = 0; gi < G; ++gi) {
        Grid16 &q = d.grid[gi];
        q.box_off = q.box_w = q.box_h = 0;
        q.slot_off = -1;
        q.gk = 0;
        if (!c3 || random || q.ncell > 0)
            continue;
        const int bw = (int)std::ceil(4 * kChunkW * (double)q.w / p->image_width) + 4;
        const int bh = (int)std::ceil(kChunkH * NG * (double)q.h / p->image_height) + 4;
        if ((size_t)d.box_lds_off + ((size_t)d.box_floats + (size_t)bw * bh * C) * 4 > kMaxLds)
            continue;
        q.box_off = d.box_floats;
        q.box_w = bw;
        q.box_h = bh;
        d.box_floats += bw * bh * C;
    }
    // A boxed grid of 1/k of the image's size, k = 1 or 2 (each texel is reached only by the
    // corners of the positions in a fixed window of 3 or 4 around k times it), sums each box
    // texel's corners by gather from per-sample records placed after the boxes, when they
    // fit; other boxed grids add each corner with an LDS atomic.
    int slot_floats = 0;
    for (int gi = 0; gi < G; ++gi) {
        Grid16 &q = d.grid[gi];
        if (q.box_w == 0)
            continue;
        int k = 0;
        for (int kk = 1; kk <= 2; ++kk)
            if ((int64_t)q.w * kk == p->image_width && (int64_t)q.h * kk == p->image_height)
                k = kk;
        const int n = NG * kChunk * 4;
        if (k == 0 || (size_t)d.box_lds_off + ((size_t)d.box_floats + slot_floats + n) * 4 > kMaxLds)
            continue;
        q.slot_off = d.box_floats + slot_floats;
        q.gk = k;
        slot_floats += n;
        ++d.gather_grids;
    }
    if (d.box_floats > 0)
        lds = (size_t)d.box_lds_off + ((size_t)d.box_floats + slot_floats) * 4;
    // The one-group kernel's gather boxes: every grid's chunk cell box, at most 64 cells
    // (one wave instruction of 64 float4 per wave), whole wave instructions per buffer.
    d.gbox_off = d.gbox_bytes = d.gbox_items = 0;
    if (NG == 1 && !c3 && !random) {
        int cells = 0;
        bool all = true;
        for (int gi = 0; gi < G; ++gi) {
            d.grid[gi].gcell0 = cells;
            cells += d.grid[gi].ncell;
            all = all && d.grid[gi].ncell > 0;
        }
        const size_t off = (lds + 1023) & ~(size_t)1023, bytes = (size_t)((4 * cells + 63) / 64) * 1024;
        if (all && cells > 0 && cells <= 64 && off + 2 * bytes <= kMaxLds) {
            d.gbox_off = (int)off;
            d.gbox_bytes = (int)bytes;
            d.gbox_items = 4 * cells;
            lds = off + 2 * bytes;
        }
    }
    // The second group's region carries its dW accumulators to the first at the end.
    const size_t handoff = (size_t)train16_slots(plan->shape) * 17 * kTrainThreads * 4;
    if (NG == 2 && (size_t)d.group_bytes < handoff) {
        // Random texels keep no tile or cell box in the group regions: enlarge them.
        if (!random)
            return;
        d.group_bytes = (int)((handoff + 15) & ~(size_t)15);
        lds = (size_t)d.group_off + (size_t)NG * d.group_bytes;
    }
    // The prologue stages the fp16 weight matrices in the group regions.
    if (lds > kMaxLds || train16_raw_bytes(plan->shape) > (size_t)NG * d.group_bytes)
        return;
    plan->use16 = 1;
    plan->groups = NG;
    plan->lds = lds;
    plan->nwg = d.nwg;
    plan->rows = d.nwg; // the groups of a workgroup merge their partials in LDS
    plan->weight_bytes = 0; // each workgroup builds its weight image in LDS
    plan->workspace = (size_t)plan->rows * (size_t)plan->P * sizeof(float);
    // Random texels: the sort of the sample indices by bin after the partial rows (keys and
    // sample indices in two buffers each, then the per-tile digit counts). From 262,144
    // samples: config 2 with random texels runs its train kernel 204 -> 176 us with it,
    // config 4 (1,048,576 samples) 1,392 -> 1,120 us.
    plan->sort_off = plan->sort_temp = 0;
    if (random && (p->num_samples >= kRandomSortMinSamples || g_hook_sort_random.load(std::memory_order_relaxed))) {
        // Bins of 64 x 64 texels (coarser ones, one 8-bit sort pass, gained less).
        const int shift = 6;
        const int bx = (p->image_width + (1 << shift) - 1) >> shift;
        const int by = (p->image_height + (1 << shift) - 1) >> shift;
        plan->sort_shift = shift;
        if ((int64_t)bx * by <= 65536) {
            int bits = 1;
            while ((1 << bits) < bx * by)
                ++bits;
            const size_t n = (size_t)p->num_samples;
            const size_t temp = (random_order_count_bytes(p->num_samples, bits) + 255) & ~(size_t)255;
            const size_t keys = (n * 2 + 255) & ~(size_t)255, vals = (n * 4 + 255) & ~(size_t)255;
            plan->sort_off = (plan->workspace + 255) & ~(size_t)255;
            plan->sort_temp = temp;
            plan->sort_bins_x = bx;
            plan->sort_key_bits = bits;
            plan->workspace = plan->sort_off + 2 * keys + 2 * vals + temp;
        }
    }
    d.image_w = p->image_width;
    d.image_h = p->image_height;
    d.off_x = p->texel_offset_x;
    d.off_y = p->texel_offset_y;
    d.region_w = rw;
    d.num_samples = p->num_samples;
    d.step = (uint32_t)p->step;
    d.inv_w = pow2_reciprocal(d.image_w);
    d.inv_h = pow2_reciprocal(d.image_h);
    d.inv_samples = pow2_reciprocal(d.num_samples);
}

int floor_div4(int v) { return v >= 0 ? v / 4 : -((3 - v) / 4); }

// Texel offset of mip m in a dense chain of a width x height grid (nt_mip_chain_layout).
int64_t chain_offset(int width, int height, int m)
{
    int64_t o = 0;
    for (int k = 0; k < m; ++k)
        o += (int64_t)mip_dim_h(width, k) * mip_dim_h(height, k);
    return o;
}

// The mips a step with mip coordinate z samples in a chain of num_mips (train.cu:266-281):
// floor(z) and, when z has a fraction, floor(z) + 1, both clamped to the last mip.
int mip_pair(int num_mips, float z, int (&m)[2])
{
    const float zb = floorf(z);
    const int top = num_mips - 1;
    m[0] = std::min((int)std::min(zb, (float)top), top);
    m[1] = std::min(m[0] + 1, top);
    return z - zb > 0.f ? 2 : 1;
}

// The inner unconstrained step of the BC6 phase: p with every grid's values and gradients
// replaced by the expanded chain in the workspace at ws (stand-in addresses, 256-byte
// aligned like the real ones, when ws is NULL), mips up to the last level sampled.
nt_params bc6_inner(const nt_params *p, const TrainPlan &plan, uint8_t *ws)
{
    nt_params q = *p;
    q.latent_update = NT_LATENT_DENSE;
    for (int gi = 0; gi < p->latents.num_grids; ++gi) {
        nt_grid &g = q.latents.grids[gi];
        g.num_mips = plan.bc6_mips[gi];
        for (int m = 0; m < NT_MAX_MIPS; ++m)
            g.mip_offset[m] = m < g.num_mips ? chain_offset(g.width, g.height, m) : 0;
        g.values = ws ? (float *)(ws + plan.bc6_values_off[gi]) : (float *)(uintptr_t)256;
        g.grads = ws ? (float *)(ws + plan.bc6_grads_off[gi]) : (float *)(uintptr_t)256;
    }
    return q;
}

int plan_train(const nt_params *p, nt_kernel_type type, TrainPlan *plan);

// The BC6 block phase (NT_BLOCK_FEATURES, NT_FINALIZE) runs an unconstrained train step on
// texels expanded from the block records of every level a sample reaches (Bc6PhaseDesc):
// the step is planned as one over grids whose texels live in the workspace, after its own
// scratch. Sets plan->bc6 (and then the inner step's plan), or leaves the plan alone.
void plan_bc6_phase(const nt_params *p, TrainPlan *plan)
{
    plan->bc6 = 0;
    const int C = p->latents.channels, G = p->latents.num_grids;
    if (C != 3 && C != 8 && C != 16)
        return;
    TrainPlan t = *plan;
    t.bc6 = 0;
    int levels = 0;
    for (int gi = 0; gi < G; ++gi) {
        const nt_grid &g = p->latents.grids[gi];
        int m[2];
        const int n = mip_pair(g.num_mips, p->sample_mip, m);
        t.bc6_mips[gi] = (n == 2 ? m[1] : m[0]) + 1;
        for (int k = 0; k < n; ++k) {
            if (k == 1 && m[1] == m[0])
                break; // both weights on the last mip: one level
            t.bc6_level_grid[levels] = gi;
            t.bc6_level_mip[levels] = m[k];
            ++levels;
        }
    }
    const nt_params q = bc6_inner(p, t, nullptr);
    TrainPlan inner;
    if (plan_train(&q, NT_UNCONSTRAINED, &inner) != NT_OK)
        return;
    // The inner plan, with the phase's fields.
    for (int gi = 0; gi < G; ++gi)
        inner.bc6_mips[gi] = t.bc6_mips[gi];
    for (int k = 0; k < levels; ++k) {
        inner.bc6_level_grid[k] = t.bc6_level_grid[k];
        inner.bc6_level_mip[k] = t.bc6_level_mip[k];
    }
    Bc6PhaseDesc &b = inner.bc6d;
    b = Bc6PhaseDesc{};
    b.nlevels = levels;
    b.C = C;
    size_t off = (inner.workspace + 255) & ~(size_t)255;
    for (int gi = 0; gi < G; ++gi) {
        const nt_grid &g = p->latents.grids[gi];
        const size_t bytes =
            ((size_t)chain_offset(g.width, g.height, inner.bc6_mips[gi]) * C * sizeof(float) + 255) & ~(size_t)255;
        inner.bc6_values_off[gi] = off;
        off += bytes;
        inner.bc6_grads_off[gi] = off;
        off += bytes;
    }
    int64_t first = 0;
    for (int k = 0; k < levels; ++k) {
        const nt_grid &g = p->latents.grids[inner.bc6_level_grid[k]];
        const int m = inner.bc6_level_mip[k];
        Bc6PhaseLevel &x = b.level[k];
        x.w = mip_dim_h(g.width, m);
        x.h = mip_dim_h(g.height, m);
        x.nbu = std::max(x.w >> 2, 1);
        x.nbv = std::max(x.h >> 2, 1);
        int r[4];
        footprint_rect(p, x.w, x.h, r);
        x.bx0 = floor_div4(r[0]);
        x.nbx = floor_div4(r[1]) - x.bx0 + 1;
        if (x.nbx >= x.nbu) {
            x.bx0 = 0;
            x.nbx = x.nbu;
        }
        x.by0 = floor_div4(r[2]);
        x.nby = floor_div4(r[3]) - x.by0 + 1;
        if (x.nby >= x.nbv) {
            x.by0 = 0;
            x.nby = x.nbv;
        }
        x.first_block = first;
        first += (int64_t)x.nbx * x.nby;
    }
    b.total_blocks = first;
    inner.workspace = off;
    inner.bc6 = 1;
    *plan = inner;
}

int plan_train(const nt_params *p, nt_kernel_type type, TrainPlan *plan)
{
    if (!p)
        return fail(NT_ERR_NULL_POINTER, "params is NULL");
    if (type != NT_UNCONSTRAINED && type != NT_BLOCK_FEATURES && type != NT_FINALIZE)
        return fail(NT_ERR_INVALID_ARGUMENT, "bad kernel type %d", (int)type);
    int shape;
    int st = check_mlp(&p->mlp, true, false, &shape);
    if (st)
        return st;
    if (shape != kShapeRef && shape != kShapeC1 && shape != kShapeC2 && shape != kShapeC4)
        return fail(NT_ERR_UNSUPPORTED, "training is built for 12->32->32->16 (C=3), 8->64->64->16 (C=8), "
                                        "32->64->64->16 (C=16) and 64->64->64->64->16 (C=16)");
    st = check_latents(&p->latents, shape, type != NT_FINALIZE, type != NT_UNCONSTRAINED);
    if (st)
        return st;
    if (p->latents.num_grids * p->latents.channels != p->mlp.sizes[0])
        return fail(NT_ERR_INVALID_ARGUMENT, "MLP input %d != num_grids*channels %d", p->mlp.sizes[0],
                    p->latents.num_grids * p->latents.channels);
    if (p->image_width < 1 || p->image_height < 1)
        return fail(NT_ERR_INVALID_ARGUMENT, "image size %dx%d", p->image_width, p->image_height);
    if (p->num_samples < 1)
        return fail(NT_ERR_INVALID_ARGUMENT, "num_samples %d", p->num_samples);
    if (p->sample_mode != NT_SAMPLES_REGION && p->sample_mode != NT_SAMPLES_RANDOM)
        return fail(NT_ERR_INVALID_ARGUMENT, "sample_mode %d", p->sample_mode);
    if (p->latent_update != NT_LATENT_DENSE && p->latent_update != NT_LATENT_TOUCHED)
        return fail(NT_ERR_INVALID_ARGUMENT, "latent_update %d", p->latent_update);
    if (!std::isfinite(p->sample_mip) || p->sample_mip < 0.f)
        return fail(NT_ERR_INVALID_ARGUMENT, "sample_mip %g", (double)p->sample_mip);
    const int rw = p->region_width > 0 ? p->region_width : NT_DEFAULT_REGION;
    const int rows = (int)(((int64_t)p->num_samples + rw - 1) / rw);
    plan->shape = shape;
    plan->chunks_per_wg = 4;
    const int tile_w = kChunkW * plan->chunks_per_wg;
    plan->tiles_x = (rw + tile_w - 1) / tile_w;
    const int tiles_y = (rows + kChunkH - 1) / kChunkH;
    if ((int64_t)plan->tiles_x * tiles_y > (1 << 30))
        return fail(NT_ERR_INVALID_ARGUMENT, "too many samples");
    plan->nwg = plan->tiles_x * tiles_y;
    plan->P = train_grad_total(shape);
    plan->weight_bytes = train_weight_bytes(shape);
    plan->workspace = plan->weight_bytes + (size_t)plan->nwg * (size_t)plan->P * sizeof(float);

    // LDS footprint box per grid: every texel a 64 x 8 block of positions can touch (the
    // bilinear corners of positions in [x, x + 64] span at most ceil(64 r) + 2 texels, plus
    // one of rounding slack on each side). Texels are `fp_stride` (odd) floats apart so
    // that neighbouring texels fall in different LDS banks.
    const int C = p->latents.channels;
    plan->fp_stride = C | 1;
    // Margin of the chunk cell box (as in the 16-channel plan; a test hook drops it).
    const int cell_margin = g_hook_no_margins.load(std::memory_order_relaxed) ? 0 : 2;
    int fp = 0, w_rows = 0, vb = 0;
    for (int gi = 0; gi < p->latents.num_grids; ++gi) {
        const nt_grid &g = p->latents.grids[gi];
        const double rx = (double)g.width / p->image_width, ry = (double)g.height / p->image_height;
        plan->fp_w[gi] = (int)std::ceil(tile_w * rx) + 4;
        plan->fp_h[gi] = (int)std::ceil(kChunkH * ry) + 4;
        plan->fp_off[gi] = fp;
        fp += plan->fp_w[gi] * plan->fp_h[gi] * plan->fp_stride;
        plan->vb_off[gi] = vb;
        vb += plan->fp_w[gi] * plan->fp_h[gi];
        // Chunk cell box for the MFMA scatter: positions in [x, x + 16] x [y, y + 8].
        plan->cb_w[gi] = (int)std::ceil(kChunkW * rx) + cell_margin;
        plan->cb_h[gi] = (int)std::ceil(kChunkH * ry) + cell_margin;
        plan->w_row0[gi] = w_rows;
        w_rows += 16 * ((plan->cb_w[gi] * plan->cb_h[gi] + 15) / 16);
    }
    plan->w_rows = w_rows;
    // The chunk's target taps are staged in LDS when every reference texture has the image
    // size (as the reference requires, main.cpp:972-978).
    plan->tile_ok = p->num_textures > 0;
    for (int ti = 0; ti < p->num_textures && ti < NT_MAX_TEXTURES; ++ti) {
        const nt_texture &t = p->textures[ti];
        if (t.texels && t.num_channels > 0 && (t.width != p->image_width || t.height != p->image_height))
            plan->tile_ok = 0;
    }
    const size_t head = train_lds_static(shape);
    const size_t transposes = train_xt_bytes(shape);
    const size_t tile = (size_t)p->num_textures * kTileW * kTileH * 16;
    const size_t scatter = ((size_t)pad16(p->mlp.sizes[0]) + 2 * (size_t)w_rows) * kRowStride * 2;
    auto fp_bytes = [](int fp_floats) { return ((size_t)fp_floats * 4 + 15) & ~(size_t)15; };
    auto union_bytes = [&](bool use_tile, bool scatter_in_union) {
        size_t un = transposes;
        if (use_tile && tile > un)
            un = tile;
        if (scatter_in_union && scatter > un)
            un = scatter;
        return un;
    };
    // Random texels have no spatial locality within a workgroup: no footprint box, value
    // box or target tile; gathers, taps and scatter atomics go to global memory.
    // Samples at a mip coordinate z > 0 take the general per-sample paths (two mips).
    const bool random = p->sample_mode == NT_SAMPLES_RANDOM || p->sample_mip != 0.f;
    if (random)
        plan->tile_ok = 0;
    plan->fp_floats = type == NT_UNCONSTRAINED && !random ? fp : 0;
    if (plan->fp_floats && head + fp_bytes(plan->fp_floats) + union_bytes(false, false) > kMaxLds)
        plan->fp_floats = 0; // box does not fit: scatter straight to global memory
    // With 16 channels the latent values under the box are staged in LDS too, so the
    // gathers read LDS instead of HBM.
    plan->vbox_floats = plan->fp_floats > 0 && C == 16 ? vb * 16 : 0;
    if (plan->vbox_floats &&
        head + fp_bytes(plan->fp_floats) + fp_bytes(plan->vbox_floats) + union_bytes(false, false) > kMaxLds)
        plan->vbox_floats = 0;
    plan->vbox_off = (int)(head + fp_bytes(plan->fp_floats));
    if (plan->tile_ok &&
        head + fp_bytes(plan->fp_floats) + fp_bytes(plan->vbox_floats) + union_bytes(true, false) > kMaxLds)
        plan->tile_ok = 0;
    const size_t base = head + fp_bytes(plan->fp_floats) + fp_bytes(plan->vbox_floats);
    plan->union_off = (int)base;
    plan->scatter_mfma = 0;
    plan->scatter_split = 0;
    plan->scatter_off = 0;
    plan->lds = base + union_bytes(plan->tile_ok, false);
    if (plan->fp_floats > 0 && C <= 16) {
        // The scatter matrices get their own region when it fits, which lets the scatter
        // share the layer-0 dW phase; otherwise they reuse the union after that phase.
        if (base + union_bytes(plan->tile_ok, false) + scatter <= kMaxLds) {
            plan->scatter_mfma = plan->scatter_split = 1;
            plan->scatter_off = (int)(base + union_bytes(plan->tile_ok, false));
            plan->lds = plan->scatter_off + scatter;
        } else if (base + union_bytes(plan->tile_ok, true) <= kMaxLds) {
            plan->scatter_mfma = 1;
            plan->lds = base + union_bytes(plan->tile_ok, true);
        }
    }
    plan->rows = plan->nwg;
    plan->bc6 = 0;
    plan16(p, type, plan);
    if (type != NT_UNCONSTRAINED)
        plan_bc6_phase(p, plan);
    if (type != NT_UNCONSTRAINED && !plan->bc6)
        return fail(NT_ERR_UNSUPPORTED, "block records train through the BC6 phase, built for 3, 8 and 16 "
                                        "channels");
    return NT_OK;
}

} // namespace

int ntk::report(int status, const char *fmt, ...)
{
    if (status == NT_OK)
        return ok();
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
    return status;
}

extern "C" {

int nt_abi_version(void) { return NT_ABI_VERSION; }

const char *nt_status_string(int status)
{
    switch (status) {
    case NT_OK:
        return "ok";
    case NT_ERR_INVALID_ARGUMENT:
        return "invalid argument";
    case NT_ERR_NULL_POINTER:
        return "null pointer";
    case NT_ERR_MISALIGNED:
        return "misaligned buffer";
    case NT_ERR_UNSUPPORTED:
        return "unsupported shape";
    case NT_ERR_WORKSPACE:
        return "workspace too small";
    case NT_ERR_HIP:
        return "HIP runtime error";
    case NT_ERR_FORMAT:
        return "bad model image";
    default:
        return "unknown status";
    }
}

const char *nt_last_error(void) { return g_error; }

int nt_set_test_hooks(int max_train_workgroups, int flags)
{
    if (max_train_workgroups < 0)
        return fail(NT_ERR_INVALID_ARGUMENT, "max_train_workgroups %d", max_train_workgroups);
    if (flags & ~(NT_HOOK_DROP_MARGINS | NT_HOOK_SORT_RANDOM))
        return fail(NT_ERR_INVALID_ARGUMENT, "test hook flags %d", flags);
    g_hook_max_workgroups.store(max_train_workgroups, std::memory_order_relaxed);
    g_hook_no_margins.store(flags & NT_HOOK_DROP_MARGINS ? 1 : 0, std::memory_order_relaxed);
    g_hook_sort_random.store(flags & NT_HOOK_SORT_RANDOM ? 1 : 0, std::memory_order_relaxed);
    return ok();
}

int nt_profile_next_launch(void *start_event, void *stop_event)
{
    g_prof_start = (hipEvent_t)start_event;
    g_prof_stop = (hipEvent_t)stop_event;
    return NT_OK;
}

int64_t nt_mip_chain_layout(int width, int height, int num_mips, int64_t *mip_offset)
{
    if (width < 1 || height < 1 || num_mips < 1 || num_mips > NT_MAX_MIPS || !mip_offset)
        return -1;
    int64_t off = 0;
    for (int m = 0; m < NT_MAX_MIPS; ++m) {
        mip_offset[m] = m < num_mips ? off : 0;
        if (m < num_mips)
            off += (int64_t)mip_dim_h(width, m) * mip_dim_h(height, m);
    }
    return off;
}

int64_t nt_block_chain_layout(int width, int height, int num_mips, int64_t *block_offset)
{
    if (width < 1 || height < 1 || num_mips < 1 || num_mips > NT_MAX_MIPS || !block_offset)
        return -1;
    int64_t off = 0;
    for (int m = 0; m < NT_MAX_MIPS; ++m) {
        block_offset[m] = m < num_mips ? off : 0;
        if (m < num_mips) {
            const int bw = mip_dim_h(width, m) >> 2, bh = mip_dim_h(height, m) >> 2;
            off += (int64_t)(bw > 0 ? bw : 1) * (bh > 0 ? bh : 1);
        }
    }
    return off;
}

size_t nt_train_workspace_bytes(const nt_params *params, nt_kernel_type type)
{
    TrainPlan plan;
    if (plan_train(params, type, &plan) != NT_OK)
        return 0;
    // Large enough for nt_inference's fixed-order SSE partials too; the update log of
    // NT_LATENT_TOUCHED after both.
    const size_t base = std::max(plan.workspace, nt_inference_workspace_bytes(params));
    const size_t mb = touched_bytes(params);
    return mb ? ((base + 255) & ~(size_t)255) + mb : base;
}

} // extern "C"

namespace {

// Scratch of nt_train_step_static: one array per GPU, held until the process ends. Host code
// never passes `scratch` itself to a kernel (in host code it names a host-side stand-in);
// it uses the device address that hipGetSymbolAddress returns for the current device.
constexpr size_t kStaticScratchBytes = (size_t)32 << 20;
__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::once_flag g_scratch_once[kMaxDevices];
void *g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

// Device address of the current device's scratch array (looked up once per device).
int static_scratch(void **ptr)
{
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return hip_status(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices)
        return fail(NT_ERR_HIP, "device %d out of range", dev);
    std::call_once(g_scratch_once[dev], [dev] {
        void *p = nullptr;
        g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? p : nullptr;
    });
    if (g_scratch_err[dev] != hipSuccess || !g_scratch_ptr[dev])
        return hip_status(g_scratch_err[dev] != hipSuccess ? g_scratch_err[dev] : hipErrorInvalidSymbol,
                          "hipGetSymbolAddress(scratch)");
    *ptr = g_scratch_ptr[dev];
    return NT_OK;
}

// With `deferred` the MLP-gradient reduction is not launched: its descriptor is returned
// for the caller's combined optimizer launch.
// The random-texel sort's buffers in the workspace (plan.sort_off != 0).
static RandomOrderDesc random_order_desc(const nt_params *p, const TrainPlan &plan, uint8_t *ws)
{
    const size_t n = (size_t)p->num_samples;
    const size_t keys = (n * 2 + 255) & ~(size_t)255, vals = (n * 4 + 255) & ~(size_t)255;
    uint8_t *b = ws + plan.sort_off;
    RandomOrderDesc r{};
    r.n = p->num_samples;
    r.step = (uint32_t)p->step;
    r.image_w = p->image_width;
    r.image_h = p->image_height;
    r.bins_x = plan.sort_bins_x;
    r.key_bits = plan.sort_key_bits;
    r.bin_shift = plan.sort_shift;
    random_order_tiles(r.n, &r.tile, &r.tiles);
    r.high_bits = random_order_high_bits(r.key_bits, r.tiles);
    r.keys = (uint16_t *)b;
    r.keys_alt = (uint16_t *)(b + keys);
    r.vals = (uint32_t *)(b + 2 * keys);
    r.vals_alt = (uint32_t *)(b + 2 * keys + vals);
    r.counts = (uint32_t *)(b + 2 * keys + 2 * vals);
    return r;
}

int train_step_with(const nt_params *p, nt_kernel_type type, void *stream, const TrainPlan &plan, uint8_t *ws,
                    UpdateLog *log, ReduceDesc *deferred = nullptr)
{
    hipStream_t s = (hipStream_t)stream;
    float *partial = (float *)(ws + plan.weight_bytes);
    hipError_t e;
    if (plan.bc6) {
        // The BC6 phase: expand the sampled levels' block records, run the unconstrained
        // step on the expanded texels, fold their gradients back into the records.
        Bc6PhaseDesc b6 = plan.bc6d;
        const int C = p->latents.channels;
        for (int k = 0; k < b6.nlevels; ++k) {
            const int gi = plan.bc6_level_grid[k], m = plan.bc6_level_mip[k];
            const nt_grid &g = p->latents.grids[gi];
            Bc6PhaseLevel &x = b6.level[k];
            const int64_t texel0 = chain_offset(g.width, g.height, m) * C;
            x.params = g.block_params + g.block_offset[m] * (4 * C + 18);
            x.grads = g.block_grads ? g.block_grads + g.block_offset[m] * (4 * C + 16) : nullptr;
            x.values = (float *)(ws + plan.bc6_values_off[gi]) + texel0;
            x.tgrads = (float *)(ws + plan.bc6_grads_off[gi]) + texel0;
        }
        // Samples at z = 0 reach mip 0 only, one level per grid: the fold logs each grid's
        // block rectangle for NT_LATENT_TOUCHED; otherwise the step logs as dense.
        const bool rects = type == NT_BLOCK_FEATURES && p->sample_mip == 0.f && b6.nlevels == p->latents.num_grids;
        b6.log = rects ? log : nullptr;
        for (int gi = 0; gi < NT_MAX_GRIDS; ++gi) {
            const bool on = rects && gi < b6.nlevels;
            const Bc6PhaseLevel &x = b6.level[on ? gi : 0];
            b6.rect[gi][0] = on ? x.bx0 : 0;
            b6.rect[gi][1] = on ? x.bx0 + x.nbx - 1 : -1;
            b6.rect[gi][2] = on ? x.by0 : 0;
            b6.rect[gi][3] = on ? x.by0 + x.nby - 1 : -1;
        }
        e = launch_bc6_expand(b6, s);
        if (e != hipSuccess)
            return hip_status(e, "BC6 expansion launch");
        const nt_params q = bc6_inner(p, plan, ws);
        TrainPlan in = plan;
        in.bc6 = 0;
        const int st = train_step_with(&q, NT_UNCONSTRAINED, stream, in, ws, nullptr, deferred);
        if (st)
            return st;
        if (type == NT_BLOCK_FEATURES) {
            e = launch_bc6_fold(b6, s);
            if (e != hipSuccess)
                return hip_status(e, "BC6 fold launch");
        }
        if (log && !b6.log) {
            e = launch_log_dense_step(log, s);
            if (e != hipSuccess)
                return hip_status(e, "update log launch");
        }
        return ok();
    }
    if (log && !(plan.use16 && type == NT_UNCONSTRAINED)) {
        // This kernel does not record its footprints: the optimizer updates every texel.
        e = launch_log_dense_step(log, s);
        if (e != hipSuccess)
            return hip_status(e, "update log launch");
    }
    if (plan.use16) {
        Train16Desc d = plan.t16;
        d.mlp = mlp_desc(&p->mlp);
        d.partial = partial;
        d.log = log;
        // The grids' arrays come from the params of this call, never from the plan: a plan
        // may be made before the arrays exist (the BC6 phase plans its inner step over
        // stand-in addresses for the workspace it has not been given yet).
        for (int gi = 0; gi < p->latents.num_grids; ++gi) {
            const nt_grid &g = p->latents.grids[gi];
            d.grid[gi].values = g.values + g.mip_offset[0] * p->latents.channels;
            d.grid[gi].grads = g.grads + g.mip_offset[0] * p->latents.channels;
        }
        for (int gi = 0; gi < NT_MAX_GRIDS && d.log; ++gi) {
            if (gi >= p->latents.num_grids) {
                d.rect[gi][0] = d.rect[gi][2] = 0;
                d.rect[gi][1] = d.rect[gi][3] = -1;
                continue;
            }
            footprint_rect(p, p->latents.grids[gi].width, p->latents.grids[gi].height, d.rect[gi]);
        }
        if (plan.sort_off) {
            // NT_SAMPLES_RANDOM: the slots' samples sorted by bin.
            e = launch_random_order(random_order_desc(p, plan, ws), s, &d.order);
            if (e != hipSuccess)
                return hip_status(e, "random-texel sample order");
        }
        {
            ProfileScope prof(s);
            e = launch_train16(plan.shape, d, plan.lds, s);
        }
        if (e != hipSuccess)
            return hip_status(e, "train kernel launch");
    } else {
    TrainDesc d{};
    d.mlp = mlp_desc(&p->mlp);
    const int C = p->latents.channels;
    for (int gi = 0; gi < p->latents.num_grids; ++gi) {
        const nt_grid &g = p->latents.grids[gi];
        d.grid[gi] = grid_desc(g, C);
        if (g.values)
            d.grid[gi].values = g.values + g.mip_offset[0] * C;
        if (g.grads)
            d.grid[gi].grads = g.grads + g.mip_offset[0] * C;
        d.grid[gi].fp_w = plan.fp_w[gi];
        d.grid[gi].fp_h = plan.fp_h[gi];
        d.grid[gi].fp_off = plan.fp_off[gi];
        d.grid[gi].vb_off = plan.vb_off[gi];
        d.grid[gi].cb_w = plan.cb_w[gi];
        d.grid[gi].cb_h = plan.cb_h[gi];
        d.grid[gi].w_row0 = plan.w_row0[gi];
    }
    const int nout = pack_targets(p->textures, p->num_textures, d.out_tex, d.out_ch, d.out_w, d.tex);
    if (nout < 0)
        return -nout;
    d.trilinear = p->sample_mip != 0.f;
    if (d.trilinear) {
        // One mip coordinate for every sample: the pairs of mips and their weights are the
        // same for the whole step (latents train.cu:266-281, targets train.cu:82-86).
        const float z = p->sample_mip, zb = floorf(z), frac = z - zb;
        const int base = (int)zb;
        for (int gi = 0; gi < p->latents.num_grids; ++gi) {
            const nt_grid &g = p->latents.grids[gi];
            GridDesc &q = d.grid[gi];
            const int top = g.num_mips - 1;
            const int m0 = std::min(base, top), m1 = std::min(base + 1, top);
            q.values = g.values + g.mip_offset[m0] * C;
            q.grads = g.grads + g.mip_offset[m0] * C;
            q.w = mip_dim_h(g.width, m0), q.h = mip_dim_h(g.height, m0);
            q.values1 = g.values + g.mip_offset[m1] * C;
            q.grads1 = g.grads + g.mip_offset[m1] * C;
            q.w1 = mip_dim_h(g.width, m1), q.h1 = mip_dim_h(g.height, m1);
            q.two_mips = frac > 0.f;
            q.mw0 = 1.f - frac;
            q.mw1 = frac;
        }
        for (int ti = 0; ti < p->num_textures && ti < NT_MAX_TEXTURES; ++ti) {
            const nt_texture &t = p->textures[ti];
            TexDesc &x = d.tex[ti];
            if (!x.texels)
                continue;
            const int top = t.num_mips > 0 ? t.num_mips - 1 : 0;
            const float mc = std::min(std::max(z, 0.f), (float)top);
            const int m0 = std::min((int)floorf(mc), top), m1 = std::min(m0 + 1, top);
            x.texels = t.texels + t.mip_offset[m0] * t.pitch;
            x.w = mip_dim_h(t.width, m0), x.h = mip_dim_h(t.height, m0);
            x.texels1 = t.texels + t.mip_offset[m1] * t.pitch;
            x.w1 = mip_dim_h(t.width, m1), x.h1 = mip_dim_h(t.height, m1);
            x.frac = m1 > m0 ? mc - (float)m0 : 0.f;
        }
    }
    d.ntex = p->num_textures;
    d.G = p->latents.num_grids;
    d.C = C;
    d.image_w = p->image_width;
    d.image_h = p->image_height;
    d.off_x = p->texel_offset_x;
    d.off_y = p->texel_offset_y;
    d.region_w = p->region_width > 0 ? p->region_width : NT_DEFAULT_REGION;
    d.num_samples = p->num_samples;
    d.step = (uint32_t)p->step;
    d.tiles_x = plan.tiles_x;
    d.chunks_per_wg = plan.chunks_per_wg;
    d.fp_floats = plan.fp_floats;
    d.fp_stride = plan.fp_stride;
    d.vbox_floats = plan.vbox_floats;
    d.vbox_off = plan.vbox_off;
    d.tile_ok = plan.tile_ok;
    d.random_texels = p->sample_mode == NT_SAMPLES_RANDOM;
    d.scatter_mfma = plan.scatter_mfma;
    d.w_rows = plan.w_rows;
    d.union_off = plan.union_off;
    d.scatter_split = plan.scatter_split;
    d.scatter_off = plan.scatter_off;
    // Workspace: weight fragments | fp32 biases | per-workgroup partials | reduction rows.
    PrepDesc prep{};
    prep.mlp = d.mlp;
    prep.frags = (uint4 *)ws;
    prep.bias = (float *)(ws + train_frag_bytes(plan.shape));
    d.wfrags = prep.frags;
    d.wbias = prep.bias;
    d.partial = partial;

    e = launch_prep_weights(plan.shape, prep, s);
    if (e != hipSuccess)
        return hip_status(e, "weight preparation launch");
    {
        ProfileScope prof(s);
        e = launch_train(plan.shape, type, d, plan.nwg, plan.lds, s);
    }
    if (e != hipSuccess)
        return hip_status(e, "train kernel launch");
    }

    ReduceDesc r{};
    r.partial = partial;
    r.rows = plan.rows;
    r.P = plan.P;
    r.num_layers = p->mlp.num_layers;
    int off = 0;
    for (int l = 0; l < p->mlp.num_layers; ++l) {
        r.off[l] = off;
        r.kin[l] = pad16(p->mlp.sizes[l]);
        r.kout[l] = pad16(p->mlp.sizes[l + 1]);
        r.nbias[l] = p->mlp.sizes[l + 1];
        r.wgrad[l] = p->mlp.weight_grads[l];
        r.bgrad[l] = p->mlp.bias_grads[l];
        off += r.kin[l] * r.kout[l] + r.kout[l];
    }
    if (deferred) {
        *deferred = r;
        return ok();
    }
    e = launch_reduce(r, s);
    if (e != hipSuccess)
        return hip_status(e, "gradient reduction launch");
    return ok();
}

} // namespace

extern "C" {

int nt_train_step(const nt_params *p, nt_kernel_type type, void *stream)
{
    TrainPlan plan;
    int st = plan_train(p, type, &plan);
    if (st)
        return st;
    const size_t mb = touched_bytes(p);
    const size_t need = mb ? ((plan.workspace + 255) & ~(size_t)255) + mb : plan.workspace;
    if (!p->workspace || p->workspace_bytes < need)
        return fail(NT_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need,
                    p->workspace ? p->workspace_bytes : (size_t)0);
    if (!aligned16(p->workspace))
        return fail(NT_ERR_MISALIGNED, "workspace must be 16-byte aligned");
    return train_step_with(p, type, stream, plan, (uint8_t *)p->workspace, update_log(p));
}

int nt_random_sample_order(const nt_params *p, uint32_t *order, void *stream)
{
    TrainPlan plan;
    int st = plan_train(p, NT_UNCONSTRAINED, &plan);
    if (st)
        return st;
    if (!order)
        return fail(NT_ERR_NULL_POINTER, "order");
    if (!plan.use16 || !plan.sort_off)
        return fail(NT_ERR_UNSUPPORTED, "these parameters train in slot order (the sort: NT_SAMPLES_RANDOM on the "
                                        "16-channel kernel, from %d samples or with NT_HOOK_SORT_RANDOM)",
                    kRandomSortMinSamples);
    if (!p->workspace || p->workspace_bytes < plan.workspace)
        return fail(NT_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", plan.workspace,
                    p->workspace ? p->workspace_bytes : (size_t)0);
    if (!aligned16(p->workspace))
        return fail(NT_ERR_MISALIGNED, "workspace must be 16-byte aligned");
    hipStream_t s = (hipStream_t)stream;
    const uint32_t *sorted = nullptr;
    hipError_t e = launch_random_order(random_order_desc(p, plan, (uint8_t *)p->workspace), s, &sorted);
    if (e == hipSuccess)
        e = hipMemcpyAsync(order, sorted, (size_t)p->num_samples * sizeof(uint32_t), hipMemcpyDeviceToDevice, s);
    if (e != hipSuccess)
        return hip_status(e, "random-texel sample order");
    return NT_OK;
}

size_t nt_train_static_scratch_bytes(void) { return kStaticScratchBytes; }

int nt_train_step_static(const nt_params *p, nt_kernel_type type, void *stream)
{
    TrainPlan plan;
    int st = plan_train(p, type, &plan);
    if (st)
        return st;
    if (p->latent_update != NT_LATENT_DENSE)
        return fail(NT_ERR_INVALID_ARGUMENT, "nt_train_step_static keeps no update log: use "
                                             "latent_update = NT_LATENT_DENSE");
    if (plan.workspace > kStaticScratchBytes)
        return fail(NT_ERR_WORKSPACE,
                    "this train step needs %zu bytes of scratch; the static scratch holds %zu (use "
                    "nt_train_step with a workspace)",
                    plan.workspace, kStaticScratchBytes);
    void *ws = nullptr;
    st = static_scratch(&ws);
    if (st)
        return st;
    return train_step_with(p, type, stream, plan, (uint8_t *)ws, nullptr);
}

static AdamDesc adam_desc(const nt_adam &a, int step)
{
    AdamDesc d;
    const int t = step > 0 ? step : 1;
    d.beta1 = a.beta1;
    d.beta2 = a.beta2;
    d.lr = a.learning_rate;
    d.eps = a.epsilon;
    d.bc1 = 1.f - powf(a.beta1, (float)t);
    d.bc2 = 1.f - powf(a.beta2, (float)t);
    return d;
}

// Validates the network optimizer's arguments and fills its descriptor.
static int net_adam_desc(const nt_params *p, NetAdamDesc &d)
{
    if (!p)
        return fail(NT_ERR_NULL_POINTER, "params is NULL");
    int shape;
    int st = check_mlp(&p->mlp, true, true, &shape);
    if (st)
        return st;
    const nt_mlp &m = p->mlp;
    d = NetAdamDesc{};
    d.a = adam_desc(p->network_adam, p->step);
    d.num_layers = m.num_layers;
    int n = 0;
    for (int l = 0; l < m.num_layers; ++l) {
        d.rows[l] = m.sizes[l];
        d.cols[l] = l == m.num_layers - 1 ? m.used_outputs : m.sizes[l + 1];
        d.pin[l] = pad16(m.sizes[l]);
        d.nbias[l] = m.sizes[l + 1];
        d.wstart[l] = n;
        n += (d.rows[l] * d.cols[l] + d.nbias[l] + 255) / 256 * 256; // layers start at whole workgroups
        d.w[l] = m.weights[l];
        d.g[l] = m.weight_grads[l];
        d.m1[l] = m.weight_moment1[l];
        d.m2[l] = m.weight_moment2[l];
        d.b[l] = m.biases[l];
        d.bg[l] = m.bias_grads[l];
        d.bm1[l] = m.bias_moment1[l];
        d.bm2[l] = m.bias_moment2[l];
    }
    d.wstart[m.num_layers] = n;
    return NT_OK;
}

int nt_optimize_network(const nt_params *p, void *stream)
{
    NetAdamDesc d;
    const int st = net_adam_desc(p, d);
    if (st)
        return st;
    return hip_status(launch_net_adam(d, (hipStream_t)stream), "network Adam launch");
}

// Validates the latent optimizer's arguments and fills its descriptor.
static int latent_adam_desc(const nt_params *p, nt_kernel_type type, LatentAdamDesc &d)
{
    if (!p)
        return fail(NT_ERR_NULL_POINTER, "params is NULL");
    if (type != NT_UNCONSTRAINED && type != NT_BLOCK_FEATURES && type != NT_FINALIZE)
        return fail(NT_ERR_INVALID_ARGUMENT, "bad kernel type %d", (int)type);
    const nt_latents &lat = p->latents;
    if (lat.num_grids < 1 || lat.num_grids > NT_MAX_GRIDS)
        return fail(NT_ERR_INVALID_ARGUMENT, "num_grids %d", lat.num_grids);
    if (lat.channels < 1 || lat.channels > 16)
        return fail(NT_ERR_INVALID_ARGUMENT, "channels %d", lat.channels);
    const int C = lat.channels;
    const bool blocks = type != NT_UNCONSTRAINED; // FINALIZE optimizes blocks too (train.cu:1018-1025)
    if (p->latent_update != NT_LATENT_DENSE && p->latent_update != NT_LATENT_TOUCHED)
        return fail(NT_ERR_INVALID_ARGUMENT, "latent_update %d", p->latent_update);
    const bool touched = p->latent_update == NT_LATENT_TOUCHED;
    UpdateLog *log = touched ? update_log(p) : nullptr;
    if (touched && !log)
        return fail(NT_ERR_WORKSPACE, "NT_LATENT_TOUCHED needs the train step's workspace");
    if (touched && !aligned16(p->workspace))
        return fail(NT_ERR_MISALIGNED, "workspace must be 16-byte aligned");
    d = LatentAdamDesc{};
    d.a = adam_desc(p->feature_adam, p->step);
    d.nseg = lat.num_grids;
    d.rec = blocks ? 4 * C + 16 : 0;
    int64_t start = 0;
    for (int gi = 0; gi < lat.num_grids; ++gi) {
        const nt_grid &g = lat.grids[gi];
        if (g.width < 1 || g.height < 1 || g.num_mips < 1 || g.num_mips > NT_MAX_MIPS)
            return fail(NT_ERR_INVALID_ARGUMENT, "grid %d: bad size or mip count", gi);
        d.start[gi] = start;
        if (!blocks) {
            // The mips must be stored back to back from mip_offset[0].
            int64_t texels = 0;
            for (int m = 0; m < g.num_mips; ++m) {
                if (g.mip_offset[m] != g.mip_offset[0] + texels)
                    return fail(NT_ERR_INVALID_ARGUMENT, "grid %d: mips are not contiguous", gi);
                texels += (int64_t)mip_dim_h(g.width, m) * mip_dim_h(g.height, m);
            }
            if (!g.values || !g.grads || !g.moment1 || !g.moment2)
                return fail(NT_ERR_NULL_POINTER, "grid %d: values/grads/moments are NULL", gi);
            const int64_t base = g.mip_offset[0] * C;
            if (!aligned16(g.values + base) || !aligned16(g.grads + base) || !aligned16(g.moment1 + base) ||
                !aligned16(g.moment2 + base))
                return fail(NT_ERR_MISALIGNED, "grid %d: latent buffers must be 16-byte aligned", gi);
            d.w[gi] = g.values + base;
            d.g[gi] = g.grads + base;
            d.m1[gi] = g.moment1 + base;
            d.m2[gi] = g.moment2 + base;
            d.n[gi] = texels * C;
            start += ((d.n[gi] + 3) / 4 + kAdamSpan - 1) / kAdamSpan * kAdamSpan; // whole workgroup spans
        } else {
            int64_t nb = 0;
            for (int m = 0; m < g.num_mips; ++m) {
                if (g.block_offset[m] != g.block_offset[0] + nb)
                    return fail(NT_ERR_INVALID_ARGUMENT, "grid %d: block mips are not contiguous", gi);
                const int bw = mip_dim_h(g.width, m) >> 2, bh = mip_dim_h(g.height, m) >> 2;
                nb += (int64_t)(bw > 0 ? bw : 1) * (bh > 0 ? bh : 1);
            }
            if (!g.block_params || !g.block_grads || !g.block_moment1 || !g.block_moment2)
                return fail(NT_ERR_NULL_POINTER, "grid %d: block buffers are NULL", gi);
            d.w[gi] = g.block_params + g.block_offset[0] * (4 * C + 18);
            d.g[gi] = g.block_grads + g.block_offset[0] * (4 * C + 16);
            d.m1[gi] = g.block_moment1 + g.block_offset[0] * (4 * C + 16);
            d.m2[gi] = g.block_moment2 + g.block_offset[0] * (4 * C + 16);
            d.n[gi] = nb;
            start += (nb + kAdamSpan - 1) / kAdamSpan * kAdamSpan;
        }
    }
    d.start[lat.num_grids] = start;
    if (touched) {
        d.log = log;
        d.C = C;
        for (int gi = 0; gi < lat.num_grids; ++gi) {
            // Block records: the logged rectangles count mip-0 blocks.
            const int w = lat.grids[gi].width, h = lat.grids[gi].height;
            d.gw[gi] = blocks ? std::max(w >> 2, 1) : w;
            d.gh[gi] = blocks ? std::max(h >> 2, 1) : h;
        }
    }
    return NT_OK;
}

int nt_optimize_latents(const nt_params *p, nt_kernel_type type, void *stream)
{
    LatentAdamDesc d;
    const int st = latent_adam_desc(p, type, d);
    if (st)
        return st;
    ProfileScope prof((hipStream_t)stream);
    return hip_status(launch_latent_adam(d, (hipStream_t)stream), "latent Adam launch");
}

// One iteration of the reference's loop body (main.cpp:1071-1076): nt_train_step, then
// nt_optimize_network, then nt_optimize_latents, with the same results. The MLP-gradient
// reduction, the network update and the latent update (texels or block records) share one
// launch after the train step. Every argument of all three is checked before anything is
// enqueued.
int nt_train_iteration(const nt_params *p, nt_kernel_type type, void *stream)
{
    TrainPlan plan;
    int st = plan_train(p, type, &plan);
    if (st)
        return st;
    const size_t mb = touched_bytes(p);
    const size_t need = mb ? ((plan.workspace + 255) & ~(size_t)255) + mb : plan.workspace;
    if (!p->workspace || p->workspace_bytes < need)
        return fail(NT_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need,
                    p->workspace ? p->workspace_bytes : (size_t)0);
    if (!aligned16(p->workspace))
        return fail(NT_ERR_MISALIGNED, "workspace must be 16-byte aligned");
    OptimizeStepDesc o{};
    NetAdamDesc net;
    st = net_adam_desc(p, net);
    if (st)
        return st;
    st = latent_adam_desc(p, type, o.lat);
    if (st)
        return st;
    o.net.a = net.a;
    for (int l = 0; l < net.num_layers; ++l) {
        o.net.rows[l] = net.rows[l];
        o.net.cols[l] = net.cols[l];
        o.net.w[l] = net.w[l];
        o.net.b[l] = net.b[l];
        o.net.m1[l] = net.m1[l];
        o.net.m2[l] = net.m2[l];
        o.net.bm1[l] = net.bm1[l];
        o.net.bm2[l] = net.bm2[l];
    }
    // The latent update's grid, sized for the rectangles this step logs (a logged step's
    // work: 512 items per workgroup pass for texels, 256 record floats for block records).
    if (p->latent_update == NT_LATENT_TOUCHED) {
        int64_t items = 0;
        if (plan.bc6 && type == NT_BLOCK_FEATURES && p->sample_mip == 0.f) {
            for (int k = 0; k < plan.bc6d.nlevels; ++k)
                items += (int64_t)plan.bc6d.level[k].nbx * plan.bc6d.level[k].nby * (4 * p->latents.channels + 16);
            o.lat_wg = (int)std::min<int64_t>((items + 255) / 256, 8192);
        } else if (!plan.bc6 && plan.use16 && type == NT_UNCONSTRAINED &&
                   (p->latents.channels == 16 || p->latents.channels == 3)) {
            for (int gi = 0; gi < p->latents.num_grids; ++gi) {
                int r[4];
                footprint_rect(p, p->latents.grids[gi].width, p->latents.grids[gi].height, r);
                items += (int64_t)(r[1] - r[0] + 1) * (r[3] - r[2] + 1) * (p->latents.channels == 16 ? 4 : 1);
            }
            o.lat_wg = (int)std::min<int64_t>((items + 511) / 512, 8192);
        }
    }
    st = train_step_with(p, type, stream, plan, (uint8_t *)p->workspace, update_log(p), &o.red);
    if (st)
        return st;
    return hip_status(launch_optimize_step(o, (hipStream_t)stream), "optimizer launch");
}

static int fwd_common(const nt_latents *lat, const nt_mlp *mlp, bool need_latents, FwdDesc *d,
                      int *shape)
{
    int st = check_mlp(mlp, false, false, shape);
    if (st)
        return st;
    *d = FwdDesc{};
    d->mlp = mlp_desc(mlp);
    if (need_latents) {
        st = check_latents(lat, *shape, false, false);
        if (st)
            return st;
        if (lat->num_grids * lat->channels != mlp->sizes[0])
            return fail(NT_ERR_INVALID_ARGUMENT, "MLP input %d != num_grids*channels %d", mlp->sizes[0],
                        lat->num_grids * lat->channels);
        d->G = lat->num_grids;
        d->C = lat->channels;
        for (int gi = 0; gi < lat->num_grids; ++gi)
            d->grid[gi] = grid_desc(lat->grids[gi], lat->channels);
    }
    return NT_OK;
}

int nt_inference(const nt_params *p, void *stream)
{
    if (!p)
        return fail(NT_ERR_NULL_POINTER, "params is NULL");
    if (!p->inference_output || !p->inference_mse_accum)
        return fail(NT_ERR_NULL_POINTER, "inference_output / inference_mse_accum are NULL");
    if (p->image_width < 1 || p->image_height < 1)
        return fail(NT_ERR_INVALID_ARGUMENT, "image size %dx%d", p->image_width, p->image_height);
    if ((int64_t)p->image_width * p->image_height > (1ll << 31) - 64)
        return fail(NT_ERR_INVALID_ARGUMENT, "image too large");
    FwdDesc d;
    int shape;
    int st = fwd_common(&p->latents, &p->mlp, true, &d, &shape);
    if (st)
        return st;
    float dummy_w[NT_MAX_OUTPUTS];
    const int nout = pack_targets(p->textures, p->num_textures, d.out_tex, d.out_ch, dummy_w, d.tex);
    if (nout < 0)
        return -nout;
    d.ntex = p->num_textures;
    d.count = p->image_width * p->image_height;
    d.image_w = p->image_width;
    d.image_h = p->image_height;
    d.inv_w = pow2_reciprocal(d.image_w);
    d.inv_h = pow2_reciprocal(d.image_h);
    d.out32 = p->inference_output;
    d.sse = p->inference_mse_accum;
    d.out_stride = p->mlp.sizes[p->mlp.num_layers];
    const int partials = forward_blocks(d.count) * kFwdWaves;
    if (p->workspace && p->workspace_bytes >= (size_t)partials * sizeof(float)) {
        if (!aligned16(p->workspace))
            return fail(NT_ERR_MISALIGNED, "workspace must be 16-byte aligned");
        d.sse_partial = (float *)p->workspace;
    }
    hipError_t e;
    {
        ProfileScope prof((hipStream_t)stream);
        e = launch_forward(shape, kFwdInference, d, (hipStream_t)stream);
    }
    if (e == hipSuccess && d.sse_partial)
        e = launch_sse_reduce(d.sse_partial, partials, d.sse, (hipStream_t)stream);
    return hip_status(e, "inference launch");
}

size_t nt_inference_workspace_bytes(const nt_params *p)
{
    if (!p || p->image_width < 1 || p->image_height < 1 ||
        (int64_t)p->image_width * p->image_height > (1ll << 31) - 64)
        return 0;
    return (size_t)forward_blocks(p->image_width * p->image_height) * kFwdWaves * sizeof(float);
}

int nt_mlp_forward(const nt_mlp *mlp, const uint16_t *inputs, uint16_t *outputs, int count, void *stream)
{
    if (!inputs || !outputs)
        return fail(NT_ERR_NULL_POINTER, "inputs/outputs are NULL");
    if (count < 0)
        return fail(NT_ERR_INVALID_ARGUMENT, "count %d", count);
    FwdDesc d;
    int shape;
    int st = fwd_common(nullptr, mlp, false, &d, &shape);
    if (st)
        return st;
    if (count == 0)
        return ok();
    d.count = count;
    d.inputs = inputs;
    d.out16 = outputs;
    d.out_stride = mlp->sizes[mlp->num_layers];
    ProfileScope prof((hipStream_t)stream);
    return hip_status(launch_forward(shape, kFwdMlp, d, (hipStream_t)stream), "MLP forward launch");
}

int nt_forward(const nt_latents *latents, const nt_mlp *mlp, nt_filter filter, const float *uvz, int count,
               uint16_t *features, uint16_t *outputs, void *stream)
{
    if (!uvz || !outputs)
        return fail(NT_ERR_NULL_POINTER, "uvz/outputs are NULL");
    if (count < 0)
        return fail(NT_ERR_INVALID_ARGUMENT, "count %d", count);
    if (filter != NT_FILTER_BILINEAR && filter != NT_FILTER_CATMULL_ROM)
        return fail(NT_ERR_INVALID_ARGUMENT, "bad filter %d", (int)filter);
    FwdDesc d;
    int shape;
    int st = fwd_common(latents, mlp, true, &d, &shape);
    if (st)
        return st;
    if (count == 0)
        return ok();
    d.count = count;
    d.uvz = uvz;
    d.features = features;
    d.out16 = outputs;
    d.out_stride = mlp->sizes[mlp->num_layers];
    const int mode = filter == NT_FILTER_BILINEAR ? kFwdBilinear : kFwdCatmullRom;
    ProfileScope prof((hipStream_t)stream);
    return hip_status(launch_forward(shape, mode, d, (hipStream_t)stream), "forward launch");
}

int nt_bc6_init(const nt_latents *lat, void *stream)
{
    if (!lat)
        return fail(NT_ERR_NULL_POINTER, "latents is NULL");
    const int C = lat->channels;
    if (C != 3 && C != 4 && C != 8 && C != 16)
        return fail(NT_ERR_UNSUPPORTED, "channels %d (3, 4, 8 or 16)", C);
    if (lat->num_grids < 1 || lat->num_grids > NT_MAX_GRIDS)
        return fail(NT_ERR_INVALID_ARGUMENT, "num_grids %d outside [1, %d]", lat->num_grids, NT_MAX_GRIDS);
    Bc6InitDesc d{};
    d.C = C;
    int64_t start = 0;
    for (int gi = 0; gi < lat->num_grids; ++gi) {
        const nt_grid &g = lat->grids[gi];
        if (g.width < 1 || g.height < 1 || g.num_mips < 1 || g.num_mips > NT_MAX_MIPS)
            return fail(NT_ERR_INVALID_ARGUMENT, "grid %d: bad size %dx%d or mip count %d", gi, g.width, g.height,
                        g.num_mips);
        if ((g.width & 3 && g.width > 4) || (g.height & 3 && g.height > 4))
            return fail(NT_ERR_INVALID_ARGUMENT, "grid %d: block storage needs sizes multiple of 4", gi);
        if (!g.values || !g.block_params)
            return fail(NT_ERR_NULL_POINTER, "grid %d: values/block_params are NULL", gi);
        if (((uintptr_t)g.values & 3u) || ((uintptr_t)g.block_params & 3u))
            return fail(NT_ERR_MISALIGNED, "grid %d: values/block_params must be 4-byte aligned", gi);
        for (int m = 0; m < g.num_mips; ++m) {
            if (g.mip_offset[m] < 0 || g.block_offset[m] < 0)
                return fail(NT_ERR_INVALID_ARGUMENT, "grid %d: negative offset at mip %d", gi, m);
            const int w = mip_dim_h(g.width, m), h = mip_dim_h(g.height, m);
            const int nbu = std::max(w >> 2, 1), nbv = std::max(h >> 2, 1);
            const int k = d.levels++;
            d.values[k] = g.values + g.mip_offset[m] * C;
            d.blocks[k] = g.block_params + g.block_offset[m] * (4 * C + 18);
            d.w[k] = w;
            d.h[k] = h;
            d.nbu[k] = nbu;
            d.start[k] = start;
            start += (int64_t)nbu * nbv;
        }
    }
    d.start[d.levels] = start;
    ProfileScope prof((hipStream_t)stream);
    return hip_status(launch_bc6_init(d, (hipStream_t)stream), "BC6 init launch");
}

size_t nt_codec_block_bytes(int channels)
{
    if (channels < 4 || channels > 16 || channels % 4)
        return 0;
    return (size_t)12 * channels;
}

size_t nt_codec_mip_chain_layout(int width, int height, int num_mips, int channels, int64_t *byte_offset)
{
    const size_t rec = nt_codec_block_bytes(channels);
    if (!rec || width < 1 || height < 1 || num_mips < 1 || num_mips > NT_MAX_MIPS || !byte_offset)
        return 0;
    size_t off = 0;
    for (int m = 0; m < NT_MAX_MIPS; ++m) {
        byte_offset[m] = m < num_mips ? (int64_t)off : 0;
        if (m < num_mips) {
            const int w = mip_dim_h(width, m), h = mip_dim_h(height, m);
            off += (size_t)((w + 3) / 4) * ((h + 3) / 4) * rec;
        }
    }
    return off;
}

int nt_codec_encode(const float *values, int width, int height, int channels, void *blocks, void *stream)
{
    if (!values || !blocks)
        return fail(NT_ERR_NULL_POINTER, "values/blocks are NULL");
    if (width < 1 || height < 1 || !nt_codec_block_bytes(channels) || (int64_t)width * channels >= (1ll << 31))
        return fail(NT_ERR_INVALID_ARGUMENT, "size %dx%d, channels %d (need 4, 8, 12 or 16)", width, height,
                    channels);
    if (((uintptr_t)blocks & 3u) || ((uintptr_t)values & 3u))
        return fail(NT_ERR_MISALIGNED, "values/blocks must be 4-byte aligned");
    ProfileScope prof((hipStream_t)stream);
    return hip_status(launch_codec_encode(values, width, height, channels, (uint8_t *)blocks, (hipStream_t)stream),
                      "codec encode launch");
}

int nt_codec_decode(const void *blocks, int width, int height, int channels, float *values, void *stream)
{
    if (!values || !blocks)
        return fail(NT_ERR_NULL_POINTER, "values/blocks are NULL");
    if (width < 1 || height < 1 || !nt_codec_block_bytes(channels) || (int64_t)width * channels >= (1ll << 31))
        return fail(NT_ERR_INVALID_ARGUMENT, "size %dx%d, channels %d (need 4, 8, 12 or 16)", width, height,
                    channels);
    if (!aligned16(blocks) || !aligned16(values))
        return fail(NT_ERR_MISALIGNED, "values/blocks must be 16-byte aligned");
    ProfileScope prof((hipStream_t)stream);
    return hip_status(
        launch_codec_decode((const uint8_t *)blocks, width, height, channels, values, (hipStream_t)stream),
        "codec decode launch");
}

// Workspace of the two-pass decode: per grid its fp16 texel chain (32 bytes per texel at
// 16 channels), each segment 256-byte aligned.
static size_t decode_workspace_layout(const nt_decode_params *p, size_t *seg_off)
{
    size_t off = 0;
    for (int gi = 0; gi < p->num_grids; ++gi) {
        const nt_codec_grid &g = p->grids[gi];
        int64_t mip_off[NT_MAX_MIPS];
        const int64_t texels = nt_mip_chain_layout(g.width, g.height, g.num_mips, mip_off);
        if (texels < 0)
            return 0;
        if (seg_off)
            seg_off[gi] = off;
        off += (((size_t)texels * (size_t)p->channels * 2) + 255) & ~(size_t)255;
    }
    return off;
}

// LDS boxes of the staged decode: for every grid the mips its pixels can sample (z ranges
// over [mip_min, mip_max] as the kernel computes it), and for each the largest box any
// block needs (footprint origins of a block's lowest and highest sample positions, plus the
// bilinear neighbour). False when the boxes exceed kBoxMaxBytes.
static bool plan_decode_box(const nt_decode_params *p, const FwdDesc &fd, int shape, DecodeBoxDesc *b)
{
    *b = DecodeBoxDesc{};
    b->mlp = fd.mlp;
    b->G = p->num_grids;
    b->image_w = p->out_width;
    b->image_h = p->out_height;
    b->inv_w = pow2_reciprocal(b->image_w);
    b->inv_h = pow2_reciprocal(b->image_h);
    b->blocks_x = (p->out_width + kBoxBlockW - 1) / kBoxBlockW;
    b->blocks_y = (p->out_height + kBoxBlockH - 1) / kBoxBlockH;
    b->out16 = p->output;
    b->out_stride = fd.out_stride;
    b->seed = p->seed;
    b->jitter = p->jitter;
    b->mip_min = p->mip_min;
    b->mip_max = p->mip_max;
    const float dz = p->mip_max - p->mip_min;
    const float za = fmaf(dz, 0.f, p->mip_min), zb = fmaf(dz, 1.f - 0x1p-24f, p->mip_min);
    const float zlo = std::min(za, zb), zhi = std::max(za, zb);
    if (!std::isfinite(zlo) || !std::isfinite(zhi) || !std::isfinite(p->jitter))
        return false;
    int texels = 0;
    for (int gi = 0; gi < p->num_grids; ++gi) {
        BoxGrid &q = b->grid[gi];
        q.texels = fd.half_values[gi];
        q.w = fd.grid[gi].w;
        q.h = fd.grid[gi].h;
        q.num_mips = fd.grid[gi].num_mips;
        for (int m = 0; m < NT_MAX_MIPS; ++m)
            q.mip_off[m] = fd.grid[gi].mip_off[m];
        const int top = q.num_mips - 1;
        const float fl = floorf(zlo), fh = floorf(zhi);
        q.mip_lo = (int)std::min(std::max(fl, 0.f), (float)top);
        q.mip_hi = (int)std::min(std::max(fh + (zhi > fh ? 1.f : 0.f), 0.f), (float)top);
        for (int m = q.mip_lo; m <= q.mip_hi; ++m) {
            const int w = mip_dim_h(q.w, m), h = mip_dim_h(q.h, m);
            int bw = 2, bh = 2;
            for (int bx = 0; bx < b->blocks_x; ++bx) {
                const int x0 = bx * kBoxBlockW, x1 = std::min(x0 + kBoxBlockW, p->out_width) - 1;
                bw = std::max(bw, box_last(x1, p->out_width, p->jitter, w) -
                                      box_origin(x0, p->out_width, p->jitter, w) + 2);
            }
            for (int by = 0; by < b->blocks_y; ++by) {
                const int y0 = by * kBoxBlockH, y1 = std::min(y0 + kBoxBlockH, p->out_height) - 1;
                bh = std::max(bh, box_last(y1, p->out_height, p->jitter, h) -
                                      box_origin(y0, p->out_height, p->jitter, h) + 2);
            }
            // The kernel packs a mip's dimensions into 16 bits each.
            if (bw > 0xFFFF || bh > 0x7FFF || (int64_t)bw * bh * 32 > kBoxMaxBytes || w > 0xFFFF || h > 0xFFFF)
                return false;
            q.box_w[m] = bw;
            q.box_h[m] = bh;
            q.box_off[m] = texels;
            texels += bw * bh;
            if ((int64_t)texels * 32 > kBoxMaxBytes)
                return false;
        }
    }
    b->box_texels = texels;
    b->lds_box_off = (int)((decode_box_weight_bytes(shape) + 15) & ~(size_t)15);
    return b->lds_box_off > 0;
}

size_t nt_decode_workspace_bytes(const nt_decode_params *p)
{
    if (!p || p->channels != 16 || p->num_grids < 1 || p->num_grids > NT_MAX_GRIDS) {
        fail(NT_ERR_INVALID_ARGUMENT, "the two-pass decode needs 1..4 grids of 16 channels");
        return 0;
    }
    return decode_workspace_layout(p, nullptr);
}

int nt_decode(const nt_decode_params *p, void *stream)
{
    if (!p)
        return fail(NT_ERR_NULL_POINTER, "params is NULL");
    if (!p->output)
        return fail(NT_ERR_NULL_POINTER, "output is NULL");
    if (p->out_width < 1 || p->out_height < 1 || (int64_t)p->out_width * p->out_height > (1ll << 31) - 64)
        return fail(NT_ERR_INVALID_ARGUMENT, "output size %dx%d", p->out_width, p->out_height);
    FwdDesc d;
    int shape;
    int st = fwd_common(nullptr, &p->mlp, false, &d, &shape);
    if (st)
        return st;
    const int C = shape_channels(shape);
    if (C != 16 && C != 8)
        return fail(NT_ERR_UNSUPPORTED, "decode is built for 8 or 16 channels per grid");
    if (p->channels != C)
        return fail(NT_ERR_UNSUPPORTED, "this MLP shape decodes %d channels per grid, got %d", C, p->channels);
    if (p->num_grids < 1 || p->num_grids > NT_MAX_GRIDS || p->num_grids * p->channels != p->mlp.sizes[0])
        return fail(NT_ERR_INVALID_ARGUMENT, "num_grids %d x channels %d != MLP input %d", p->num_grids,
                    p->channels, p->mlp.sizes[0]);
    if (p->mlp.used_outputs < 1)
        return fail(NT_ERR_INVALID_ARGUMENT, "used_outputs must be >= 1");
    for (int gi = 0; gi < p->num_grids; ++gi) {
        const nt_codec_grid &g = p->grids[gi];
        if (!g.blocks)
            return fail(NT_ERR_NULL_POINTER, "grid %d blocks are NULL", gi);
        if (g.width < 1 || g.height < 1 || g.num_mips < 1 || g.num_mips > NT_MAX_MIPS)
            return fail(NT_ERR_INVALID_ARGUMENT, "grid %d: bad size or mip count", gi);
        for (int m = 0; m < g.num_mips; ++m)
            if (!aligned16((const uint8_t *)g.blocks + g.byte_offset[m]))
                return fail(NT_ERR_MISALIGNED, "grid %d mip %d blocks must be 16-byte aligned", gi, m);
        d.cgrid[gi].blocks = (const uint8_t *)g.blocks;
        d.cgrid[gi].w = g.width;
        d.cgrid[gi].h = g.height;
        d.cgrid[gi].num_mips = g.num_mips;
        d.grid[gi].w = g.width;
        d.grid[gi].h = g.height;
        d.grid[gi].num_mips = g.num_mips;
        for (int m = 0; m < NT_MAX_MIPS; ++m)
            d.cgrid[gi].byte_off[m] = g.byte_offset[m];
    }
    d.G = p->num_grids;
    d.C = p->channels;
    d.count = p->out_width * p->out_height;
    d.image_w = p->out_width;
    d.image_h = p->out_height;
    d.inv_w = pow2_reciprocal(d.image_w);
    d.inv_h = pow2_reciprocal(d.image_h);
    d.out16 = p->output;
    d.out_stride = p->mlp.used_outputs;
    d.seed = p->seed;
    d.jitter = p->jitter;
    d.mip_min = p->mip_min;
    d.mip_max = p->mip_max;
    hipStream_t s = (hipStream_t)stream;
    if (p->workspace) {
        // Two passes: expand every block once into fp16 texels, then sample those.
        if (C != 16)
            return fail(NT_ERR_UNSUPPORTED, "the two-pass decode is built for 16 channels per grid");
        size_t seg[NT_MAX_GRIDS];
        const size_t need = decode_workspace_layout(p, seg);
        if (p->workspace_bytes < need)
            return fail(NT_ERR_WORKSPACE, "decode workspace of %zu bytes needed, %zu given", need,
                        p->workspace_bytes);
        if (!aligned16(p->workspace))
            return fail(NT_ERR_MISALIGNED, "decode workspace must be 16-byte aligned");
        CodecExpandDesc x{};
        int64_t items = 0;
        for (int gi = 0; gi < p->num_grids; ++gi) {
            const nt_codec_grid &g = p->grids[gi];
            uint16_t *chain = (uint16_t *)((uint8_t *)p->workspace + seg[gi]);
            nt_mip_chain_layout(g.width, g.height, g.num_mips, d.grid[gi].mip_off);
            d.grid[gi].w = g.width;
            d.grid[gi].h = g.height;
            d.grid[gi].num_mips = g.num_mips;
            d.half_values[gi] = chain;
            for (int m = 0; m < g.num_mips; ++m) {
                const int k = x.levels++;
                const int w = std::max(g.width >> m, 1), h = std::max(g.height >> m, 1);
                x.w[k] = w;
                x.blocks[k] = (const uint8_t *)g.blocks + g.byte_offset[m];
                x.out[k] = chain + d.grid[gi].mip_off[m] * 16;
                x.start[k] = items;
                items += (int64_t)w * h * 2;
            }
        }
        x.start[x.levels] = items;
        hipError_t e = launch_codec_expand(x, s);
        if (e != hipSuccess)
            return hip_status(e, "decode expand launch");
        DecodeBoxDesc b;
        if (plan_decode_box(p, d, shape, &b)) {
            ProfileScope prof(s);
            return hip_status(launch_decode_box(shape, b, s), "decode launch");
        }
        ProfileScope prof(s);
        return hip_status(launch_forward(shape, kFwdDecode16, d, s), "decode launch");
    }
    ProfileScope prof(s);
    return hip_status(launch_forward(shape, kFwdDecode, d, s), "decode launch");
}

} // extern "C"
