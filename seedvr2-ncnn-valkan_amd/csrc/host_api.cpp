// Host half of the C ABI: window plans, RoPE tables, error strings.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "sv2_internal.h"

namespace sv2
{

namespace
{
thread_local std::string g_last_error = "no error";

inline int ceil_div(int value, int divisor)
{
    return (value + divisor - 1) / divisor;
}

// Adaptive window extents (seedvr2_dit_block.cpp:832-838): about 3600 latent
// pixels per frame group, three windows per spatial axis, frames in fours
// (capped at 30).  nearbyint rounds ties to even like Python's round.
void adaptive_window(int T, int H, int W, int* wt, int* wh, int* ww)
{
    const double scale = std::sqrt(3600.0 / static_cast<double>(H * W));
    const int resized_h = static_cast<int>(std::nearbyint(H * scale));
    const int resized_w = static_cast<int>(std::nearbyint(W * scale));
    *wh = ceil_div(resized_h, 3);
    *ww = ceil_div(resized_w, 3);
    *wt = ceil_div(std::min(T, 30), 4);
}

// One axis of seedvr2_dit_block.cpp:840-866: shift by half a window when the
// window is smaller than the extent, count, then the truncating interval
// bounds.  Appends the interval list in loop order, empty ones included, so
// the caller can reproduce the reference's skip rule.
void axis_intervals(int extent, int window, bool shifted, std::vector<int>* lo, std::vector<int>* hi)
{
    const double shift = shifted && window < extent ? 0.5 : 0.0;
    const int count = shifted
                          ? (shift > 0.0 ? static_cast<int>(std::ceil((extent - shift) / window)) + 1 : 1)
                          : ceil_div(extent, window);
    for (int i = 0; i < count; i++)
    {
        lo->push_back(std::max(static_cast<int>((i - shift) * window), 0));
        hi->push_back(std::min(static_cast<int>((i - shift + 1.0) * window), extent));
    }
}

int validate_rule(const sv2_window_rule& rule)
{
    if (rule.frames <= 0 || rule.height <= 0 || rule.width <= 0)
        return set_error(SV2_EINVAL, "window rule: frames/height/width must be positive");
    if (rule.wt < 0 || rule.wh < 0 || rule.ww < 0)
        return set_error(SV2_EINVAL, "window rule: window extents must be >= 0 (0 = adaptive)");
    if (static_cast<int64_t>(rule.frames) * rule.height * rule.width > (int64_t(1) << 30))
        return set_error(SV2_EUNSUPPORTED, "window rule: grid too large");
    return SV2_OK;
}

void rule_extents(const sv2_window_rule& rule, int* wt, int* wh, int* ww)
{
    int at, ah, aw;
    adaptive_window(rule.frames, rule.height, rule.width, &at, &ah, &aw);
    *wt = rule.wt > 0 ? rule.wt : at;
    *wh = rule.wh > 0 ? rule.wh : ah;
    *ww = rule.ww > 0 ? rule.ww : aw;
}

// Keeps the non-empty intervals of one axis and checks they partition
// [0, extent) in order (true for this rule: consecutive intervals share their
// bounds, the first starts at or below 0 and the last ends at or past extent).
int compress_axis(const std::vector<int>& lo, const std::vector<int>& hi, int extent, AxisPlan* axis)
{
    axis->n = 0;
    int expect = 0;
    for (size_t i = 0; i < lo.size(); i++)
    {
        if (hi[i] <= lo[i])
            continue;
        if (lo[i] != expect)
            return set_error(SV2_EUNSUPPORTED, "window plan: axis intervals do not tile the grid");
        if (axis->n >= kMaxAxisIntervals)
            return set_error(SV2_EUNSUPPORTED, "window plan: more than 48 windows along one axis");
        axis->b[axis->n] = lo[i];
        axis->n++;
        expect = hi[i];
    }
    if (expect != extent || axis->n == 0)
        return set_error(SV2_EUNSUPPORTED, "window plan: axis intervals do not cover the grid");
    axis->b[axis->n] = extent;
    return SV2_OK;
}
} // namespace

int set_error(int code, const std::string& message)
{
    g_last_error = message;
    return code;
}

int caught_exception(const char* entry) noexcept
{
    std::string what;
    try
    {
        throw;
    }
    catch (const std::bad_alloc&)
    {
        what = "out of host memory";
    }
    catch (const std::exception& e)
    {
        what = e.what();
    }
    catch (...)
    {
        what = "unknown exception";
    }
    try
    {
        return set_error(SV2_EDEVICE, std::string(entry) + ": " + what);
    }
    catch (...)
    {
        return SV2_EDEVICE; // no memory left even for the message
    }
}

int hip_error(hipError_t err, const char* what)
{
    char buffer[256];
    std::snprintf(buffer, sizeof(buffer), "%s: %s", what, hipGetErrorString(err));
    return set_error(SV2_EDEVICE, buffer);
}

int set_dynamic_lds(const void* kernel, int bytes, const char* what)
{
    static std::mutex lock;
    static std::map<std::pair<const void*, int>, int> done; // (kernel, device) -> limit set
    int device = 0;
    hipError_t err = hipGetDevice(&device);
    if (err != hipSuccess)
        return hip_error(err, what);
    std::lock_guard<std::mutex> guard(lock);
    int& limit = done[std::make_pair(kernel, device)];
    if (limit >= bytes)
        return SV2_OK;
    err = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (err != hipSuccess)
        return hip_error(err, what);
    limit = bytes;
    return SV2_OK;
}

int build_plan(const sv2_window_rule& rule, PlanArgs* plan)
{
    int rc = validate_rule(rule);
    if (rc != SV2_OK)
        return rc;
    int wt, wh, ww;
    rule_extents(rule, &wt, &wh, &ww);
    std::vector<int> lo_t, hi_t, lo_h, hi_h, lo_w, hi_w;
    axis_intervals(rule.frames, wt, rule.shifted != 0, &lo_t, &hi_t);
    axis_intervals(rule.height, wh, rule.shifted != 0, &lo_h, &hi_h);
    axis_intervals(rule.width, ww, rule.shifted != 0, &lo_w, &hi_w);
    std::memset(plan, 0, sizeof(*plan));
    if ((rc = compress_axis(lo_t, hi_t, rule.frames, &plan->t)) != SV2_OK)
        return rc;
    if ((rc = compress_axis(lo_h, hi_h, rule.height, &plan->h)) != SV2_OK)
        return rc;
    if ((rc = compress_axis(lo_w, hi_w, rule.width, &plan->w)) != SV2_OK)
        return rc;
    plan->T = rule.frames;
    plan->H = rule.height;
    plan->W = rule.width;
    plan->nwin = plan->t.n * plan->h.n * plan->w.n;
    return SV2_OK;
}

} // namespace sv2

extern "C" {

int sv2_window_plan(const sv2_window_rule* rule, sv2_window* out, int cap)
try
{
    using namespace sv2;
    if (!rule || cap < 0 || (cap > 0 && !out))
        return set_error(SV2_EINVAL, "sv2_window_plan: null argument");
    PlanArgs plan;
    const int rc = build_plan(*rule, &plan);
    if (rc != SV2_OK)
        return rc;
    const int n = std::min(cap, plan.nwin);
    for (int wi = 0; wi < n; wi++)
    {
        const WindowBox b = window_box(plan, wi);
        out[wi].t0 = b.t0;
        out[wi].t1 = b.t1;
        out[wi].h0 = b.h0;
        out[wi].h1 = b.h1;
        out[wi].w0 = b.w0;
        out[wi].w1 = b.w1;
    }
    return plan.nwin;
}
catch (...)
{
    return sv2::caught_exception("sv2_window_plan");
}

size_t sv2_rope_table_floats(int npos)
{
    return npos > 0 ? static_cast<size_t>(3) * npos * sv2::kRopePairSlots * 2 : 0;
}

int sv2_rope_table_build(int rope_mode, const float* freqs, float theta, int npos, float* host_table)
try
{
    using namespace sv2;
    if (npos <= 0 || !host_table)
        return set_error(SV2_EINVAL, "sv2_rope_table_build: bad table size or null table");
    int pairs[3] = {0, 0, 0};
    float freq[3][kRopePairSlots] = {};
    if (rope_mode == SV2_ROPE_REFERENCE)
    {
        if (!freqs)
            return set_error(SV2_EINVAL, "sv2_rope_table_build: reference mode needs rope_freqs");
        for (int a = 0; a < 3; a++)
        {
            pairs[a] = 21;
            for (int p = 0; p < 21; p++)
                freq[a][p] = freqs[p];
        }
    }
    else if (rope_mode == SV2_ROPE_ABSOLUTE)
    {
        if (!(theta > 0.f))
            return set_error(SV2_EINVAL, "sv2_rope_table_build: theta must be positive");
        const int dims[3] = {32, 48, 48};
        for (int a = 0; a < 3; a++)
        {
            pairs[a] = dims[a] / 2;
            for (int p = 0; p < pairs[a]; p++)
                freq[a][p] = static_cast<float>(1.0 / std::pow(static_cast<double>(theta), (2.0 * p) / dims[a]));
        }
    }
    else if (rope_mode != SV2_ROPE_NONE)
    {
        return set_error(SV2_EINVAL, "sv2_rope_table_build: unknown rope mode");
    }
    for (int a = 0; a < 3; a++)
        for (int pos = 0; pos < npos; pos++)
            for (int p = 0; p < kRopePairSlots; p++)
            {
                float* slot = host_table + ((static_cast<size_t>(a) * npos + pos) * kRopePairSlots + p) * 2;
                if (p >= pairs[a])
                {
                    // unused slots rotate by zero: dims the variant leaves
                    // unrotated (126, 127 of the reference layout) read one
                    slot[0] = 1.f;
                    slot[1] = 0.f;
                    continue;
                }
                // float(pos) * freq in fp32, then the C library's cosf / sinf:
                // the reference evaluates std::cos / std::sin of that float
                const float angle = static_cast<float>(pos) * freq[a][p];
                slot[0] = std::cos(angle);
                slot[1] = std::sin(angle);
            }
    return SV2_OK;
}
catch (...)
{
    return sv2::caught_exception("sv2_rope_table_build");
}

int sv2_rope_positions_needed(const sv2_window_rule* rule, int text_len, int rope_mode)
try
{
    using namespace sv2;
    if (!rule || text_len < 0)
        return set_error(SV2_EINVAL, "sv2_rope_positions_needed: bad argument");
    PlanArgs plan;
    const int rc = build_plan(*rule, &plan);
    if (rc != SV2_OK)
        return rc;
    if (rope_mode == SV2_ROPE_NONE)
        return 1;
    if (rope_mode == SV2_ROPE_ABSOLUTE)
        return std::max(rule->frames, std::max(rule->height, rule->width));
    int max_t = 0, max_h = 0, max_w = 0;
    for (int i = 0; i < plan.t.n; i++)
        max_t = std::max(max_t, plan.t.b[i + 1] - plan.t.b[i]);
    for (int i = 0; i < plan.h.n; i++)
        max_h = std::max(max_h, plan.h.b[i + 1] - plan.h.b[i]);
    for (int i = 0; i < plan.w.n; i++)
        max_w = std::max(max_w, plan.w.b[i + 1] - plan.w.b[i]);
    // video positions (L_txt + t_local, y_local, x_local); text (l, l, l)
    return std::max(std::max(text_len + max_t, text_len), std::max(max_h, max_w));
}
catch (...)
{
    return sv2::caught_exception("sv2_rope_positions_needed");
}

const char* sv2_last_error(void)
{
    return sv2::g_last_error.c_str();
}

const char* sv2_version(void)
{
    return "seedvr2-hip 0.1 gfx950";
}

} // extern "C"
