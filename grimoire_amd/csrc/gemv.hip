// gemv.hip -- host planning and format dispatch of the decode kernel
// (kernels in gemv_impl.hpp, one translation unit per weight format).
#include <algorithm>

#include "gemv.hpp"

namespace grim {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kRuGU = 2;
constexpr int kPairsDN = 2;

hipError_t decode_launch_fmt_0(hipStream_t, const DecodeArgs&);
hipError_t decode_launch_fmt_3(hipStream_t, const DecodeArgs&);
hipError_t decode_launch_fmt_4(hipStream_t, const DecodeArgs&);
hipError_t decode_launch_fmt_6(hipStream_t, const DecodeArgs&);
hipError_t decode_launch_fmt_64(hipStream_t, const DecodeArgs&);

// ------------------------------------------------------------------ host

static int pow2_at_least(int v, int lo, int hi) {
    int l = lo;
    while (l < hi && l < v) l <<= 1;
    return l;
}

int chunk_elems(int fmt) {
    switch (fmt) {
    case GRIM_FMT_BF16: return Chunk<GRIM_FMT_BF16>::CH;
    case GRIM_FMT_INT8: return Chunk<GRIM_FMT_INT8>::CH;
    case GRIM_FMT_INT4:
    case GRIM_FMT_INT4_F16: return Chunk<GRIM_FMT_INT4>::CH;
    case GRIM_FMT_MXFP4: return Chunk<GRIM_FMT_MXFP4>::CH;
    }
    return 0;
}

// gate_up: full waves per row while there are >= 64 chunks, else the
// smallest group covering the row.  down: about three chunks per lane.
static int lpr_gate_up(int chunks) { return pow2_at_least(chunks, 8, 64); }
static int lpr_down(int chunks) { return pow2_at_least((chunks + 2) / 3, 4, 32); }

static int down_rows_per_block(int lpr, int KS) {
    const int G = kGemvThreads / lpr;
    const int rb = G * kPairsDN / KS;
    return rb > 0 ? rb : 1;
}

static int gu_rows_per_block(int lpr) { return kGemvWaves * (kWave / lpr) * kRuGU; }

void decode_plan(int fmt, DecodeArgs& a, int roles) {
    const int CH = chunk_elems(fmt);
    const int KS = a.K + (a.shared ? 1 : 0);
    a.lpr_gu = lpr_gate_up(a.H / CH);
    a.lpr_dn = lpr_down(a.I / CH);
    a.gu_rb = (a.I + gu_rows_per_block(a.lpr_gu) - 1) / gu_rows_per_block(a.lpr_gu);
    if (a.xf) {
        // wave-centric gate_up: 4 waves x RU rows (RU 4 for one chunk iteration, else 2)
        const int nci = (a.H / 32 + kWave - 1) / kWave;
        int ru = nci == 1 ? 4 : 2;
        if (nci == 1) {
            // the row count per wave that levels the work over the 256 CUs:
            // fewest (work-groups per CU) x (rows per work-group)
            auto cost = [&](int r) {
                const int64_t ng = int64_t(a.M) * KS * ((a.I + kGemvWaves * r - 1) / (kGemvWaves * r));
                return ((ng + 255) / 256) * r;
            };
            for (int r : {6, 8})
                if (cost(r) < cost(ru)) ru = r;
        }
        a.gu_ru = ru;
        a.gu_rb = (a.I + kGemvWaves * ru - 1) / (kGemvWaves * ru);
    }
    a.dn_rb = down_rows_per_block(a.lpr_dn, KS);
    a.dn_wave = 0;
    if (a.xf && KS <= 8 && a.I % 32 == 0 && a.I <= 4096) {
        // wave-centric down: 2 * RH rows per work-group, RH 4 for one chunk
        // iteration (I <= 1024), else 2
        a.dn_wave = 1;
        a.dn_rb = (a.I / 32 + 31) / 32 == 1 ? 8 : 4;
    }
    a.NR = (roles & kRoleRouter) ? a.E : 0;
    a.NG = (roles & kRoleGateUp) ? a.M * KS * a.gu_rb : 0;
    a.ND = (roles & kRoleDown) ? a.M * ((a.H + a.dn_rb - 1) / a.dn_rb) : 0;
}

bool decode_plan_fused(int fmt, DecodeArgs& a) {
    a.fused = 0;
    const bool wave_fmt = fmt == GRIM_FMT_INT4 || fmt == GRIM_FMT_INT4_F16 || fmt == GRIM_FMT_MXFP4;
    if (!wave_fmt || a.M != 1 || a.shared || !a.sync || a.K > 8 || a.K < 1 || a.E > 512 ||
        a.H % 32 || a.H > 2048 || a.I % 32 || a.I > 1024 || a.H < 32 || a.I < 32 || a.K * a.I > 8192)
        return false;
    // at most one 512-thread work-group per CU of this device (a partitioned
    // device has fewer than 256), so every work-group is resident while
    // others poll for its results
    static int cu_count[64];   // per device, looked up once
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
    int cus = __atomic_load_n(&cu_count[dev], __ATOMIC_RELAXED);
    if (cus == 0) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return false;
        __atomic_store_n(&cu_count[dev], cus, __ATOMIC_RELAXED);
    }
    const int kMaxGrid = std::min(cus, kSyncMaxGrid);
    auto gu_groups = [&](int ru) { return (a.K * (a.I / ru) + 7) / 8; };
    int ru = 0;
    for (int r : {2, 3, 4})
        if (a.I % r == 0 && gu_groups(r) <= kMaxGrid) { ru = r; break; }
    if (!ru) return false;
    const int gg = gu_groups(ru);
    int rh = 0, G = 0;
    for (int r : {2, 4}) {
        const int nb = (a.H + 2 * r - 1) / (2 * r);
        const int g = std::max(gg, nb);
        if (g <= kMaxGrid && (!rh || g < G)) { rh = r; G = g; }
        if (rh && nb <= gg) break;
    }
    if (!rh) return false;
    if (a.E > kSyncMaxE || !a.hrep) return false;
    a.fz_ru = ru;
    a.fz_rh = rh;
    a.fz_G = G;
    a.fused = 1;
    return true;
}

size_t decode_lds_bytes(int fmt, const DecodeArgs& a) {
    const int CH = chunk_elems(fmt);
    const int KS = a.K + (a.shared ? 1 : 0);
    // a staged vector of n elements: n words (bf16 pairs hi + lo, or fp32)
    // plus one fp32 sum per chunk
    auto act = [&](size_t n) { return (n + n / CH) * sizeof(uint32_t); };
    size_t b = 0;
    if (a.NR) b = std::max(b, size_t(kGemvWaves) * (512 + 64) * sizeof(float));
    if (a.NG && !a.xf) b = std::max(b, act(size_t(a.H)));
    if (a.ND && !a.dn_wave) b = std::max(b, act(size_t(KS) * a.I) + size_t(KS) * a.dn_rb * sizeof(float));
    return b;
}

hipError_t decode_launch(hipStream_t st, int fmt, const DecodeArgs& a) {
    switch (fmt) {
    case GRIM_FMT_BF16: return decode_launch_fmt_0(st, a);
    case GRIM_FMT_INT8: return decode_launch_fmt_3(st, a);
    case GRIM_FMT_INT4: return decode_launch_fmt_4(st, a);
    case GRIM_FMT_INT4_F16: return decode_launch_fmt_64(st, a);
    case GRIM_FMT_MXFP4: return decode_launch_fmt_6(st, a);
    }
    return hipErrorInvalidValue;
}

}  // namespace grim
