// Launch-plan overrides (timing runs and tests only; unset in normal use).
//
// Every knob has a compiled-in default chosen from measurements on MI355X; an override is set through
// the C ABI (nmq_set_tuning / nmq_get_tuning) and read on the launch path with one relaxed atomic
// load.  The environment is not consulted: a production process cannot change its kernel choice by
// an inherited variable, and no launch pays for a getenv.
#pragma once

#include <atomic>
#include <climits>
#include <cstring>

namespace nmq {

enum Tune : int {
    TUNE_MV1,         // 0 disables the persistent one-token kernel
    TUNE_MV1_MAXNIT,  // most units per lane of the persistent one-token kernel
    TUNE_MV1_RW,      // rows per team of the persistent one-token kernel (1, 2)
    TUNE_MV1_NBUF,    // step buffers of the persistent one-token kernel (3, 4)
    TUNE_MV1_WPC,     // its resident waves per CU
    TUNE_MV1_W,       // its waves per workgroup
    TUNE_MV1_MODE,    // 0: general kernel, 1: chunk kernel, 2: persistent kernel (one token)
    TUNE_MV1_HR,      // 0: compiler-scheduled reads in the persistent kernel
    TUNE_MVL,         // 0 disables the long-row kernel
    TUNE_MVL_WPC,     // long-row kernel: resident waves per CU
    TUNE_MVL_W,       // long-row kernel: waves per workgroup
    TUNE_MVC_WGPC,    // chunk kernel: workgroups per CU
    TUNE_MVC_RW,      // chunk kernel: rows per team
    TUNE_MVC_ROWS,    // rows per CU up to which one token runs in the chunk kernel
    TUNE_MVT_MAX,     // most tokens of the few-token Q4_K kernel (1 disables it)
    TUNE_MVT_WPC,     // few-token Q4_K kernel: resident waves per CU
    TUNE_MVLT_MAX,    // most tokens of the few-token long-row Q6_K kernel (1 disables it)
    TUNE_MVM,         // matrix cores for 2..16 tokens: 0 never, 1 from the format's threshold, 2 from 2
    TUNE_MVM_TPW,     // matrix-core kernel: row tiles per workgroup
    TUNE_MVM_KS,      // matrix-core kernel: slices of the row
    TUNE_MMH_T,       // fp16 matrix-core kernel: row tiles per workgroup
    TUNE_MMH_G,       // fp16 matrix-core kernel: groups of 16 tokens per workgroup
    TUNE_MVK,         // 0 disables the K-split long-row kernel (one token, rows of 129..256 units)
    TUNE_MVK_WPC,     // K-split long-row kernel: resident waves per CU
    TUNE_MVD,         // 0 disables the dense-read matrix-core kernel (2..8 tokens)
    TUNE_MVD_MIN,     // fewest tokens that it takes
    TUNE_MVD_TPW,     // its row tiles per workgroup
    TUNE_MVD_KS,      // its slices of the row
    TUNE_MV1_T,       // lanes per row of the persistent one-token kernel (16, 32, 64; 0: by row length)
    TUNE_MVK_HR,      // 0: compiler-scheduled reads in the K-split long-row kernel
    TUNE_MVK_NBUF,    // its row buffers with hand-issued reads (3, 4)
    TUNE_MOE_GU_RW,   // rows per team of the MoE gate|up kernel (2, 4; 4, 8 for rows of 2049..4096 values)
    TUNE_MOE_GU_WGS,  // most workgroups of the gate|up kernel in the layer (default one per CU)
    TUNE_MVP_RPW,     // rows per wave and group of the dense gate|up kernel with the activation (4, 8)
    TUNE_MVP_WGS,     // its workgroups (default: the fewest groups of 32 rows per workgroup, spread evenly)
    TUNE_MVD_WGPC,    // workgroups per CU the dense-read kernel's plan aims at (1 .. 4)
    TUNE_MVD_LONG,    // rows beyond 4096 values: 1 one dense launch over K ranges, 2 one launch per range, 0 neither
    TUNE_MVD_UNEQ,    // 0: long rows only in equal K ranges (not 16-block ranges and a shorter last one)
    TUNE_COUNT
};

// Names as the C ABI takes them (index = Tune).
inline const char* const kTuneNames[TUNE_COUNT] = {
    "MV1",      "MV1_MAXNIT", "MV1_RW",  "MV1_NBUF", "MV1_WPC", "MV1_W",   "MV1_MODE", "MV1_HR",
    "MVL",      "MVL_WPC",    "MVL_W",   "MVC_WGPC", "MVC_RW",  "MVC_ROWS", "MVT_MAX", "MVT_WPC",
    "MVLT_MAX", "MVM",        "MVM_TPW", "MVM_KS",   "MMH_T",   "MMH_G",    "MVK",     "MVK_WPC",
    "MVD",      "MVD_MIN",    "MVD_TPW", "MVD_KS",   "MV1_T",    "MVK_HR",   "MVK_NBUF",
    "MOE_GU_RW", "MOE_GU_WGS", "MVP_RPW", "MVP_WGS", "MVD_WGPC", "MVD_LONG", "MVD_UNEQ"};

constexpr int TUNE_UNSET = INT_MIN;

// One table per process (an inline variable: every translation unit of the library shares it).
inline std::atomic<int> g_tune[TUNE_COUNT] = {};
inline std::atomic<bool> g_tune_ready{false};

inline void tune_reset_all() {
    for (int i = 0; i < TUNE_COUNT; ++i) g_tune[i].store(TUNE_UNSET, std::memory_order_relaxed);
    g_tune_ready.store(true, std::memory_order_release);
}

inline int tune_index(const char* name) {
    if (!name) return -1;
    if (std::strncmp(name, "NMQ_", 4) == 0) name += 4;  // the prefix is optional
    for (int i = 0; i < TUNE_COUNT; ++i)
        if (std::strcmp(name, kTuneNames[i]) == 0) return i;
    return -1;
}

// The override of knob k, or dflt when none is set.
inline int tune(Tune k, int dflt) {
    if (!g_tune_ready.load(std::memory_order_acquire)) return dflt;
    const int v = g_tune[k].load(std::memory_order_relaxed);
    return v == TUNE_UNSET ? dflt : v;
}

}  // namespace nmq
