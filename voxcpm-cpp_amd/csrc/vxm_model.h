// vxm_model.h -- internal types of the MiniCPM4 / LocDiT drivers.
#pragma once

#include <algorithm>
#include <vector>

#include "vxm_ops.h"

struct vxm_block_dims {
    int64_t H = 0, F = 0;
    int nh = 0, nkv = 0, hd = 0;
    float eps = 1e-6f;
    int no_rope = 0;
    float res_scale = 1.0f;
    // NEOX rope: the (cos, sin) of every (position, pair) is computed on the
    // host with the C library (as ggml-cpu's rope cache is) and read from a
    // device table [rope_rows][hd/2], grown on demand.
    float rope_base = 10000.0f;
    std::vector<float> ff_host;   // frequency factors [hd/2], empty = none
    float2 *rope_cs = nullptr;
    int rope_rows = 0;
};

struct vxm_block {
    vxm_weight *wqkv = nullptr, *wo = nullptr, *wgu = nullptr, *wd = nullptr;
    float *g_in = nullptr, *g_post = nullptr;
};

// Scratch of one model for M tokens.
struct vxm_workspace {
    void *base = nullptr;
    size_t bytes = 0;
    int8_t *xq = nullptr;
    uint16_t *xd = nullptr;
    float *qkv = nullptr, *q = nullptr, *att = nullptr, *o = nullptr, *gu = nullptr, *dn = nullptr;
    uint16_t *lk = nullptr, *lv = nullptr;   // fresh K/V of non-causal runs
    int max_parts = 1;                       // K-split slices the projection buffers hold
    vxm_parts dn_out{};                      // the last block's down projection (slices of dn)
};

// Where a block's attention reads and writes K/V.
struct vxm_attn_site {
    uint16_t *kc, *vc;
    int cap;               // rows per kv head in the cache
    int64_t seg_stride;    // elements between segment caches (CFG branches)
    int S;                 // tokens per segment
    int pos0;              // rope position of token 0 of a segment
    int cache_pos0;        // cache row of token 0 (causal: keys 0..cache_pos0+t)
    int causal;
};

struct vxm_kv_cache {
    vxm_ctx *ctx = nullptr;
    // unique per created cache (never reused, unlike the struct's address):
    // what a decode that caches device pointers of a cache keys them on
    uint64_t id = 0;
    int n_layers = 0, nkv = 0, hd = 0, cap = 0;
    int32_t n_used = 0;
    int64_t layer_elems = 0;   // nkv * cap * hd
    void *base = nullptr;      // [layer][k|v][nkv][cap][hd] f16
    uint16_t *k(int l) { return (uint16_t *)base + (int64_t)l * 2 * layer_elems; }
    uint16_t *v(int l) { return (uint16_t *)base + ((int64_t)l * 2 + 1) * layer_elems; }
};

struct vxm_persistent_state;

struct vxm_minicpm4 {
    vxm_ctx *ctx = nullptr;
    vxm_minicpm4_config cfg{};
    vxm_block_dims dims;
    std::vector<vxm_block> blocks;
    float *final_norm = nullptr;
    vxm_workspace ws;
    int decode_mode = VXM_DECODE_AUTO;
    vxm_persistent_state *pstate = nullptr;
    // debug: every forward writes the input of each layer and the last layer's
    // output before the final norm here, [n_layers + 1][n_tokens][H] (null: off)
    float *layer_dump = nullptr;
};

// persistent single-launch decode (decode_persistent.hip)
bool vxm_persistent_supported(const vxm_minicpm4 *m, const vxm_kv_cache *kv);
int vxm_persistent_max_cap(const vxm_block_dims &d);
int vxm_persistent_decode(vxm_minicpm4 *m, vxm_kv_cache *kv, float *x, int32_t pos, float *dump);
int vxm_persistent_check(vxm_minicpm4 *m);
int vxm_persistent_set_epoch(vxm_minicpm4 *m, uint32_t epoch);
int vxm_persistent_get_epoch(vxm_minicpm4 *m, uint32_t *epoch);
void vxm_persistent_free(vxm_minicpm4 *m);

int vxm_ws_ensure(vxm_ctx *ctx, vxm_workspace &ws, int64_t M, int64_t H, int64_t qd, int64_t kvd, int64_t F,
                  int64_t local_kv);
void vxm_ws_free(vxm_workspace &ws);
int vxm_block_upload(vxm_ctx *ctx, const vxm_block_dims &d, const vxm_layer_weights_q8_0 &w, vxm_block &b);
void vxm_block_free(vxm_ctx *ctx, vxm_block &b);
void vxm_rope_setup(vxm_block_dims &d, int32_t theta, const float *ff_host);
int vxm_rope_ensure(vxm_ctx *ctx, vxm_block_dims &d, int64_t n_pos);
void vxm_rope_free(vxm_block_dims &d);
// F32 host vector -> new device buffer (nullptr in, nullptr out)
int vxm_upload_vec(vxm_ctx *ctx, const float *src, int64_t n, float **out);
int vxm_block_run(vxm_ctx *ctx, const vxm_block_dims &d, const vxm_block &b, vxm_workspace &ws, float *x,
                  int64_t M, const vxm_attn_site &site);

// every non-causal block of a LocDiT / LocEnc evaluation in one launch (locdit_persistent.hip):
// x [M][H] holds block 0's input and receives the last block's output (its residual added)
struct vxm_lpersist;
bool vxm_locdit_persistent_fits(vxm_ctx *ctx, const vxm_block_dims &d, int64_t M, int S);
// the block strategy (VXM_DECODE_*) resolved for one evaluation: true = the single launch
bool vxm_locdit_persistent_pick(vxm_ctx *ctx, const vxm_block_dims &d, int64_t M, int S, int mode);
// The final RMSNorm of the x rows fused into the launch (or none: g null): rows r0 .. S - 1 of
// every segment, normalised with gain g, as Q8_0 rows q [n_seg * (S - r0)][H] / d [..][H / 32]
// (segment-major), the steps of vxm_launch_rmsnorm with its Q8_0 output.
struct vxm_lfinal {
    const float *g = nullptr;
    int r0 = 0;
    int8_t *q = nullptr;
    uint16_t *d = nullptr;
};
// A whole CFM solve in the launch (vxm_cfm_solve's Euler loop): n_eval steps of sizes dts
// (host), time rows tc [n_eval][H], segment 0 with mu (n_mu = 1) or none, cond rows
// ch [Pc][H] + cb, x [P][feat] updated in place from its Q8_0 xq0 / xd0; the final norm
// (fin.g, r0 = 3 + Pc) and out_proj / in_proj run inside the launch.
struct vxm_lsolve {
    int n_eval = 0;
    const float *dts = nullptr;
    const float *tc = nullptr, *mu = nullptr, *ch = nullptr, *cb = nullptr;
    int n_mu = 0;
    const vxm_weight *in_proj = nullptr, *out_proj = nullptr;
    const float *in_b = nullptr, *out_b = nullptr;
    int P = 0, Pc = 0, feat = 0, n_seg = 1, use_cfg = 0;
    float cfg = 1.0f;
    float *x = nullptr;
    const int8_t *xq0 = nullptr;
    const uint16_t *xd0 = nullptr;
};
// whether vxm_locdit_persistent_run can take the solve (steps, feat, P, weight layout)
bool vxm_locdit_persistent_solve_fits(vxm_ctx *ctx, const vxm_block_dims &d, int64_t M, int S,
                                      const vxm_lsolve &sv);
// dump (debug, or null): [L + 1][M][H], the rows entering every block and the last block's output
// (not with a solve); with sv, the launch runs the solve (fin gives the final norm's gain and rows,
// its q / d are unused) and x is not read or written
int vxm_locdit_persistent_run(vxm_ctx *ctx, const vxm_block_dims &d, const std::vector<vxm_block> &blocks,
                              vxm_lpersist **st, float *x, int64_t M, int S, float *dump,
                              const vxm_lfinal &fin = vxm_lfinal{}, const vxm_lsolve *sv = nullptr);
int vxm_locdit_persistent_check(vxm_ctx *ctx, vxm_lpersist *st);
void vxm_locdit_persistent_free(vxm_lpersist *st);

// Every single-launch kernel (the decode, the LocDiT / LocEnc blocks) needs all
// 256 workgroups resident at once.  Two such launches on different streams of
// one device could interleave their workgroups and wait on each other until the
// bounded waits give up, so each eager launch is ordered after the previous one
// on its device (one event per device, waited on when the stream changes).
// Launches recorded into a HIP graph are not ordered this way: replays must not
// overlap another stream's single-launch work on the device.
struct vxm_launch_slot;
int vxm_ordered_launch_begin(vxm_ctx *ctx, vxm_launch_slot **slot, bool *capturing);
int vxm_ordered_launch_end(vxm_ctx *ctx, vxm_launch_slot *slot, bool capturing);
