// q3t_dev.hip -- device context and C ABI (include/q3t_dev.h) of the MI355X
// frame loop.  Host code here only moves data, sizes launches and records
// the per-frame hipGraph; every arithmetic step of the loop runs in the
// kernels of q3t_kernels.h.  There is no CPU fallback: without a HIP device
// every entry point fails with an error.

#include "../../include/q3t_dev.h"
#include "q3t_kernels.h"
#include "q3t_frame_kernel.h"
#include "q3t_prefill.h"
#include "q3t_streams.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

using namespace q3t;

namespace {

struct Slot {                 // one uploaded tensor (a view into device memory)
    int32_t type = -1;
    int64_t ne0 = 0, ne1 = 0;
    void * data = nullptr;         // Q8_0: int8 [ne1][ne0]; F16: [ne1][ne0]; F32
    uint16_t * scales = nullptr;   // Q8_0: fp16 [ne1][ne0/32]
};

struct Weight {               // what a GEMV launch needs
    int32_t kind = -1;        // W_Q8 / W_F16
    const void * w = nullptr;
    const uint16_t * d = nullptr;
};

struct LayerDev {
    Slot qkv;                 // attn_q | attn_k | attn_v rows, concatenated
    int32_t qkv_parts = 0;
    Slot wo, wg, wu, wd;
    const float * attn_norm = nullptr, * ffn_norm = nullptr, * q_norm = nullptr, * k_norm = nullptr;
};


}  // namespace

// Device scratch of q3t_dev_text_proj_noalloc, the entry point for callers
// that cannot allocate device memory: the ids, the gathered text_embd rows,
// the fc1 output, the Q8_0 copies of the GEMM inputs and the result rows of
// up to kNoAllocMaxIds ids.  Each GPU the library runs on holds its own copy
// until the process ends; calls that overlap on one GPU share it and race.
// In host code `scratch` names a host-side stand-in, never a device address:
// kernels get the address hipGetSymbolAddress returns for the current device
// (scratch_setup, once per device; q3t_dev::scratch).
constexpr size_t kScratchBytes = (size_t) 2 << 20;
constexpr int kNoAllocMaxIds = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct q3t_dev {
    q3t_config cfg{};
    int device = 0;
    hipStream_t stream = nullptr;
    unsigned char * scratch = nullptr;   // this device's copy of `scratch` (q3t_dev_text_proj_noalloc)
    std::string err;
    std::vector<void *> allocs;
    std::map<std::string, Slot> slots;
    std::vector<LayerDev> talker, cp;
    std::vector<Slot> cp_embd, cp_head;
    Slot codec_embd, codec_head, text_embd, fc1, fc1_b, fc2, fc2_b, out_norm, cp_out_norm;
    Slot mtp_w, mtp_b;                 // code_pred.mtp_proj (cp_hidden != hidden_size, the 1.7B layout)
    float * cpx = nullptr;             // the code predictor's projected input rows [2][cp_hidden]

    // workspace
    float * xa = nullptr, * xb = nullptr, * qkv = nullptr, * attn = nullptr, * ffn = nullptr;
    float * hidden = nullptr, * logits = nullptr, * cp_logits = nullptr, * tp_a = nullptr, * tp_b = nullptr;
    float * stage = nullptr; int32_t stage_rows = 0;
    float * hidden_all = nullptr; int32_t hidden_all_rows = 0;
    // MFMA prefill work buffers (sized for pf_rows tokens)
    int32_t pf_rows = 0;
    int8_t * pf_q = nullptr; float * pf_dx = nullptr;
    float * pf_xa = nullptr, * pf_xb = nullptr, * pf_qkv = nullptr, * pf_att = nullptr;
    // f64 MFMA prefill attention: scores and probabilities [n_head][n][ls]
    float * pf_s = nullptr; uint16_t * pf_p = nullptr; size_t pf_sp_cap = 0;
    float * pf_g = nullptr, * pf_u = nullptr, * pf_f = nullptr;
    uint16_t * pf_h = nullptr, * pf_l = nullptr;  // fp16 GEMM inputs of the fast F16 prefill (rows x kmax / ffn)
    float * pf_sc = nullptr;                      // per-row power-of-two scales of the widened ffn_down input
    // multi-stream decode: nb independent streams sharing the weights
    int32_t nb = 0, sb_ctx = 0;
    uint16_t * skc = nullptr, * svc = nullptr;        // [stream][layer][kv_head][sb_ctx][128]
    uint16_t * scpk = nullptr, * scpv = nullptr;      // [stream][cp_layer][kv_head][16][128]
    FrameState * sst = nullptr;
    SampleParams * sparams = nullptr;
    uint8_t * sseen = nullptr;                        // [stream][codec_vocab]
    int32_t * scodes = nullptr; int32_t scodes_cap = 0;      // [stream][scodes_cap][16]
    float * strail = nullptr; int32_t strail_cap = 0;        // [stream][strail_cap][d]
    int32_t * sntrail = nullptr;                      // [stream]
    float * spad = nullptr, * shidden = nullptr;      // [stream][d]
    float * slogits = nullptr, * scplogits = nullptr; // [stream][codec_vocab], [stream][cp_vocab]
    float * sstage = nullptr;                         // [stream][2][d]
    float * bxa = nullptr, * bxb = nullptr, * bqkv = nullptr, * batt = nullptr;   // [2 * nb][...]
    int8_t * bq8 = nullptr; float * bdx8 = nullptr;   // Q8_0 rows [2 * nb][max(qd, ffn)] and scales
    float * bff = nullptr;                             // F16 layers: SwiGLU rows [2 * nb][ffn]
    bool s_f16 = false;                                // multi-stream layers are F16 (else Q8_0)
    float * srs = nullptr;                            // RMSNorm row scales [2 * nb]
    double * sss[2] = {nullptr, nullptr};             // per-tile sums of squares of Wo / down outputs [d/16][2 nb]
    // split-K partials and per-tile tickets, one set per GEMM call type
    // (QKV, Wo, gate/up, down): a set's tickets advance by S per launch
    uint64_t * spart[4] = {}; uint32_t * scnt[4] = {}; int32_t * serr = nullptr;
    hipGraphExec_t s_exec = nullptr; hipGraph_t s_graph = nullptr;
    bool s_hm = false;            // F16 layers: the fp16-MFMA decode GEMMs (else the exact f64-MFMA ones)
    int32_t s_launched = 0, s_max = 0; bool s_ready = false;
    bool stats_streams = false;    // frame statistics describe the multi-stream loop
    std::vector<int32_t> s_emitted;
    int32_t * ids = nullptr; int32_t ids_cap = 0;
    // text projection and prefill row assembly: fc1 rows (quantised and
    // fp32) and projected rows for bp_rows ids; assembled rows, their specs
    // and the ICL reference codes
    int32_t bp_rows = 0; int8_t * bp_q = nullptr; float * bp_dx = nullptr, * bp_h = nullptr, * bp_proj = nullptr;
    int32_t bp_out_rows = 0; float * bp_out = nullptr; RowSpec * bp_spec = nullptr;
    int32_t * bp_frames = nullptr; int32_t bp_frames_cap = 0; float * bp_spk = nullptr;
    FrameState * st = nullptr;
    SampleParams * params = nullptr;
    uint8_t * seen = nullptr;
    int32_t * codes_out = nullptr; int32_t codes_cap = 0;
    bool codes_begun = false;          // codes_out holds a frame loop's rows (q3t_dev_frame_codes)
    float * trailing = nullptr; int32_t trailing_cap = 0; int32_t n_trailing = 0;
    float * pad = nullptr;
    // attention-row capture (q3t_dev_set_attn_capture): post-softmax rows
    // [n_head][n_kv] of talker layer attn_layer, one per talker step
    float * probs = nullptr; int32_t probs_cap = 0;
    int32_t attn_layer = -1;
    int32_t attn_emitted = 0;          // frames of the current loop whose rows are kept
    std::vector<std::vector<float>> attn_rows;

    // caches
    uint16_t * kc = nullptr, * vc = nullptr; int32_t n_ctx = 0;
    bool kv_bf16 = false;          // talker cache elements are bfloat16 (q3t_dev_kv_set_type), else fp16
    uint16_t * cpk = nullptr, * cpv = nullptr;
    float * rope_cos = nullptr, * rope_sin = nullptr, * cp_rope_cos = nullptr, * cp_rope_sin = nullptr;
    int32_t rope_rows = 0;

    hipGraphExec_t frame_exec = nullptr;
    hipGraph_t frame_graph = nullptr;
    // persistent frame kernel (q3t_frame_kernel.h)
    bool fk_ok = false;            // model / context qualify this context for it
    int fk_variant = 0;            // see fk_kernel()
    int xcd_map = -1;              // frame-launch workgroups dealt round-robin over the XCDs: -1 unknown, 0 no, 1 yes
    bool fk_no_xcd = false;        // a re-probe found the dealing changed: the row-parallel program from then on
    // streamed tensor upload (q3t_dev_upload_tensor_rows): the pinned host
    // staging buffer callers fill from the file, the device buffer raw Q8_0
    // blocks land in before the repack, and rows received per tensor
    void * up_host = nullptr; size_t up_host_cap = 0;
    void * up_raw = nullptr; size_t up_raw_cap = 0;
    std::map<std::string, int64_t> up_rows;
    unsigned char * fk_snap = nullptr;   // the frame loop's carried state before a frames_run on the XCD program
    bool gqa_lds_ok = false;       // ms::k_attn_gqa may take the LDS this context's n_ctx needs
    bool fk_refused = false;       // a cooperative launch was refused: this context stays on the graph
    bool fk_tab = false;           // the persistent kernel reads cp_tab
    int fk_grid = 0;
    fk::LayerQ8 * fk_layers = nullptr;
    uint64_t * fk_arena = nullptr; size_t fk_arena_bytes = 0;
    int32_t * fk_err = nullptr;
    // pinned host staging of the single-step calls (talker step): state and
    // input row in, logits, hidden row and error flag out, so every copy is a
    // plain DMA and one synchronisation ends the call
    char * pin = nullptr; size_t pin_bytes = 0;
    fk::Args * fk_args_dev = nullptr;
    bool fk_args_ok = false;           // fk_args_dev holds this context's current arguments
    bool fk_layers_stale = false;      // a layer tensor was uploaded after fk_layers was built
    int32_t fk_epoch = 0;              // launches since the arena was cleared (the phase tags)
    float * fk_cand = nullptr;         // talker-head greedy candidates: 256 values then 256 indices
    // code-predictor layer-0 QKV rows of every (codebook step, code): the
    // input of steps 1..14 is an embedding row, so their first QKV GEMV is a
    // table lookup ([15][cp_vocab][qkv width] fp32, XCD-parallel program only)
    float * cp_tab = nullptr;
    bool cp_tab_stale = true;
    bool s_tab = false;                // multi-stream code-predictor layer 0 from cp_tab (steps 1..14)
    hipEvent_t run_ev[2] = {nullptr, nullptr};
    uint8_t * copy_buf = nullptr;      // copy-kernel calibration buffers (time_kernel class 5)
    double run_us = 0.0;
    int64_t run_frames = 0;
    int32_t host_emitted = 0;
    int32_t frames_launched = 0;
    int32_t frames_max = 0;
    bool frames_ready = false;
    bool resolved = false;
    int n_cu = 256;
};

namespace {

int fail(q3t_dev * c, const std::string & msg) { c->err = msg; return -1; }

#define HIP_OK(call)                                                                         \
    do {                                                                                     \
        hipError_t e_ = (call);                                                              \
        if (e_ != hipSuccess) return fail(c, std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)

int dev_alloc(q3t_dev * c, void ** p, size_t bytes) {
    HIP_OK(hipMalloc(p, std::max<size_t>(bytes, 256)));
    c->allocs.push_back(*p);
    return 0;
}

template <typename T>
int dev_alloc_t(q3t_dev * c, T ** p, size_t count) {
    void * v = nullptr;
    if (dev_alloc(c, &v, count * sizeof(T))) return -1;
    *p = (T *) v;
    return 0;
}

void dev_free(q3t_dev * c, void * p) {
    if (!p) return;
    auto it = std::find(c->allocs.begin(), c->allocs.end(), p);
    if (it != c->allocs.end()) c->allocs.erase(it);
    (void) hipFree(p);
}

void drop_stream_graph(q3t_dev * c) {
    if (c->s_exec) { (void) hipGraphExecDestroy(c->s_exec); c->s_exec = nullptr; }
    if (c->s_graph) { (void) hipGraphDestroy(c->s_graph); c->s_graph = nullptr; }
    c->s_ready = false;
}

void drop_graph(q3t_dev * c) {
    if (c->frame_exec) { (void) hipGraphExecDestroy(c->frame_exec); c->frame_exec = nullptr; }
    if (c->frame_graph) { (void) hipGraphDestroy(c->frame_graph); c->frame_graph = nullptr; }
    c->frames_ready = false;
    c->fk_args_ok = false;
}

// Expected (ne0, ne1) of a named tensor; false if the name is not used by
// the frame loop (the reference skips such names, src/tts_transformer.cpp:407-409).
bool expected_shape(const q3t_config & g, const std::string & n, int64_t & ne0, int64_t & ne1,
                    int & layer, int & cb, std::string & field, bool & is_cp) {
    layer = -1; cb = -1; is_cp = false; field.clear(); ne1 = 1;
    const int64_t d = g.hidden_size, qd = (int64_t) g.n_head * g.head_dim, kd = (int64_t) g.n_kv_head * g.head_dim;
    if (n == "talker.text_embd.weight") { ne0 = g.text_embd_dim; ne1 = g.text_vocab; return true; }
    if (n == "talker.text_proj.fc1.weight") { ne0 = g.text_embd_dim; ne1 = g.text_embd_dim; return true; }
    if (n == "talker.text_proj.fc1.bias") { ne0 = g.text_embd_dim; return true; }
    if (n == "talker.text_proj.fc2.weight") { ne0 = g.text_embd_dim; ne1 = d; return true; }
    if (n == "talker.text_proj.fc2.bias") { ne0 = d; return true; }
    if (n == "talker.codec_embd.weight" || n == "talker.codec_head.weight") { ne0 = d; ne1 = g.codec_vocab; return true; }
    if (n == "talker.output_norm.weight") { ne0 = d; return true; }
    // the code predictor's own width (the 1.7B layout) and the projection to it
    const int64_t dc = g.cp_hidden;
    if (n == "code_pred.output_norm.weight") { ne0 = dc; return true; }
    if (dc != d && n == "code_pred.mtp_proj.weight") { ne0 = d; ne1 = dc; return true; }
    if (dc != d && n == "code_pred.mtp_proj.bias") { ne0 = dc; return true; }
    int idx = -1; char buf[64] = {0};
    const char * s = n.c_str();
    if (std::sscanf(s, "code_pred.codec_embd.%d.weight", &idx) == 1) {
        if (idx < 0 || idx >= g.n_codebooks - 1) return false;
        cb = idx; field = "cp_embd"; ne0 = d; ne1 = g.cp_vocab; return true;
    }
    if (std::sscanf(s, "code_pred.lm_head.%d.weight", &idx) == 1) {
        if (idx < 0 || idx >= g.n_codebooks - 1) return false;
        cb = idx; field = "cp_head"; ne0 = dc; ne1 = g.cp_vocab; return true;
    }
    int nl = 0, ffn = 0;
    int64_t w = d;
    if (std::sscanf(s, "talker.blk.%d.%63s", &idx, buf) == 2) { nl = g.n_layers; ffn = g.ffn_size; }
    else if (std::sscanf(s, "code_pred.blk.%d.%63s", &idx, buf) == 2) { nl = g.cp_layers; ffn = g.cp_ffn; is_cp = true; w = dc; }
    else return false;
    if (idx < 0 || idx >= nl) return false;
    layer = idx;
    field = buf;
    if (field == "attn_norm.weight" || field == "ffn_norm.weight") { ne0 = w; return true; }
    if (field == "attn_q_norm.weight" || field == "attn_k_norm.weight") { ne0 = g.head_dim; return true; }
    if (field == "attn_q.weight") { ne0 = w; ne1 = qd; return true; }
    if (field == "attn_k.weight" || field == "attn_v.weight") { ne0 = w; ne1 = kd; return true; }
    if (field == "attn_output.weight") { ne0 = qd; ne1 = w; return true; }
    if (field == "ffn_gate.weight" || field == "ffn_up.weight") { ne0 = w; ne1 = ffn; return true; }
    if (field == "ffn_down.weight") { ne0 = ffn; ne1 = w; return true; }
    return false;
}

size_t type_bytes(int type, int64_t ne0, int64_t ne1) {
    const int64_t n = ne0 * ne1;
    if (type == Q3T_TYPE_Q8_0) return (size_t) (n / 32) * 34;
    if (type == Q3T_TYPE_F16) return (size_t) n * 2;
    return (size_t) n * 4;
}

// Repack ggml Q8_0 blocks (fp16 d + 32 int8) into split arrays and copy.
// GGUF Q8_0 blocks (fp16 scale + 32 int8, 34 bytes) split into the int8
// quants [row][K] and the fp16 scales [row][K/32]: one thread per block, no
// value changes.
__global__ void k_repack_q8(const uint8_t * __restrict__ raw, int64_t n_blocks, int8_t * __restrict__ q,
                            uint16_t * __restrict__ d) {
    const int64_t b = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= n_blocks) return;
    const uint8_t * src = raw + b * 34;
    d[b] = (uint16_t) (src[0] | ((uint16_t) src[1] << 8));
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
        w[i] = (uint32_t) src[2 + 4 * i] | ((uint32_t) src[3 + 4 * i] << 8) | ((uint32_t) src[4 + 4 * i] << 16) |
               ((uint32_t) src[5 + 4 * i] << 24);
    int4 * dst = (int4 *) (q + b * 32);
    dst[0] = make_int4((int) w[0], (int) w[1], (int) w[2], (int) w[3]);
    dst[1] = make_int4((int) w[4], (int) w[5], (int) w[6], (int) w[7]);
}

// Rows [row0, row0 + n) of a slot whose rows are ne0 wide, from host memory
// in ggml layout (Q8_0: raw 34-byte blocks, repacked on the device through
// c->up_raw).  Synchronous: the caller may reuse `data` on return.
int upload_rows(q3t_dev * c, Slot & s, int64_t row0, int type, int64_t ne0, int64_t n, const void * data) {
    if (n <= 0) return 0;
    if (type == Q3T_TYPE_Q8_0) {
        const int64_t nb = ne0 / 32, blocks = nb * n;
        const size_t raw = (size_t) blocks * 34;
        if (raw > c->up_raw_cap) {
            dev_free(c, c->up_raw);
            c->up_raw = nullptr;
            c->up_raw_cap = 0;
            if (dev_alloc(c, &c->up_raw, raw)) return -1;
            c->up_raw_cap = raw;
        }
        HIP_OK(hipMemcpyAsync(c->up_raw, data, raw, hipMemcpyHostToDevice, c->stream));
        hipLaunchKernelGGL(k_repack_q8, dim3((unsigned) ((blocks + 255) / 256)), dim3(256), 0, c->stream,
                           (const uint8_t *) c->up_raw, blocks, (int8_t *) s.data + row0 * ne0, s.scales + row0 * nb);
    } else {
        const size_t eb = type == Q3T_TYPE_F16 ? 2 : 4;
        HIP_OK(hipMemcpyAsync((char *) s.data + row0 * ne0 * eb, data, (size_t) (ne0 * n) * eb, hipMemcpyHostToDevice,
                              c->stream));
    }
    HIP_OK(hipStreamSynchronize(c->stream));
    return 0;
}

int alloc_slot(q3t_dev * c, Slot & s, int type, int64_t ne0, int64_t ne1) {
    s.type = type; s.ne0 = ne0; s.ne1 = ne1;
    if (type == Q3T_TYPE_Q8_0) {
        if (dev_alloc(c, &s.data, (size_t) (ne0 * ne1))) return -1;
        void * sc = nullptr;
        if (dev_alloc(c, &sc, (size_t) (ne0 / 32 * ne1) * 2)) return -1;
        s.scales = (uint16_t *) sc;
    } else {
        if (dev_alloc(c, &s.data, type_bytes(type, ne0, ne1))) return -1;
    }
    return 0;
}

Weight weight_of(const Slot & s, bool widen_f16 = false) {
    Weight w;
    w.kind = s.type == Q3T_TYPE_Q8_0 ? W_Q8 : (widen_f16 ? W_F16W : W_F16);
    w.w = s.data; w.d = s.scales;
    return w;
}

int resolve(q3t_dev * c) {
    if (c->resolved) return 0;
    const q3t_config & g = c->cfg;
    // every tensor sent in row ranges must have all its rows
    for (const auto & kv : c->up_rows) {
        int64_t e0, e1; int layer, cb; std::string field; bool is_cp;
        if (expected_shape(g, kv.first, e0, e1, layer, cb, field, is_cp) && kv.second != e1)
            return fail(c, "tensor " + kv.first + " incomplete: " + std::to_string(kv.second) + " of " +
                               std::to_string(e1) + " rows uploaded");
    }
    auto need = [&](const Slot & s, const char * what) -> int {
        if (!s.data) return fail(c, std::string("missing tensor: ") + what);
        return 0;
    };
    for (int i = 0; i < g.n_layers + g.cp_layers; ++i) {
        LayerDev & L = i < g.n_layers ? c->talker[i] : c->cp[i - g.n_layers];
        char nm[64];
        std::snprintf(nm, sizeof nm, "%s.blk.%d", i < g.n_layers ? "talker" : "code_pred", i < g.n_layers ? i : i - g.n_layers);
        if (L.qkv_parts != 7) return fail(c, std::string("missing attn_q/k/v in ") + nm);
        if (need(L.wo, nm) || need(L.wg, nm) || need(L.wu, nm) || need(L.wd, nm)) return -1;
        if (!L.attn_norm || !L.ffn_norm || !L.q_norm || !L.k_norm) return fail(c, std::string("missing norm in ") + nm);
        if (L.wg.type != L.wu.type) return fail(c, std::string("ffn_gate/ffn_up types differ in ") + nm);
    }
    for (int i = 0; i < g.n_codebooks - 1; ++i) {
        if (!c->cp_embd[i].data || !c->cp_head[i].data) return fail(c, "missing code_pred.codec_embd/lm_head " + std::to_string(i));
        if (c->cp_embd[i].type != Q3T_TYPE_F16 || c->cp_head[i].type != Q3T_TYPE_F16)
            return fail(c, "code_pred embeddings and heads must be F16");
    }
    if (need(c->codec_embd, "talker.codec_embd.weight") || need(c->codec_head, "talker.codec_head.weight") ||
        need(c->out_norm, "talker.output_norm.weight") || need(c->cp_out_norm, "code_pred.output_norm.weight"))
        return -1;
    if (c->codec_embd.type != Q3T_TYPE_F16 || c->codec_head.type != Q3T_TYPE_F16)
        return fail(c, "talker.codec_embd / codec_head must be F16");
    if (g.cp_hidden != g.hidden_size &&
        (need(c->mtp_w, "code_pred.mtp_proj.weight") || need(c->mtp_b, "code_pred.mtp_proj.bias")))
        return -1;
    c->resolved = true;
    return 0;
}

// ------------------------------------------------------------ launches
struct GemvSpec {
    Weight w, w2;
    int rows, K;
    const float * x; int x_stride;
    const float * norm_w = nullptr;
    float * hidden_out = nullptr; int hidden_stride = 0;
    float * y; int y_stride;
    const float * resid = nullptr; int resid_stride = 0;
    const float * bias = nullptr;
    int epi = EPI_STORE;
    bool no_done = false;      // multi-stream heads: no single frame state to consult
};

template <int WT, int NT, bool DUAL>
void launch_gemv_t(q3t_dev * c, const GemvArgs & a) {
    const int BPR = a.K / kQK, LPR = BPR < 32 ? BPR : 32, RPW = 64 / LPR;
    const int groups = a.rows / RPW;
    int grid = (groups + 3) / 4;
    grid = std::max(1, std::min(grid, 2048));
    const size_t lds = act_red_bytes(NT) + act_bytes<WT>(NT, a.K);
    hipLaunchKernelGGL((k_gemv<WT, NT, DUAL>), dim3(grid), dim3(kBlock), lds, c->stream, a);
}

// register path: G row groups per wave, SLOTS = blocks per lane
template <int WT, int NT, bool DUAL, int SLOTS, int G>
void launch_gemv_r(q3t_dev * c, const GemvArgs & a) {
    const int BPR = a.K / kQK, LPR = BPR / SLOTS, RPW = 64 / LPR;
    const int groups = a.rows / RPW;
    const int grid = std::max(1, (groups + 4 * G - 1) / (4 * G));
    hipLaunchKernelGGL((k_gemv_r<WT, NT, DUAL, SLOTS, G>), dim3(grid), dim3(kBlock), 0, c->stream, a);
}

template <int WT, int NT, bool DUAL>
void launch_gemv_rs(q3t_dev * c, const GemvArgs & a) {
    const int BPR = a.K / kQK;
    if (BPR <= 32) launch_gemv_r<WT, NT, DUAL, 1, 2>(c, a);
    else if (BPR == 64) launch_gemv_r<WT, NT, DUAL, 2, 1>(c, a);
    else launch_gemv_r<WT, NT, DUAL, 3, 1>(c, a);
}

template <int WT, bool DUAL>
void launch_gemv_nt(q3t_dev * c, const GemvArgs & a, int nt, bool reg) {
    if (reg && nt == 1) launch_gemv_rs<WT, 1, DUAL>(c, a);
    else if (reg && nt == 2) launch_gemv_rs<WT, 2, DUAL>(c, a);
    else if (nt == 1) launch_gemv_t<WT, 1, DUAL>(c, a);
    else if (nt == 2) launch_gemv_t<WT, 2, DUAL>(c, a);
    else if constexpr (WT == W_F16 && !DUAL) {
        // the multi-stream heads: up to 16 streams' rows per launch
        if (nt == 16) launch_gemv_t<WT, 16, DUAL>(c, a);
        else if (nt == 8) launch_gemv_t<WT, 8, DUAL>(c, a);
        else launch_gemv_t<WT, 4, DUAL>(c, a);
    } else {
        launch_gemv_t<WT, 4, DUAL>(c, a);
    }
}

// K values the register path covers: K/32 a power of two up to 32, or 64, or 96.
bool reg_path_ok(int K) {
    const int b = K / kQK;
    return (b <= 32 && (b & (b - 1)) == 0) || b == 64 || b == 96;
}

void gemv(q3t_dev * c, const GemvSpec & s, int nt) {
    GemvArgs a{};
    a.w = s.w.w; a.wd = s.w.d; a.w2 = s.w2.w; a.w2d = s.w2.d;
    a.rows = s.rows; a.K = s.K;
    a.x = s.x; a.x_stride = s.x_stride;
    a.norm_w = s.norm_w; a.eps = c->cfg.rms_eps;
    a.hidden_out = s.hidden_out; a.hidden_stride = s.hidden_stride;
    a.y = s.y; a.y_stride = s.y_stride;
    a.resid = s.resid; a.resid_stride = s.resid_stride;
    a.bias = s.bias;
    a.done = s.no_done ? nullptr : &c->st->done;
    a.pro = s.norm_w ? PRO_NORM : PRO_NONE;
    a.epi = s.epi;
    // 1-2 tokens take the register path; more tokens (prefill chunks of 4)
    // take the LDS path, which reads plain fp32 rows only
    const bool reg = nt <= 2 && reg_path_ok(s.K);
    const bool dual = s.epi == EPI_SWIGLU;
    // 8 or 16 rows of an F16 head (the multi-stream heads): 1024-thread kernel
    if (s.w.kind == W_F16 && (nt == 8 || nt == 16) && s.epi == EPI_STORE && s.rows % 8 == 0 && s.K % kQK == 0 &&
        (nt == 16 ? gemv_mt_lds_bytes<16>(s.K) : gemv_mt_lds_bytes<8>(s.K)) <= 65536) {
        const dim3 grid(s.rows / 8);
        if (nt == 16)
            hipLaunchKernelGGL(k_gemv_mt<16>, grid, dim3(kMtThreads), gemv_mt_lds_bytes<16>(s.K), c->stream, a);
        else
            hipLaunchKernelGGL(k_gemv_mt<8>, grid, dim3(kMtThreads), gemv_mt_lds_bytes<8>(s.K), c->stream, a);
        return;
    }
    switch (s.w.kind) {
        case W_Q8: dual ? launch_gemv_nt<W_Q8, true>(c, a, nt, reg) : launch_gemv_nt<W_Q8, false>(c, a, nt, reg); break;
        case W_F16: dual ? launch_gemv_nt<W_F16, true>(c, a, nt, reg) : launch_gemv_nt<W_F16, false>(c, a, nt, reg); break;
        default: launch_gemv_nt<W_F16W, false>(c, a, nt, reg); break;
    }
}

struct AttnSpec {
    const float * qkv; const LayerDev * L;
    uint16_t * kc; uint16_t * vc; int n_ctx;
    const float * rc; const float * rs;
    const int32_t * pos_ptr; int pos_const;
    float * probs = nullptr;
    bool f32_prefill = false;   // the code predictor's 2-token prefill: F32 q, K, V, P
};

void attention(q3t_dev * c, const AttnSpec & s, int nt) {
    const q3t_config & g = c->cfg;
    const int G = g.n_head / g.n_kv_head;
    // the talker cache may be bfloat16; the code predictor's is always fp16
    const size_t kv_elems = (size_t) g.n_layers * g.n_kv_head * c->n_ctx * g.head_dim;
    const bool bf = c->kv_bf16 && s.kc >= c->kc && s.kc < c->kc + kv_elems;
    if (nt == 1 && s.rc == c->rope_cos && !s.probs && (G == 1 || G == 2 || G == 4) && c->gqa_lds_ok) {
        // one talker token: a 16-wave workgroup per query head streams its KV
        // head's cache (ms::k_attn_gqa, one head per workgroup)
        ms::GqaArgs q{};
        q.qkv = s.qkv; q.qkv_stride = (g.n_head + 2 * g.n_kv_head) * g.head_dim;
        q.q_norm = s.L->q_norm; q.k_norm = s.L->k_norm; q.eps = g.rms_eps;
        q.rope_cos = s.rc; q.rope_sin = s.rs;
        q.kc = s.kc; q.vc = s.vc; q.kv_stream = 0; q.n_ctx = s.n_ctx;
        q.n_head = g.n_head; q.n_kv_head = g.n_kv_head;
        q.pos = s.pos_ptr; q.pos_stream = 0; q.pos_const = s.pos_const;
        q.done = &c->st->done; q.done_stream = 0;
        q.out = c->attn; q.out_stride = g.n_head * g.head_dim;
        q.scale = 1.0f / std::sqrt((float) g.head_dim);
        const dim3 grid(g.n_head, 1), block(ms::kAThreads);
        if (bf) hipLaunchKernelGGL((ms::k_attn_gqa<1, true>), grid, block, ms::attn_gqa_lds_bytes(1, s.n_ctx), c->stream, q);
        else hipLaunchKernelGGL(ms::k_attn_gqa<1>, grid, block, ms::attn_gqa_lds_bytes(1, s.n_ctx), c->stream, q);
        return;
    }
    AttnArgs a{};
    a.qkv = s.qkv; a.qkv_stride = (g.n_head + 2 * g.n_kv_head) * g.head_dim;
    a.q_norm = s.L->q_norm; a.k_norm = s.L->k_norm; a.eps = g.rms_eps;
    a.rope_cos = s.rc; a.rope_sin = s.rs;
    a.kc = s.kc; a.vc = s.vc; a.n_ctx = s.n_ctx;
    a.n_head = g.n_head; a.n_kv_head = g.n_kv_head;
    a.pos_ptr = s.pos_ptr; a.pos_const = s.pos_const;
    a.out = c->attn; a.out_stride = g.n_head * g.head_dim;
    a.done = &c->st->done;
    a.scale = 1.0f / std::sqrt((float) g.head_dim);
    a.nt = nt;
    a.probs_out = s.probs;
    a.f32_new = s.f32_prefill ? 1 : 0;
    a.kv_bf16 = bf ? 1 : 0;
    hipLaunchKernelGGL(k_attention, dim3(g.n_head, nt), dim3(kBlock), attn_lds_bytes(s.n_ctx), c->stream, a);
}

// A block's second half over nt rows whose attention output is in c->attn:
// Wo plus the residual `xin` into c->xb, then the FFN with its residual into
// c->xa.  no_done: the kernels ignore the frame state's done flag.
void layer_tail(q3t_dev * c, const LayerDev & L, const float * xin, int nt, int d, int ffn, bool no_done) {
    const int qd = c->cfg.n_head * c->cfg.head_dim;
    GemvSpec o{};
    o.w = weight_of(L.wo); o.rows = d; o.K = qd; o.x = c->attn; o.x_stride = qd;
    o.y = c->xb; o.y_stride = d; o.resid = xin; o.resid_stride = d; o.epi = EPI_RESID; o.no_done = no_done;
    gemv(c, o, nt);
    GemvSpec f{};
    f.w = weight_of(L.wg); f.w2 = weight_of(L.wu); f.rows = ffn; f.K = d; f.x = c->xb; f.x_stride = d;
    f.norm_w = L.ffn_norm; f.y = c->ffn; f.y_stride = ffn; f.epi = EPI_SWIGLU; f.no_done = no_done;
    gemv(c, f, nt);
    GemvSpec dn{};
    dn.w = weight_of(L.wd, true); dn.rows = d; dn.K = ffn; dn.x = c->ffn; dn.x_stride = ffn;
    dn.y = c->xa; dn.y_stride = d; dn.resid = c->xb; dn.resid_stride = d; dn.epi = EPI_RESID; dn.no_done = no_done;
    gemv(c, dn, nt);
}

// One transformer block over nt tokens; input rows `xin` (stride d),
// output rows left in c->xa.
void layer(q3t_dev * c, const LayerDev & L, const float * xin, int nt, int d, int ffn, uint16_t * kc, uint16_t * vc,
           int n_ctx, const float * rc, const float * rs, const int32_t * pos_ptr, int pos_const,
           bool f32_prefill = false, float * probs = nullptr) {
    const q3t_config & g = c->cfg;
    const int qd = g.n_head * g.head_dim, kd = g.n_kv_head * g.head_dim, qkvd = qd + 2 * kd;
    GemvSpec s{};
    s.w = weight_of(L.qkv); s.rows = qkvd; s.K = d; s.x = xin; s.x_stride = d; s.norm_w = L.attn_norm;
    s.y = c->qkv; s.y_stride = qkvd;
    gemv(c, s, nt);
    AttnSpec as{c->qkv, &L, kc, vc, n_ctx, rc, rs, pos_ptr, pos_const};
    as.f32_prefill = f32_prefill;
    as.probs = probs;
    attention(c, as, nt);
    layer_tail(c, L, xin, nt, d, ffn, false);
}

// Rows [row0, ..) of a [rows][K] matrix as a weight of their own.
Weight weight_rows(const Slot & s, int64_t row0, int64_t K) {
    Weight w = weight_of(s);
    if (s.type == Q3T_TYPE_Q8_0) {
        w.w = (const int8_t *) s.data + row0 * K;
        w.d = s.scales + row0 * (K / 32);
    } else {
        w.w = (const uint16_t *) s.data + row0 * K;
    }
    return w;
}

// One transformer block of the single-pass code predictor on one row at one
// position with no cache (build_code_pred_graph, src/tts_transformer.cpp:
// 1823-1890): the attention over the row itself returns its V row, so only
// the V rows of the fused QKV matrix are multiplied; Q, K, their norms and
// the score leave no trace in the output.  No kernel reads the frame state.
void layer_single(q3t_dev * c, const LayerDev & L, const float * xin, int d, int ffn) {
    const q3t_config & g = c->cfg;
    const int qd = g.n_head * g.head_dim, kd = g.n_kv_head * g.head_dim;
    GemvSpec s{};
    s.w = weight_rows(L.qkv, qd + kd, d); s.rows = kd; s.K = d; s.x = xin; s.x_stride = d;
    s.norm_w = L.attn_norm; s.y = c->qkv; s.y_stride = kd; s.no_done = true;
    gemv(c, s, 1);
    hipLaunchKernelGGL(k_v_to_heads, dim3((qd + 255) / 256), dim3(256), 0, c->stream, c->qkv, g.head_dim,
                       g.n_head / g.n_kv_head, g.n_head, c->attn);
    layer_tail(c, L, xin, 1, d, ffn, true);
}

// Talker forward of nt (<= 4) tokens whose input rows are `xin`.  The codec
// head runs on the last row when `head` is set (normed hidden of that row ->
// c->hidden, logits -> c->logits).  A single-token step (`step`) writes the
// post-softmax rows of layer c->attn_layer to c->probs when capture is on.
void talker_chunk(q3t_dev * c, const float * xin, int nt, const int32_t * pos_ptr, int pos_const, bool head,
                  bool step = false) {
    const q3t_config & g = c->cfg;
    const int d = g.hidden_size;
    const size_t lstride = (size_t) g.n_kv_head * c->n_ctx * g.head_dim;
    for (int il = 0; il < g.n_layers; ++il)
        layer(c, c->talker[il], il == 0 ? xin : c->xa, nt, d, g.ffn_size, c->kc + il * lstride, c->vc + il * lstride,
              c->n_ctx, c->rope_cos, c->rope_sin, pos_ptr, pos_const, false,
              step && nt == 1 && il == c->attn_layer ? c->probs : nullptr);
    if (head) {
        GemvSpec h{};
        h.w = weight_of(c->codec_head); h.rows = g.codec_vocab; h.K = d;
        h.x = c->xa + (size_t) (nt - 1) * d; h.x_stride = d; h.norm_w = (const float *) c->out_norm.data;
        h.hidden_out = c->hidden; h.hidden_stride = d; h.y = c->logits; h.y_stride = g.codec_vocab;
        gemv(c, h, 1);
    }
}

SampleArgs sample_args(q3t_dev * c, int mode, int group) {
    const q3t_config & g = c->cfg;
    SampleArgs sa{};
    sa.mode = mode; sa.group = group;
    sa.vocab = mode == 0 ? g.codec_vocab : g.cp_vocab;
    sa.logits = mode == 0 ? c->logits : c->cp_logits + (size_t) (group - 1) * g.cp_vocab;
    sa.params = c->params; sa.st = c->st; sa.seen = c->seen; sa.eos_id = g.codec_eos_id;
    sa.stage = c->stage; sa.hidden = c->hidden; sa.codec_embd = (const uint16_t *) c->codec_embd.data;
    for (int i = 0; i < g.n_codebooks - 1; ++i) sa.cp_embd[i] = (const uint16_t *) c->cp_embd[i].data;
    sa.trailing = c->trailing; sa.n_trailing = c->n_trailing; sa.pad = c->pad;
    sa.d = g.hidden_size;
    return sa;
}

// Code predictor for the frame in c->st.  Its prefill rows [hidden;
// codec_embd[codebook-0 token]] are already in c->stage; each sampler gathers
// the next step's input row into c->stage.  Fills st->codes[1..15] and
// c->cp_logits; in the frame loop the codebook-15 sampler emits the frame and
// gathers the talker step embedding.
void code_pred_seq(q3t_dev * c, bool frame_loop) {
    const q3t_config & g = c->cfg;
    const int d = g.cp_hidden;
    const bool mtp = g.cp_hidden != g.hidden_size;
    const size_t lstride = (size_t) g.n_kv_head * 16 * g.head_dim;
    for (int step = 0; step < g.n_codebooks - 1; ++step) {
        const int nt = step == 0 ? 2 : 1;
        const int pos = step == 0 ? 0 : step + 1;
        if (mtp) {
            // talker-width input rows -> the code predictor's width
            // (src/tts_transformer.cpp:1942-1947, :2096-2101)
            GemvSpec m{};
            m.w = weight_of(c->mtp_w); m.rows = d; m.K = g.hidden_size; m.x = c->stage; m.x_stride = g.hidden_size;
            m.y = c->cpx; m.y_stride = d; m.bias = (const float *) c->mtp_b.data; m.epi = EPI_BIAS;
            gemv(c, m, nt);
        }
        for (int il = 0; il < g.cp_layers; ++il)
            layer(c, c->cp[il], il == 0 ? (mtp ? c->cpx : c->stage) : c->xa, nt, d, g.cp_ffn, c->cpk + il * lstride,
                  c->cpv + il * lstride, 16, c->cp_rope_cos, c->cp_rope_sin, nullptr, pos, step == 0);
        GemvSpec h{};
        h.w = weight_of(c->cp_head[step]); h.rows = g.cp_vocab; h.K = d;
        h.x = c->xa + (size_t) (nt - 1) * d; h.x_stride = d; h.norm_w = (const float *) c->cp_out_norm.data;
        h.y = c->cp_logits + (size_t) step * g.cp_vocab; h.y_stride = g.cp_vocab;
        gemv(c, h, 1);
        SampleArgs sa = sample_args(c, 1, step + 1);
        if (frame_loop) sa.codes_out = c->codes_out;
        hipLaunchKernelGGL(k_sample, dim3(1), dim3(kSampleThreads), 0, c->stream, sa);
    }
}

// The single-pass code predictor (build_code_pred_graph, src/tts_transformer.
// cpp:1771-1899) on the row in c->stage: its input sum, the MTP projection
// when the layout has one, the layers on one position with no cache, and the
// 15 heads on the last layer's row with no output norm, into c->cp_logits.
// Touches neither the frame state nor c->hidden / c->logits.
void code_pred_single(q3t_dev * c, SingleInArgs in) {
    const q3t_config & g = c->cfg;
    const int d = g.cp_hidden;
    const bool mtp = g.cp_hidden != g.hidden_size;
    in.hidden = c->stage; in.out = c->stage; in.d = g.hidden_size;
    hipLaunchKernelGGL(k_cp_single_input, dim3((g.hidden_size + 255) / 256), dim3(256), 0, c->stream, in);
    if (mtp) {
        GemvSpec m{};
        m.w = weight_of(c->mtp_w); m.rows = d; m.K = g.hidden_size; m.x = c->stage; m.x_stride = g.hidden_size;
        m.y = c->cpx; m.y_stride = d; m.bias = (const float *) c->mtp_b.data; m.epi = EPI_BIAS; m.no_done = true;
        gemv(c, m, 1);
    }
    for (int il = 0; il < g.cp_layers; ++il)
        layer_single(c, c->cp[il], il == 0 ? (mtp ? c->cpx : c->stage) : c->xa, d, g.cp_ffn);
    for (int h = 0; h < g.n_codebooks - 1; ++h) {
        GemvSpec o{};
        o.w = weight_of(c->cp_head[h]); o.rows = g.cp_vocab; o.K = d; o.x = c->xa; o.x_stride = d;
        o.y = c->cp_logits + (size_t) h * g.cp_vocab; o.y_stride = g.cp_vocab; o.no_done = true;
        gemv(c, o, 1);
    }
}

// One whole frame: open the frame and sample codebook 0 (gathering the
// code-predictor prefill rows), the code predictor (emits the frame and
// gathers the step embedding), the talker step.  Every kernel reads its
// dynamic inputs from c->st.
void frame_seq(q3t_dev * c) {
    SampleArgs sa = sample_args(c, 0, 0);
    sa.open_frame = 1;
    hipLaunchKernelGGL(k_sample, dim3(1), dim3(kSampleThreads), 0, c->stream, sa);
    code_pred_seq(c, true);
    talker_chunk(c, c->stage, 1, &c->st->talker_pos, 0, true, true);
}

int set_state(q3t_dev * c, const FrameState & s) {
    HIP_OK(hipMemcpyAsync(c->st, &s, sizeof s, hipMemcpyHostToDevice, c->stream));
    return 0;
}

int ensure_stage(q3t_dev * c, int rows) {
    if (rows <= c->stage_rows) return 0;
    dev_free(c, c->stage);
    c->stage = nullptr;
    const int r = std::max(rows, 16);
    if (dev_alloc_t(c, &c->stage, (size_t) r * std::max(c->cfg.hidden_size, c->cfg.text_embd_dim))) return -1;
    c->stage_rows = r;
    drop_graph(c);
    return 0;
}

int check_ready(q3t_dev * c) {
    if (resolve(c)) return -1;
    if (!c->kc) return fail(c, "KV cache not reserved");
    return 0;
}

int sync(q3t_dev * c) {
    HIP_OK(hipStreamSynchronize(c->stream));
    HIP_OK(hipGetLastError());
    return 0;
}

}  // namespace

constexpr size_t kCopyBytes = (size_t) 64 << 20;

// Plain 16-byte streaming copy: the reference point for the HBM byte
// counters (FETCH_SIZE / WRITE_SIZE) of the other kernels.
__global__ __launch_bounds__(256) void k_copy16(const int4 * __restrict__ src, int4 * __restrict__ dst, size_t n) {
    for (size_t i = (size_t) blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t) gridDim.x * 256) dst[i] = src[i];
}

// Decides whether the persistent frame kernel can run this context and
// prepares its tables.  Falls back to the multi-kernel graph otherwise.
// The kernel is instantiated for fixed (talker width, code-predictor width,
// query width, talker FFN, code-predictor FFN) and layer weight type:
// variant 1 / 3 = (1024, 1024, 2048, 3072, 3072), the 0.6B talker and code
// predictor, Q8_0 / F16 layers; variant 2 / 4 = (256, 256, 512, 512, 512), the
// small test shapes; 5 / 8 = the 0.6B shapes on the XCD-parallel layer
// program, Q8_0 / F16; 6 = the 1.7B layout (2048, 1024, 2048, 6144, 3072)
// with code_pred.mtp_proj, Q8_0; 7 = its small test form (512, 256, 512, 512,
// 512); 9 / 10 = the same two with F16 layers.
bool fk_xcd(int variant) { return variant == 5 || variant == 8; }
const void * fk_kernel(int variant) {
    switch (variant) {
        case 1: return (const void *) fk::k_frame<1024, 1024, 2048, 3072, 3072, W_Q8, false>;
        case 2: return (const void *) fk::k_frame<256, 256, 512, 512, 512, W_Q8, false>;
        case 3: return (const void *) fk::k_frame<1024, 1024, 2048, 3072, 3072, W_F16, false>;
        case 5: return (const void *) fk::k_frame<1024, 1024, 2048, 3072, 3072, W_Q8, true>;
        case 6: return (const void *) fk::k_frame<2048, 1024, 2048, 6144, 3072, W_Q8, false>;
        case 7: return (const void *) fk::k_frame<512, 256, 512, 512, 512, W_Q8, false>;
        case 8: return (const void *) fk::k_frame<1024, 1024, 2048, 3072, 3072, W_F16, true>;
        case 9: return (const void *) fk::k_frame<2048, 1024, 2048, 6144, 3072, W_F16, false>;
        case 10: return (const void *) fk::k_frame<512, 256, 512, 512, 512, W_F16, false>;
        default: return (const void *) fk::k_frame<256, 256, 512, 512, 512, W_F16, false>;
    }
}

// Q8_0 block slots per lane of the frame kernel's GEMV geometry (Geo<K>):
// up to 32 blocks, a power of two, in one slot; wider rows in slots of 32.
int slots_for(int K) {
    const int b = K / kQK;
    if (b <= 32) return (b & (b - 1)) == 0 ? 1 : 0;
    return b % 32 == 0 ? b / 32 : 0;
}

// The XCD of each workgroup of a 256-workgroup cooperative launch with the
// frame kernel's LDS footprint (one workgroup per CU, as the frame kernel).
__global__ __launch_bounds__(fk::kT) void k_xcc_map(int32_t * out) {
    __shared__ fk::Lds L;
    if (threadIdx.x == 0) {
        L.codes[0] = (int32_t) fk::xcc_id();
        out[blockIdx.x] = L.codes[0];
    }
}

// Whether the workgroups of a frame-sized cooperative launch are dealt to the
// XCDs round-robin, workgroup b on XCD (b + r) % 8 for one rotation r (the
// XCD-parallel layer program relies on the classes b % 8 each sharing an
// XCD; r itself varies between launches); checked once per context.
// Q3T_TEST_XCD_REPROBE_FAIL=1 (read per call) makes a re-probe after a
// frames_run on the XCD-parallel program report a changed dealing, so tests
// can exercise the switch to the row-parallel program from the host.
bool test_reprobe_fail() {
    const char * e = std::getenv("Q3T_TEST_XCD_REPROBE_FAIL");
    return e && e[0] == '1';
}

int xcd_map_ok(q3t_dev * c, int grid, bool & ok, bool forced_fail = false) {
    if (forced_fail) {
        c->xcd_map = 0;
        std::fprintf(stderr, "q3t: XCD map re-check forced to fail; using the row-parallel frame program\n");
    }
    if (c->xcd_map < 0) {
        int32_t * d = nullptr;
        if (dev_alloc_t(c, &d, (size_t) grid)) return -1;
        void * args[] = {&d};
        std::vector<int32_t> h(grid, -1);
        const hipError_t e =
            hipLaunchCooperativeKernel((const void *) k_xcc_map, dim3(grid), dim3(fk::kT), args, 0, c->stream);
        if (e == hipSuccess) {
            HIP_OK(hipMemcpyAsync(h.data(), d, (size_t) grid * 4, hipMemcpyDeviceToHost, c->stream));
            HIP_OK(hipStreamSynchronize(c->stream));
        } else {
            (void) hipGetLastError();   // refused: the row-parallel program runs instead
        }
        dev_free(c, d);
        int good = 0;
        for (int b = 0; b < grid; ++b) good += h[b] == (h[0] + b) % fk::kXcd;
        c->xcd_map = good == grid ? 1 : 0;
        if (!c->xcd_map)
            std::fprintf(stderr, "q3t: XCD map check %s (%d of %d workgroups dealt round-robin; wg 0..7 on %d %d %d %d %d %d %d %d); "
                                 "using the row-parallel frame program\n",
                         e == hipSuccess ? "failed" : hipGetErrorString(e), good, grid, h[0], h[1], h[2], h[3], h[4], h[5],
                         h[6], h[7]);
    }
    ok = c->xcd_map == 1;
    return 0;
}

const char * fk_err_msg(int32_t) { return "frame kernel: a phase wait timed out (results invalid)"; }

namespace {
int build_cp_tab(q3t_dev * c);   // below, with the prefill helpers it uses
}  // namespace

int fk_prepare(q3t_dev * c) {
    c->fk_ok = false;
    // attention capture runs the multi-kernel step
    if (c->fk_refused || c->attn_layer >= 0) return 0;
    if (const char * e = std::getenv("Q3T_FRAME_KERNEL")) if (e[0] == '0') return 0;
    const q3t_config & g = c->cfg;
    const int qd = g.n_head * g.head_dim, kd = g.n_kv_head * g.head_dim, qkvd = qd + 2 * kd;
    const int dc = g.cp_hidden;
    const int sq = slots_for(g.hidden_size), so = slots_for(qd), sd = slots_for(g.ffn_size);
    const int sqc = slots_for(dc), sdc = slots_for(g.cp_ffn);
    const bool mtp = dc != g.hidden_size;
    int variant = 0;
    if (!mtp && g.hidden_size == 1024 && qd == 2048 && g.ffn_size == 3072 && g.cp_ffn == 3072) variant = 1;
    if (!mtp && g.hidden_size == 256 && qd == 512 && g.ffn_size == 512 && g.cp_ffn == 512) variant = 2;
    if (mtp && g.hidden_size == 2048 && dc == 1024 && qd == 2048 && g.ffn_size == 6144 && g.cp_ffn == 3072) variant = 6;
    if (mtp && g.hidden_size == 512 && dc == 256 && qd == 512 && g.ffn_size == 512 && g.cp_ffn == 512) variant = 7;
    if (!variant || g.n_head != 2 * g.n_kv_head ||
        g.head_dim != 128 || g.cp_layers > fk::kCpLayers || g.codec_vocab > 3072 ||
        g.cp_vocab > 3072 || g.codec_vocab < 1024 || g.n_codebooks != 16 || qkvd > fk::kHS)
        return 0;
    // every layer matrix Q8_0, or every one F16 (and code_pred.mtp_proj of the
    // same type in the 1.7B layout)
    const int lt = c->talker[0].qkv.type;
    if (lt != Q3T_TYPE_Q8_0 && lt != Q3T_TYPE_F16) return 0;
    if (mtp && (c->mtp_w.type != lt || !c->mtp_b.data)) return 0;
    for (int i = 0; i < g.n_layers + g.cp_layers; ++i) {
        const LayerDev & L = i < g.n_layers ? c->talker[i] : c->cp[i - g.n_layers];
        if (L.qkv.type != lt || L.wo.type != lt || L.wg.type != lt || L.wu.type != lt || L.wd.type != lt) return 0;
    }
    if (lt == Q3T_TYPE_F16) variant = mtp ? variant + 3 : variant + 2;
    // one workgroup per CU (the LDS footprint allows no more), all co-resident
    int per_cu = 0;
    HIP_OK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fk_kernel(variant), fk::kT, 0));
    const int grid = std::min(256, per_cu * c->n_cu);
    if (grid < 1) return 0;
    const int nw = grid * fk::kW;
    // row groups per wave: what the phase needs on 1024 waves, as the kernel's
    // register sets hold (fk::ngroups); a smaller grid must cover the rows with
    // that many
    auto fits = [&](int rows, int K, int slots) {
        if (slots <= 0) return false;
        const int rpw = 64 / ((K / kQK) / slots);
        const int ng = std::max(1, (rows / rpw + 1023) / 1024);
        return rows % rpw == 0 && rows / rpw <= ng * nw;
    };
    auto head_fits = [&](int rows, int K) {
        const int lpr = std::min(K / kQK, 32);
        return (K / kQK) % lpr == 0 && (K / kQK) / lpr <= 2 && rows % (64 / lpr) == 0 && rows / (64 / lpr) <= 2 * nw;
    };
    if (!fits(qkvd, g.hidden_size, sq) || !fits(g.ffn_size, g.hidden_size, sq) ||
        !fits(g.hidden_size, qd, so) || !fits(g.hidden_size, g.ffn_size, sd) || !head_fits(g.codec_vocab, g.hidden_size) ||
        !fits(qkvd, dc, sqc) || !fits(g.cp_ffn, dc, sqc) || !fits(dc, qd, so) ||
        !fits(dc, g.cp_ffn, sdc) || !head_fits(g.cp_vocab, dc) || (mtp && !fits(dc, g.hidden_size, sq)) ||
        g.n_kv_head > grid)
        return 0;
    // talker attention: grid / n_kv_head position chunks per KV head, each
    // chunk's scores in LDS; phase C's partials fill kPvSlots slots
    const int chunks = grid / g.n_kv_head;
    const int chunk_len = 16 * ((c->n_ctx + 16 * chunks - 1) / (16 * chunks));
    if (chunk_len > fk::kMaxChunk || chunks > 128 || (size_t) grid * 512 > (size_t) fk::kPvSlots * fk::kSlot ||
        (g.n_head * 128 + grid - 1) / grid * 2 * chunks > 2 * fk::kMaxChunk)
        return 0;
    // the XCD-parallel layer program: 0.6B shapes (Q8_0 or F16), one
    // workgroup per CU on 256 CUs, workgroups dealt round-robin over the 8
    // XCDs (Q3T_FRAME_XCD=0 turns it off)
    bool xcd = (variant == 1 || variant == 3) && grid == 256 && g.n_kv_head == fk::kXcd && g.n_layers + g.cp_layers > 0 &&
               !c->fk_no_xcd;
    if (const char * e = std::getenv("Q3T_FRAME_XCD")) if (e[0] == '0') xcd = false;
    if (xcd && xcd_map_ok(c, grid, xcd)) return -1;
    if (xcd) variant = variant == 1 ? 5 : 8;
    // the code predictor's layer-0 QKV table
    bool tab = xcd;
    if (const char * e = std::getenv("Q3T_CP_QKV_TABLE")) if (e[0] == '0') tab = false;
    if (tab && (!c->cp_tab || c->cp_tab_stale) && build_cp_tab(c)) return -1;
    c->fk_tab = tab;
    // arena slots: row-parallel layer 5 (code predictor) or 7 + kPvSlots
    // (talker); XCD-parallel layer 15 or 17 + kPvSlots (device-wide partial
    // sums take 4 slots, XCD-local rows 2)
    const int phases = xcd ? 15 * (2 + 15 * g.cp_layers) + 1 + (17 + fk::kPvSlots) * g.n_layers
                           : 15 * (2 + (mtp ? 1 : 0) + 5 * g.cp_layers) + 1 + (7 + fk::kPvSlots) * g.n_layers;
    if (phases >= 4096) return 0;
    if (!c->fk_layers || c->fk_layers_stale) {
        std::vector<fk::LayerQ8> t(g.n_layers + g.cp_layers);
        for (int i = 0; i < g.n_layers + g.cp_layers; ++i) {
            const LayerDev & L = i < g.n_layers ? c->talker[i] : c->cp[i - g.n_layers];
            t[i] = fk::LayerQ8{(const int8_t *) L.qkv.data, L.qkv.scales, (const int8_t *) L.wo.data, L.wo.scales,
                               (const int8_t *) L.wg.data, L.wg.scales, (const int8_t *) L.wu.data, L.wu.scales,
                               (const int8_t *) L.wd.data, L.wd.scales, L.attn_norm, L.ffn_norm, L.q_norm, L.k_norm};
        }
        if (!c->fk_layers && dev_alloc_t(c, &c->fk_layers, t.size())) return -1;
        HIP_OK(hipMemcpy(c->fk_layers, t.data(), t.size() * sizeof(fk::LayerQ8), hipMemcpyHostToDevice));
        c->fk_layers_stale = false;
    }
    const size_t bytes = (size_t) phases * fk::kSlot * sizeof(uint64_t);
    if (bytes > c->fk_arena_bytes) {
        dev_free(c, c->fk_arena);
        c->fk_arena = nullptr;
        if (dev_alloc(c, (void **) &c->fk_arena, bytes)) return -1;
        c->fk_arena_bytes = bytes;
    }
    if (!c->fk_err && dev_alloc_t(c, &c->fk_err, 1)) return -1;
    if (!c->fk_args_dev && dev_alloc_t(c, &c->fk_args_dev, 1)) return -1;
    if (!c->fk_cand && dev_alloc_t(c, &c->fk_cand, 2 * 256)) return -1;
    c->fk_grid = grid;
    c->fk_variant = variant;
    c->fk_ok = true;
    c->fk_args_ok = false;
    return 0;
}

fk::Args fk_args(q3t_dev * c) {
    const q3t_config & g = c->cfg;
    fk::Args A{};
    A.talker = c->fk_layers; A.cp = c->fk_layers + g.n_layers;
    A.n_layers = g.n_layers; A.cp_layers = g.cp_layers; A.d = g.hidden_size; A.n_head = g.n_head;
    A.n_kv_head = g.n_kv_head; A.ffn = g.ffn_size; A.cp_ffn = g.cp_ffn; A.codec_vocab = g.codec_vocab;
    A.cp_vocab = g.cp_vocab; A.eos_id = g.codec_eos_id; A.n_ctx = c->n_ctx; A.kv_bf16 = c->kv_bf16 ? 1 : 0;
    A.eps = g.rms_eps; A.attn_scale = 1.0f / std::sqrt((float) g.head_dim);
    A.codec_embd = (const uint16_t *) c->codec_embd.data;
    for (int i = 0; i < 15; ++i) {
        A.cp_embd[i] = (const uint16_t *) c->cp_embd[i].data;
        A.cp_head[i] = (const uint16_t *) c->cp_head[i].data;
    }
    A.codec_head = (const uint16_t *) c->codec_head.data;
    A.out_norm = (const float *) c->out_norm.data; A.cp_out_norm = (const float *) c->cp_out_norm.data;
    A.rope_cos = c->rope_cos; A.rope_sin = c->rope_sin; A.cp_rope_cos = c->cp_rope_cos; A.cp_rope_sin = c->cp_rope_sin;
    A.kc = c->kc; A.vc = c->vc;
    A.arena = c->fk_arena;
    A.logits = c->logits; A.hidden = c->hidden;
    A.st = c->st; A.params = c->params; A.seen = c->seen; A.codes_out = c->codes_out;
    A.trailing = c->trailing; A.n_trailing = c->n_trailing; A.pad = c->pad;
    A.err = c->fk_err;
    A.cand_val = c->fk_cand;
    A.cand_idx = (int32_t *) (c->fk_cand + 256);
    A.step_in = c->stage;
    A.cp_qkv0 = c->fk_tab ? c->cp_tab : nullptr;
    if (g.cp_hidden != g.hidden_size) {
        A.mtp_w = (const int8_t *) c->mtp_w.data;
        A.mtp_d = c->mtp_w.scales;
        A.mtp_b = (const float *) c->mtp_b.data;
    }
    return A;
}

// Uploads the kernel arguments (the device copy is read by every launch).
int fk_upload_args(q3t_dev * c) {
    static thread_local fk::Args host_args;
    host_args = fk_args(c);
    HIP_OK(hipMemcpyAsync(c->fk_args_dev, &host_args, sizeof host_args, hipMemcpyHostToDevice, c->stream));
    HIP_OK(hipStreamSynchronize(c->stream));
    c->fk_args_ok = true;
    return 0;
}

// One launch of the persistent kernel.  Every launch since the arena was last
// cleared gets its own epoch, so no phase tag repeats; before the 20-bit epoch
// would wrap, the arena is cleared again (stream-ordered before the launch).
hipError_t fk_launch(q3t_dev * c, int32_t frame, int32_t mode) {
    constexpr int32_t kMaxEpoch = (1 << 20) - 2;
    if (c->fk_epoch >= kMaxEpoch) {
        const hipError_t e = hipMemsetAsync(c->fk_arena, 0, c->fk_arena_bytes, c->stream);
        if (e != hipSuccess) return e;
        c->fk_epoch = 0;
    }
    int32_t epoch = c->fk_epoch;
    void * args[] = {&c->fk_args_dev, &frame, &epoch, &mode};
    const hipError_t e =
        hipLaunchCooperativeKernel(fk_kernel(c->fk_variant), dim3(c->fk_grid), dim3(fk::kT), args, 0, c->stream);
    if (e == hipSuccess) ++c->fk_epoch;
    return e;
}

// The state one frame carries to the next on the persistent kernel: the frame
// state, the repetition set, the talker's logits and normed hidden row, and
// the talker head's greedy candidates.  frames_run keeps a copy while the
// XCD-parallel program runs, so a batch whose waits timed out can be run again
// from where it began.
struct SnapPart { void * p; size_t bytes; };
static int fk_snap_parts(q3t_dev * c, SnapPart (&parts)[5]) {
    const q3t_config & g = c->cfg;
    parts[0] = {c->st, sizeof(FrameState)};
    parts[1] = {c->seen, (size_t) g.codec_vocab};
    parts[2] = {c->logits, (size_t) g.codec_vocab * 4};
    parts[3] = {c->hidden, (size_t) g.hidden_size * 4};
    parts[4] = {c->fk_cand, (size_t) 2 * 256 * 4};
    return 5;
}

static int fk_snapshot(q3t_dev * c, bool restore) {
    SnapPart parts[5];
    const int np = fk_snap_parts(c, parts);
    if (!c->fk_snap) {
        size_t total = 0;
        for (int i = 0; i < np; ++i) total += (parts[i].bytes + 255) / 256 * 256;
        if (dev_alloc(c, (void **) &c->fk_snap, total)) return -1;
    }
    size_t off = 0;
    for (int i = 0; i < np; ++i) {
        void * dst = restore ? parts[i].p : (void *) (c->fk_snap + off);
        const void * src = restore ? (const void *) (c->fk_snap + off) : parts[i].p;
        HIP_OK(hipMemcpyAsync(dst, src, parts[i].bytes, hipMemcpyDeviceToDevice, c->stream));
        off += (parts[i].bytes + 255) / 256 * 256;
    }
    return 0;
}

// Whether a single-step call (talker step or code predictor) can run on the
// persistent kernel: prepares it and uploads the arguments when needed.
int fk_step_ready(q3t_dev * c, bool & ok) {
    ok = false;
    if (!c->fk_ok || !c->fk_args_ok) {
        if (fk_prepare(c)) return -1;
        if (!c->fk_ok) return 0;
        if (!c->fk_args_ok) {
            HIP_OK(hipMemsetAsync(c->fk_arena, 0, c->fk_arena_bytes, c->stream));
            c->fk_epoch = 0;
            if (fk_upload_args(c)) return -1;
        }
    }
    ok = true;
    return 0;
}

// The code predictor's head logits of a MODE_CODE_PRED launch, from the tagged
// head slots (slot first + s * stride for step s) into out [n][vocab].
__global__ void k_untag_heads(const uint64_t * __restrict__ arena, int first, int stride, int n, int vocab,
                              float * __restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n * vocab) return;
    const int s = i / vocab, r = i - s * vocab;
    out[i] = __uint_as_float((uint32_t) arena[(size_t) (first + s * stride) * fk::kSlot + r]);
}

// A single-step launch (talker step or code predictor) on the persistent
// kernel; false when it cannot run (the caller then takes the multi-kernel
// path, which gives the same results).
int fk_step(q3t_dev * c, int32_t frame, int32_t mode, bool & ran) {
    ran = false;
    bool ok = false;
    if (fk_step_ready(c, ok)) return -1;
    if (!ok) return 0;
    HIP_OK(hipMemsetAsync(c->fk_err, 0, sizeof(int32_t), c->stream));
    const hipError_t e = fk_launch(c, frame, mode);
    if (e != hipSuccess) {
        (void) hipGetLastError();
        std::fprintf(stderr, "q3t: cooperative frame-kernel launch refused (%s); using the multi-kernel path\n",
                     hipGetErrorString(e));
        c->fk_ok = false;
        c->fk_refused = true;
        return 0;
    }
    ran = true;
    return 0;
}



// Appends the captured attention row of the step at position n_kv - 1
// ([n_head][n_kv] floats in c->probs) to c->attn_rows.
int keep_attn_row(q3t_dev * c, int n_kv) {
    std::vector<float> row((size_t) c->cfg.n_head * n_kv);
    HIP_OK(hipMemcpy(row.data(), c->probs, row.size() * 4, hipMemcpyDeviceToHost));
    c->attn_rows.push_back(std::move(row));
    return 0;
}

// The captured multi-kernel frame, built on first use.
int ensure_frame_graph(q3t_dev * c) {
    if (c->frame_exec) return 0;
    HIP_OK(hipStreamSynchronize(c->stream));
    HIP_OK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    frame_seq(c);
    hipGraph_t graph = nullptr;
    HIP_OK(hipStreamEndCapture(c->stream, &graph));
    c->frame_graph = graph;
    HIP_OK(hipGraphInstantiate(&c->frame_exec, graph, nullptr, nullptr, 0));
    return 0;
}

// =================================================================== C ABI
extern "C" {

namespace {
std::mutex g_scratch_mu;
std::map<int, unsigned char *> g_scratch_addr;   // device ordinal -> its copy of `scratch`
}  // namespace

// With c->device current: the device address of this GPU's `scratch`, looked
// up once per device.
static int scratch_setup(q3t_dev * c) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto it = g_scratch_addr.find(c->device);
    if (it == g_scratch_addr.end()) {
        void * p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(c, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        it = g_scratch_addr.emplace(c->device, (unsigned char *) p).first;
    }
    c->scratch = it->second;
    return 0;
}

int q3t_dev_create(const q3t_config * cfg, int32_t device, q3t_dev ** out) {
    if (!cfg || !out) return -1;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return -2;
    if (device < 0 || device >= n) return -3;
    q3t_dev * c = new q3t_dev();
    c->cfg = *cfg;
    c->device = device;
    const q3t_config & g = c->cfg;
    auto bad = [&](const char * m) { c->err = m; *out = c; return -1; };
    if (g.head_dim != 128) return bad("head_dim must be 128");
    if (g.cp_hidden <= 0 || g.cp_hidden > g.hidden_size)
        return bad("code predictor width must be positive and at most the talker width");
    if (g.hidden_size % 256 || g.cp_hidden % 256 || g.ffn_size % 256 || g.cp_ffn % 256 || g.text_embd_dim % 256)
        return bad("hidden/ffn/text widths must be multiples of 256");
    auto ok_k = [](int k) { int b = k / 32; return b % 32 == 0 || (b <= 32 && (b & (b - 1)) == 0); };
    if (!ok_k(g.hidden_size) || !ok_k(g.cp_hidden) || !ok_k(g.ffn_size) || !ok_k(g.cp_ffn) ||
        !ok_k(g.text_embd_dim) || !ok_k(g.n_head * g.head_dim))
        return bad("unsupported reduction width");
    if (g.n_head % g.n_kv_head) return bad("n_head must be a multiple of n_kv_head");
    if (g.codec_vocab > kMaxVocab || g.cp_vocab > kMaxVocab) return bad("vocabulary too large for the on-device sampler");
    if (g.codec_vocab < 1024 || g.n_codebooks != 16) return bad("codec vocabulary must be >= 1024 with 16 codebooks");
    if (hipSetDevice(device) != hipSuccess) return bad("hipSetDevice failed");
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) return bad("hipStreamCreate failed");
    if (scratch_setup(c)) { *out = c; return -1; }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) c->n_cu = prop.multiProcessorCount;
    c->talker.resize(g.n_layers);
    c->cp.resize(g.cp_layers);
    c->cp_embd.resize(g.n_codebooks - 1);
    c->cp_head.resize(g.n_codebooks - 1);
    const int d = g.hidden_size, qd = g.n_head * g.head_dim, kd = g.n_kv_head * g.head_dim;
    const int wide = std::max({d, g.text_embd_dim, g.ffn_size, g.cp_ffn});
    int rc = 0;
    rc |= dev_alloc_t(c, &c->xa, (size_t) 4 * wide);
    rc |= dev_alloc_t(c, &c->xb, (size_t) 4 * wide);
    rc |= dev_alloc_t(c, &c->qkv, (size_t) 4 * (qd + 2 * kd));
    rc |= dev_alloc_t(c, &c->attn, (size_t) 4 * qd);
    rc |= dev_alloc_t(c, &c->ffn, (size_t) 4 * wide);
    rc |= dev_alloc_t(c, &c->tp_a, (size_t) 4 * wide);
    rc |= dev_alloc_t(c, &c->tp_b, (size_t) 4 * wide);
    rc |= dev_alloc_t(c, &c->hidden, (size_t) 4 * d);
    rc |= dev_alloc_t(c, &c->cpx, (size_t) 2 * g.cp_hidden);
    rc |= dev_alloc_t(c, &c->logits, (size_t) g.codec_vocab);
    rc |= dev_alloc_t(c, &c->cp_logits, (size_t) (g.n_codebooks - 1) * g.cp_vocab);
    rc |= dev_alloc_t(c, &c->st, 1);
    rc |= dev_alloc_t(c, &c->params, 1);
    rc |= dev_alloc_t(c, &c->seen, (size_t) g.codec_vocab);
    rc |= dev_alloc_t(c, &c->pad, (size_t) d);
    rc |= dev_alloc_t(c, &c->trailing, (size_t) d);
    rc |= dev_alloc_t(c, &c->codes_out, (size_t) 16);
    c->trailing_cap = 1; c->codes_cap = 1;
    rc |= ensure_stage(c, 16);
    if (rc) { *out = c; return -1; }
    FrameState s{};
    s.max_frames = 0;
    if (set_state(c, s) || sync(c)) { *out = c; return -1; }
    *out = c;
    return 0;
}

void q3t_dev_destroy(q3t_dev * c) {
    if (!c) return;
    (void) hipSetDevice(c->device);
    if (c->stream) (void) hipStreamSynchronize(c->stream);
    drop_graph(c);
    drop_stream_graph(c);
    for (hipEvent_t e : c->run_ev) if (e) (void) hipEventDestroy(e);
    for (void * p : c->allocs) (void) hipFree(p);
    if (c->pin) (void) hipHostFree(c->pin);
    if (c->up_host) (void) hipHostFree(c->up_host);
    if (c->stream) (void) hipStreamDestroy(c->stream);
    delete c;
}

const char * q3t_dev_last_error(const q3t_dev * c) { return c ? c->err.c_str() : "null context"; }

int q3t_dev_upload_tensor_rows(q3t_dev * c, const char * name, int32_t type, const int64_t ne[4], int64_t row0,
                               int64_t n_rows, const void * data, size_t nbytes) {
    if (!c || !name || !ne || (!data && n_rows > 0)) return -1;
    int64_t e0, e1; int layer, cb; std::string field; bool is_cp;
    if (!expected_shape(c->cfg, name, e0, e1, layer, cb, field, is_cp)) return 0;   // not on this path
    if (type != Q3T_TYPE_F32 && type != Q3T_TYPE_F16 && type != Q3T_TYPE_Q8_0)
        return fail(c, std::string("unsupported tensor type ") + std::to_string(type) + " for " + name +
                           " (this build loads F32, F16 and Q8_0 tensors)");
    if (ne[0] != e0 || ne[1] != e1 || ne[2] != 1 || ne[3] != 1)
        return fail(c, std::string("shape mismatch for ") + name);
    if (type == Q3T_TYPE_Q8_0 && e0 % 32) return fail(c, std::string("Q8_0 row not a multiple of 32: ") + name);
    if (row0 < 0 || n_rows < 0 || row0 + n_rows > e1) return fail(c, std::string("row range out of bounds for ") + name);
    if (nbytes != type_bytes(type, e0, n_rows)) return fail(c, std::string("byte size mismatch for ") + name);
    const bool is_matrix = e1 > 1;
    if (!is_matrix && type != Q3T_TYPE_F32) return fail(c, std::string("1-D tensors must be F32: ") + name);
    HIP_OK(hipSetDevice(c->device));
    drop_graph(c);
    c->resolved = false;
    c->fk_layers_stale = true;
    c->cp_tab_stale = true;
    const q3t_config & g = c->cfg;
    // a tensor's slot is made by its first range (row0 == 0); later ranges fill it
    auto seen = c->up_rows.find(name);
    const bool first = row0 == 0 && (seen == c->up_rows.end() || seen->second >= e1);
    if (!first && (seen == c->up_rows.end() || c->slots.find(name) == c->slots.end()))
        return fail(c, std::string("rows of ") + name + " before its first range");
    if (first) c->up_rows[name] = 0;
    c->up_rows[name] += n_rows;
    if (layer >= 0) {
        LayerDev & L = is_cp ? c->cp[layer] : c->talker[layer];
        if (field == "attn_q.weight" || field == "attn_k.weight" || field == "attn_v.weight") {
            const int64_t qd = (int64_t) g.n_head * g.head_dim, kd = (int64_t) g.n_kv_head * g.head_dim;
            if (!L.qkv.data) { if (alloc_slot(c, L.qkv, type, e0, qd + 2 * kd)) return -1; }
            else if (L.qkv.type != type) return fail(c, std::string("attn_q/k/v must share one type: ") + name);
            const int part = field == "attn_q.weight" ? 1 : field == "attn_k.weight" ? 2 : 4;
            const int64_t prow = part == 1 ? 0 : part == 2 ? qd : qd + kd;
            if (upload_rows(c, L.qkv, prow + row0, type, e0, n_rows, data)) return -1;
            if (c->up_rows[name] == e1) L.qkv_parts |= part;
            Slot v = L.qkv; v.ne1 = e1;
            v.data = type == Q3T_TYPE_Q8_0 ? (void *) ((int8_t *) L.qkv.data + prow * e0)
                                           : (void *) ((char *) L.qkv.data + prow * e0 * (type == Q3T_TYPE_F16 ? 2 : 4));
            if (v.scales) v.scales = L.qkv.scales + prow * (e0 / 32);
            c->slots[name] = v;
            return 0;
        }
    }
    Slot s;
    if (first) {
        if (alloc_slot(c, s, type, e0, e1)) return -1;
        c->slots[name] = s;
    } else {
        s = c->slots[name];
        if (s.type != type) return fail(c, std::string("tensor type changed between ranges: ") + name);
    }
    if (upload_rows(c, s, row0, type, e0, n_rows, data)) return -1;
    if (layer >= 0) {
        LayerDev & L = is_cp ? c->cp[layer] : c->talker[layer];
        if (field == "attn_output.weight") L.wo = s;
        else if (field == "ffn_gate.weight") L.wg = s;
        else if (field == "ffn_up.weight") L.wu = s;
        else if (field == "ffn_down.weight") L.wd = s;
        else if (field == "attn_norm.weight") L.attn_norm = (const float *) s.data;
        else if (field == "ffn_norm.weight") L.ffn_norm = (const float *) s.data;
        else if (field == "attn_q_norm.weight") L.q_norm = (const float *) s.data;
        else if (field == "attn_k_norm.weight") L.k_norm = (const float *) s.data;
        return 0;
    }
    const std::string n = name;
    if (field == "cp_embd") c->cp_embd[cb] = s;
    else if (field == "cp_head") c->cp_head[cb] = s;
    else if (n == "talker.text_embd.weight") c->text_embd = s;
    else if (n == "talker.text_proj.fc1.weight") c->fc1 = s;
    else if (n == "talker.text_proj.fc1.bias") c->fc1_b = s;
    else if (n == "talker.text_proj.fc2.weight") c->fc2 = s;
    else if (n == "talker.text_proj.fc2.bias") c->fc2_b = s;
    else if (n == "talker.codec_embd.weight") c->codec_embd = s;
    else if (n == "talker.codec_head.weight") c->codec_head = s;
    else if (n == "talker.output_norm.weight") c->out_norm = s;
    else if (n == "code_pred.output_norm.weight") c->cp_out_norm = s;
    else if (n == "code_pred.mtp_proj.weight") c->mtp_w = s;
    else if (n == "code_pred.mtp_proj.bias") c->mtp_b = s;
    return 0;
}

int q3t_dev_upload_tensor(q3t_dev * c, const char * name, int32_t type, const int64_t ne[4], const void * data,
                          size_t nbytes) {
    if (!c || !name || !ne || !data) return -1;
    return q3t_dev_upload_tensor_rows(c, name, type, ne, 0, ne[1], data, nbytes);
}

void * q3t_dev_staging(q3t_dev * c, size_t min_bytes, size_t * cap_out) {
    if (!c) return nullptr;
    if (hipSetDevice(c->device) != hipSuccess) { fail(c, "hipSetDevice failed"); return nullptr; }
    constexpr size_t kDefault = (size_t) 64 << 20;
    const size_t want = std::max(min_bytes, kDefault);
    if (want > c->up_host_cap) {
        if (c->up_host) (void) hipHostFree(c->up_host);
        c->up_host = nullptr;
        c->up_host_cap = 0;
        if (hipHostMalloc(&c->up_host, want, hipHostMallocDefault) != hipSuccess) {
            c->up_host = nullptr;
            fail(c, "pinned staging allocation failed");
            return nullptr;
        }
        c->up_host_cap = want;
    }
    if (cap_out) *cap_out = c->up_host_cap;
    return c->up_host;
}

int q3t_dev_download_tensor(q3t_dev * c, const char * name, void * data, size_t nbytes) {
    if (!c || !name || !data) return -1;
    auto it = c->slots.find(name);
    if (it == c->slots.end()) return fail(c, std::string("no such tensor: ") + name);
    const Slot & s = it->second;
    if (nbytes != type_bytes(s.type, s.ne0, s.ne1)) return fail(c, "byte size mismatch");
    HIP_OK(hipSetDevice(c->device));
    if (s.type == Q3T_TYPE_Q8_0) {
        const int64_t nb = s.ne0 / 32;
        std::vector<int8_t> q((size_t) (s.ne0 * s.ne1));
        std::vector<uint16_t> d((size_t) (nb * s.ne1));
        HIP_OK(hipMemcpy(q.data(), s.data, q.size(), hipMemcpyDeviceToHost));
        HIP_OK(hipMemcpy(d.data(), s.scales, d.size() * 2, hipMemcpyDeviceToHost));
        uint8_t * dst = (uint8_t *) data;
        for (int64_t b = 0; b < nb * s.ne1; ++b) {
            std::memcpy(dst + b * 34, &d[b], 2);
            std::memcpy(dst + b * 34 + 2, &q[b * 32], 32);
        }
    } else {
        HIP_OK(hipMemcpy(data, s.data, nbytes, hipMemcpyDeviceToHost));
    }
    return 0;
}

int q3t_dev_dequantize(q3t_dev * c, const char * name, float * out, size_t n_floats) {
    if (!c || !name || !out) return -1;
    auto it = c->slots.find(name);
    if (it == c->slots.end()) return fail(c, std::string("no such tensor: ") + name);
    const Slot & s = it->second;
    if (s.type != Q3T_TYPE_Q8_0) return fail(c, "not a Q8_0 tensor");
    const int64_t n = s.ne0 * s.ne1;
    if ((int64_t) n_floats != n) return fail(c, "size mismatch");
    HIP_OK(hipSetDevice(c->device));
    float * tmp = nullptr;
    HIP_OK(hipMalloc(&tmp, (size_t) n * 4));
    hipLaunchKernelGGL(k_dequant_q8, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, c->stream,
                       (const int8_t *) s.data, s.scales, n, tmp);
    hipError_t e = hipMemcpyAsync(out, tmp, (size_t) n * 4, hipMemcpyDeviceToHost, c->stream);
    hipError_t e2 = hipStreamSynchronize(c->stream);
    (void) hipFree(tmp);
    if (e != hipSuccess || e2 != hipSuccess) return fail(c, "dequantize failed");
    return 0;
}

int q3t_dev_kv_reserve(q3t_dev * c, int32_t n_ctx) {
    if (!c) return -1;
    const q3t_config & g = c->cfg;
    if (n_ctx <= 0) return fail(c, "n_ctx must be > 0");
    HIP_OK(hipSetDevice(c->device));
    // The single-workgroup attention kernels (k_attention, pf::k_attn_rows)
    // hold a head's n_ctx scores in LDS: 160 KiB per workgroup on gfx950
    // bounds n_ctx at about 38,600 positions (the talker's position table
    // ends at 32,768).
    int max_lds = 0;
    HIP_OK(hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, c->device));
    const size_t need_att = attn_lds_bytes(n_ctx), need_pf = pf::attn_rows_lds_bytes(n_ctx);
    if (std::max(need_att, need_pf) > (size_t) max_lds) {
        char msg[160];
        snprintf(msg, sizeof msg, "n_ctx %d needs %zu bytes of LDS for the decode attention; the device has %d",
                 (int) n_ctx, std::max(need_att, need_pf), max_lds);
        return fail(c, msg);
    }
    HIP_OK(hipFuncSetAttribute((const void *) k_attention, hipFuncAttributeMaxDynamicSharedMemorySize, (int) need_att));
    HIP_OK(hipFuncSetAttribute((const void *) pf::k_attn_rows, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int) need_pf));
    HIP_OK(hipStreamSynchronize(c->stream));
    drop_graph(c);
    drop_stream_graph(c);
    dev_free(c, c->kc); dev_free(c, c->vc); dev_free(c, c->cpk); dev_free(c, c->cpv);
    dev_free(c, c->rope_cos); dev_free(c, c->rope_sin); dev_free(c, c->cp_rope_cos); dev_free(c, c->cp_rope_sin);
    dev_free(c, c->probs);
    c->kc = c->vc = c->cpk = c->cpv = nullptr;
    c->probs = nullptr;
    c->probs_cap = 0;
    const size_t kv = (size_t) g.n_layers * g.n_kv_head * n_ctx * g.head_dim;
    const size_t ckv = (size_t) g.cp_layers * g.n_kv_head * 16 * g.head_dim;
    if (dev_alloc_t(c, &c->kc, kv) || dev_alloc_t(c, &c->vc, kv) || dev_alloc_t(c, &c->cpk, ckv) ||
        dev_alloc_t(c, &c->cpv, ckv) || dev_alloc_t(c, &c->probs, (size_t) g.n_head * n_ctx))
        return -1;
    c->probs_cap = n_ctx;
    HIP_OK(hipMemsetAsync(c->kc, 0, kv * 2, c->stream));
    HIP_OK(hipMemsetAsync(c->vc, 0, kv * 2, c->stream));
    HIP_OK(hipMemsetAsync(c->cpk, 0, ckv * 2, c->stream));
    HIP_OK(hipMemsetAsync(c->cpv, 0, ckv * 2, c->stream));
    // RoPE tables: theta_i = pos * base^(-2i/hd) by cumulative fp32 product
    // (ggml_rope_cache_init), cos/sin from the C library, once per context.
    const int rows = std::max(n_ctx, 16), half = g.head_dim / 2;
    std::vector<float> tc((size_t) rows * half), ts((size_t) rows * half), cc((size_t) rows * half), cs((size_t) rows * half);
    auto fill = [&](float base, std::vector<float> & co, std::vector<float> & si) {
        const float theta_scale = std::pow(base, -2.0f / (float) g.head_dim);
        for (int p = 0; p < rows; ++p) {
            float theta = (float) p;
            for (int i = 0; i < half; ++i) {
                co[(size_t) p * half + i] = std::cos(theta);
                si[(size_t) p * half + i] = std::sin(theta);
                theta *= theta_scale;
            }
        }
    };
    fill(g.rope_theta, tc, ts);
    fill(g.cp_rope_theta, cc, cs);
    if (dev_alloc_t(c, &c->rope_cos, tc.size()) || dev_alloc_t(c, &c->rope_sin, ts.size()) ||
        dev_alloc_t(c, &c->cp_rope_cos, cc.size()) || dev_alloc_t(c, &c->cp_rope_sin, cs.size()))
        return -1;
    HIP_OK(hipMemcpy(c->rope_cos, tc.data(), tc.size() * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(c->rope_sin, ts.data(), ts.size() * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(c->cp_rope_cos, cc.data(), cc.size() * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(c->cp_rope_sin, cs.data(), cs.size() * 4, hipMemcpyHostToDevice));
    c->n_ctx = n_ctx;
    c->rope_rows = rows;
    {
        // single-token talker attention through the GQA kernel when its LDS fits
        int max_lds = 0;
        HIP_OK(hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, c->device));
        const int G = g.n_kv_head > 0 ? g.n_head / g.n_kv_head : 0;
        c->gqa_lds_ok = false;
        if (G == 1 || G == 2 || G == 4) {
            const size_t al = ms::attn_gqa_lds_bytes(1, n_ctx);
            if (al <= (size_t) max_lds) {
                HIP_OK(hipFuncSetAttribute((const void *) ms::k_attn_gqa<1>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int) al));
                HIP_OK(hipFuncSetAttribute((const void *) ms::k_attn_gqa<1, true>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int) al));
                c->gqa_lds_ok = true;
            }
        }
    }
    return sync(c);
}

int q3t_dev_kv_clear(q3t_dev * c) { return c ? 0 : -1; }

int32_t q3t_dev_kv_capacity(const q3t_dev * c) { return c ? c->n_ctx : 0; }

int q3t_dev_kv_set_type(q3t_dev * c, int32_t type) {
    if (!c) return -1;
    if (type != Q3T_TYPE_F16 && type != Q3T_TYPE_BF16) return fail(c, "talker KV type must be F16 or BF16");
    const bool bf = type == Q3T_TYPE_BF16;
    if (bf == c->kv_bf16) return 0;
    c->kv_bf16 = bf;
    c->fk_ok = false;
    c->fk_args_ok = false;
    c->frames_ready = false;
    // a reserved cache is re-reserved (cleared) in the new type
    return c->n_ctx > 0 ? q3t_dev_kv_reserve(c, c->n_ctx) : 0;
}

int q3t_dev_set_attn_capture(q3t_dev * c, int32_t layer) {
    if (!c) return -1;
    if (layer < -1 || layer >= c->cfg.n_layers) return fail(c, "attention capture layer out of range");
    HIP_OK(hipSetDevice(c->device));
    HIP_OK(hipStreamSynchronize(c->stream));
    if (layer != c->attn_layer) {
        // the captured frame and the persistent kernel's arguments describe
        // the other mode; both are rebuilt on next use
        drop_graph(c);
        c->fk_ok = false;
        c->fk_args_ok = false;
        c->frames_ready = false;
    }
    c->attn_layer = layer;
    c->attn_rows.clear();
    return 0;
}

int32_t q3t_dev_attn_row_count(const q3t_dev * c) { return c ? (int32_t) c->attn_rows.size() : 0; }

int q3t_dev_attn_row(q3t_dev * c, int32_t index, float * out, int64_t cap, int32_t * n_kv_out) {
    if (!c) return -1;
    if (index < 0 || index >= (int32_t) c->attn_rows.size()) return fail(c, "attention row index out of range");
    const std::vector<float> & r = c->attn_rows[(size_t) index];
    if (n_kv_out) *n_kv_out = (int32_t) (r.size() / (size_t) c->cfg.n_head);
    if (!out) return 0;
    if (cap < (int64_t) r.size()) return fail(c, "attention row buffer too small");
    std::memcpy(out, r.data(), r.size() * sizeof(float));
    return 0;
}

int q3t_dev_kv_write(q3t_dev * c, int32_t layer, int32_t n_pos, const uint16_t * k, const uint16_t * v) {
    if (!c || !k || !v) return -1;
    const q3t_config & g = c->cfg;
    if (!c->kc) return fail(c, "KV cache not reserved");
    if (layer < 0 || layer >= g.n_layers || n_pos < 0 || n_pos > c->n_ctx) return fail(c, "kv_write out of range");
    HIP_OK(hipSetDevice(c->device));
    const size_t lstride = (size_t) g.n_kv_head * c->n_ctx * g.head_dim;
    std::vector<uint16_t> tk((size_t) n_pos * g.head_dim);
    for (int h = 0; h < g.n_kv_head; ++h) {
        for (int which = 0; which < 2; ++which) {
            const uint16_t * src = which ? v : k;
            for (int p = 0; p < n_pos; ++p)
                std::memcpy(&tk[(size_t) p * g.head_dim], src + ((size_t) p * g.n_kv_head + h) * g.head_dim,
                            g.head_dim * 2);
            uint16_t * dst = (which ? c->vc : c->kc) + layer * lstride + (size_t) h * c->n_ctx * g.head_dim;
            HIP_OK(hipMemcpy(dst, tk.data(), tk.size() * 2, hipMemcpyHostToDevice));
        }
    }
    return 0;
}

}  // extern "C"

namespace {

// Which tiled path the talker prefill of n tokens takes: 1 = int8 MFMA GEMMs
// (Q8_0 layers), 2 = exact F16 VALU GEMMs (F16 layers), 0 = the chunked GEMV
// prefill.  Tiled needs GEMM-friendly widths and, measured on the 0.6B shapes,
// pays from 9 rows for Q8_0 (10 rows: 5.2 ms against 5.8 ms in 4-row GEMV
// chunks) and from 40 rows for F16 (its VALU tiles take ~22 ms for any n up to
// 64, the GEMV ~2.3 ms per 4 rows).  Q3T_PREFILL_MFMA=0 disables it, =1 uses
// it for any n.
int tiled_prefill(q3t_dev * c, int n) {
    const char * e = std::getenv("Q3T_PREFILL_MFMA");
    if (e && e[0] == '0') return 0;
    const bool any = e && e[0] == '1';
    if (!any && n < 9) return 0;
    const q3t_config & g = c->cfg;
    const int d = g.hidden_size, qd = g.n_head * g.head_dim, qkvd = qd + 2 * g.n_kv_head * g.head_dim;
    if (g.head_dim != 128 || d % 128 || qd % 128 || g.ffn_size % 128 || qkvd % pf::kTile || d % pf::kTile ||
        g.ffn_size % pf::kTile)
        return 0;
    const int lt = c->talker[0].qkv.type;
    if (lt != Q3T_TYPE_Q8_0 && lt != Q3T_TYPE_F16) return 0;
    if (!any && lt == Q3T_TYPE_F16 && n < 40) return 0;
    for (int i = 0; i < g.n_layers; ++i) {
        const LayerDev & L = c->talker[i];
        if (L.qkv.type != lt || L.wo.type != lt || L.wg.type != lt || L.wu.type != lt || L.wd.type != lt) return 0;
    }
    return lt == Q3T_TYPE_Q8_0 ? 1 : 2;
}

int ensure_pf(q3t_dev * c, int n) {
    if (n <= c->pf_rows) return 0;
    const q3t_config & g = c->cfg;
    const int d = g.hidden_size, qd = g.n_head * g.head_dim, qkvd = qd + 2 * g.n_kv_head * g.head_dim;
    const int kmax = std::max(std::max(d, qd), g.ffn_size);
    for (void * p : {(void *) c->pf_q, (void *) c->pf_dx, (void *) c->pf_xa, (void *) c->pf_xb, (void *) c->pf_qkv,
                     (void *) c->pf_att, (void *) c->pf_g, (void *) c->pf_u, (void *) c->pf_f, (void *) c->pf_h,
                     (void *) c->pf_l, (void *) c->pf_sc})
        if (p) dev_free(c, p);
    c->pf_rows = 0;
    const size_t r = (size_t) n;
    if (dev_alloc_t(c, &c->pf_q, r * kmax) || dev_alloc_t(c, &c->pf_dx, r * (kmax / kQK)) ||
        dev_alloc_t(c, &c->pf_xa, r * d) || dev_alloc_t(c, &c->pf_xb, r * d) || dev_alloc_t(c, &c->pf_qkv, r * qkvd) ||
        dev_alloc_t(c, &c->pf_att, r * qd) || dev_alloc_t(c, &c->pf_g, r * g.ffn_size) ||
        dev_alloc_t(c, &c->pf_u, r * g.ffn_size) || dev_alloc_t(c, &c->pf_f, r * g.ffn_size) ||
        dev_alloc_t(c, &c->pf_h, r * kmax) || dev_alloc_t(c, &c->pf_l, r * g.ffn_size) ||
        dev_alloc_t(c, &c->pf_sc, r))
        return -1;
    c->pf_rows = n;
    return 0;
}

void pf_gemm(q3t_dev * c, const Slot & w, int N, int K, int n, float * y, const float * res, int rs = -1,
             const int8_t * q = nullptr, const float * dx = nullptr) {
    // tile: 64 weight rows x 32 JT tokens, JT = 2 unless that leaves the launch
    // with fewer workgroups than CUs; two Q8_0 blocks per stage
    int IR = 2, JT = 2, GB = 2;
    while (JT > 1 && (int64_t) (N / (32 * IR)) * ((n + 32 * JT - 1) / (32 * JT)) < c->n_cu) JT >>= 1;
    if (const char * e = std::getenv("Q3T_PF_TILE")) {      // "<IR>x<JT>x<GB>"
        const int ir = e[0] - '0', jt = e[1] == 'x' ? e[2] - '0' : 0, gb = e[1] == 'x' && e[3] == 'x' ? e[4] - '0' : 2;
        if ((ir == 2 || (ir == 4 && N % 128 == 0 && gb == 2)) && (jt == 1 || jt == 2 || jt == 4) &&
            (gb == 2 || gb == 4) && (K / kQK) % gb == 0) { IR = ir; JT = jt; GB = gb; }
    }
    const dim3 grid(N / (32 * IR), (n + 32 * JT - 1) / (32 * JT));
    const int8_t * qq = q ? q : (const int8_t *) c->pf_q;
    const float * dd = dx ? dx : (const float *) c->pf_dx;
    const int epi = res ? (int) EPI_RESID : (int) EPI_STORE;
    const int r = rs < 0 ? N : rs;
#define Q3T_PF_GEMM(ir, jt, gb)                                                                                  \
    hipLaunchKernelGGL((pf::k_gemm_q8<ir, jt, gb>), grid, dim3(kBlock), 0, c->stream, (const int8_t *) w.data, \
                       (const uint16_t *) w.scales, N, K, qq, dd, n, y, N, res, r, epi)
#define Q3T_PF_GEMM_JT(ir, gb)                                                                                   \
    if (JT == 4) Q3T_PF_GEMM(ir, 4, gb); else if (JT == 2) Q3T_PF_GEMM(ir, 2, gb); else Q3T_PF_GEMM(ir, 1, gb)
    if (GB == 4) {
        Q3T_PF_GEMM_JT(2, 4);
    } else {
        if (IR == 4) { Q3T_PF_GEMM_JT(4, 2); } else { Q3T_PF_GEMM_JT(2, 2); }
    }
#undef Q3T_PF_GEMM_JT
#undef Q3T_PF_GEMM
}

// Q8_0 rows of x (after an RMSNorm with weights w, or with u the SwiGLU
// silu(x) * u) into q / dx (default: the prefill's pf_q / pf_dx).
void pf_quant(q3t_dev * c, const float * x, int n, int K, const float * w, int xs = -1, int8_t * q = nullptr,
              float * dx = nullptr, const float * u = nullptr) {
    hipLaunchKernelGGL(pf::k_quant_rows, dim3(n), dim3(kBlock), 0, c->stream, x, xs < 0 ? K : xs, K, w, c->cfg.rms_eps,
                       q ? q : c->pf_q, dx ? dx : c->pf_dx, u);
}

__global__ __launch_bounds__(256) void k_h2f(const uint16_t * __restrict__ in, size_t n, float * __restrict__ out) {
    const size_t i = (size_t) blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = h2f(in[i]);
}

// cp_tab[s][code] = the QKV output of code-predictor layer 0 on the row
// codec_embd.s[code] (the input of codebook step s + 1): RMSNorm, Q8_0
// activation quantisation and the int8 GEMM of the prefill path, whose rows
// equal the frame kernel's GEMV bit for bit.  Rebuilt after any upload.
void pf_gemm_f16(q3t_dev * c, const Slot & w, int N, int K, int n, const float * x, int xs, bool wide, float * y,
                 const float * res, int rs);

int build_cp_tab(q3t_dev * c) {
    const q3t_config & g = c->cfg;
    const int d = g.cp_hidden, V = g.cp_vocab, ncb = g.n_codebooks - 1;
    const int qkvd = (g.n_head + 2 * g.n_kv_head) * g.head_dim;
    const LayerDev & L = c->cp[0];
    const bool q8 = L.qkv.type == Q3T_TYPE_Q8_0;
    if ((!q8 && L.qkv.type != Q3T_TYPE_F16) || d != g.hidden_size)
        return fail(c, "cp QKV table needs Q8_0 or F16 layers");
    if (!c->cp_tab && dev_alloc_t(c, &c->cp_tab, (size_t) ncb * V * qkvd)) return -1;
    if (ensure_pf(c, V)) return -1;
    const size_t n = (size_t) V * d;
    for (int sidx = 0; sidx < ncb; ++sidx) {
        if (c->cp_embd[sidx].type != Q3T_TYPE_F16) return fail(c, "embedding tables must be F16");
        hipLaunchKernelGGL(k_h2f, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, c->stream,
                           (const uint16_t *) c->cp_embd[sidx].data, n, c->pf_xa);
        float * rows = c->cp_tab + (size_t) sidx * V * qkvd;
        if (q8) {
            pf_quant(c, c->pf_xa, V, d, L.attn_norm);
            pf_gemm(c, L.qkv, qkvd, d, V, rows, nullptr);
        } else {
            // RMSNorm, then the exact F16 GEMM on fp16-rounded rows (the GEMV's numbers)
            hipLaunchKernelGGL(k_rmsnorm_rows, dim3(V), dim3(kBlock), 0, c->stream, (const float *) c->pf_xa,
                               L.attn_norm, g.rms_eps, d, c->pf_f);
            pf_gemm_f16(c, L.qkv, qkvd, d, V, c->pf_f, d, false, rows, nullptr, 0);
        }
    }
    HIP_OK(hipStreamSynchronize(c->stream));
    c->cp_tab_stale = false;
    return 0;
}

// F16 weights x fp32 rows on the exact f64-MFMA GEMM: y = epi(W . rows of x),
// x rounded to fp16 unless wide (the widened ffn_down).  K chunks of 64
// where K allows (Q3T_PF_F16_KC=32 forces 32).
void pf_gemm_f16(q3t_dev * c, const Slot & w, int N, int K, int n, const float * x, int xs, bool wide, float * y,
                 const float * res, int rs) {
    static const int kc_env = [] { const char * e = std::getenv("Q3T_PF_F16_KC"); return e ? std::atoi(e) : 0; }();
    const char * te = std::getenv("Q3T_PF_F16_TAIL");   // read per call (tests switch it)
    const bool tail_off = te && te[0] == '0';
    const int kc = (kc_env == 32 || K % 64) ? 32 : 64;
    // a remainder of at most 32 tokens goes to 16-row tail workgroups
    // (Q3T_PF_F16_TAIL=0 keeps it in a partial 64-token tile)
    const int rem = n % pf::kTile;
    const bool tail = rem != 0 && rem <= 32 && !tail_off;
    const int nfull = tail ? n / pf::kTile : (n + pf::kTile - 1) / pf::kTile;
    const dim3 grid((unsigned) ((N / pf::kTile) * nfull + (tail ? N / 16 : 0)));
#define Q3T_PF_F16(wd, kcv)                                                                                       \
    hipLaunchKernelGGL((pf::k_gemm_f16<wd, kcv>), grid, dim3(kBlock), 0, c->stream, (const uint16_t *) w.data, N, K, \
                       x, xs, n, y, N, res, rs, nfull)
    if (wide) {
        if (kc == 64) Q3T_PF_F16(true, 64); else Q3T_PF_F16(true, 32);
    } else {
        if (kc == 64) Q3T_PF_F16(false, 64); else Q3T_PF_F16(false, 32);
    }
#undef Q3T_PF_F16
}

// F16 weights x fp16 rows on the fast fp16-MFMA GEMM (fp32 accumulation):
// y = (W . xh[t] (+ W . xl[t])) * xsc[t] (+ res).  128 x 128 tiles with one
// stage in flight when that gives at least one workgroup per CU, else
// 128 x 64 tiles with two stages in flight (and always for the two-plane
// input); measured best on the 0.6B shapes at 2,048 rows: QKV 30 us, Wo 27 us,
// gate / up 29 us, the two-plane down 47 us.
void pf_gemm_h16(q3t_dev * c, const Slot & w, int N, int K, int n, const uint16_t * xh, const uint16_t * xl, int xs,
                 const float * xsc, float * y, const float * res, int rs) {
    constexpr int BR = 32 * 4;
    const bool big = !xl && (int64_t) (N / BR) * ((n + 127) / 128) >= c->n_cu;
    const int TT = big ? 4 : 2;
    const dim3 grid(N / BR, (n + 32 * TT - 1) / (32 * TT));
#define Q3T_PF_H16(tt, lo, pd)                                                                                    \
    hipLaunchKernelGGL((pf::k_gemm_h16<4, tt, lo, pd>), grid, dim3(kBlock), 0, c->stream, (const uint16_t *) w.data, \
                       K, xh, xl, xs, xsc, n, y, N, res, rs)
    if (xl) Q3T_PF_H16(2, true, 2);
    else if (big) Q3T_PF_H16(4, false, 1);
    else Q3T_PF_H16(2, false, 2);
#undef Q3T_PF_H16
}

// The tiled prefill's fast forms for F16 layers (fp16 MFMA, fp32
// accumulation: the F16 GEMMs and the causal attention's scores and P.V) are
// the default; Q3T_PF_EXACT=1 (read per call) keeps the exact f64-MFMA forms,
// whose rows equal the GEMV path's bit for bit.  Q8_0 layers keep the exact
// attention: their GEMM inputs are quantised per 32-block, so a difference at
// fp32 rounding level in an attention row can move a quantised value by a
// whole step, and 28 layers of such steps leave the logits ~3e-2 apart
// (measured on 200 rows), where the exact forms match the oracle bit for bit.
bool pf_exact() {
    const char * e = std::getenv("Q3T_PF_EXACT");
    return e && e[0] == '1';
}

bool pf_f16_fast(const q3t_config & g) {
    if (pf_exact()) return false;
    const int d = g.hidden_size, qd = g.n_head * g.head_dim, qkvd = qd + 2 * g.n_kv_head * g.head_dim;
    return d % 128 == 0 && qkvd % 128 == 0 && g.ffn_size % 128 == 0 && qd % pf::kHK == 0 && d % pf::kHK == 0 &&
           g.ffn_size <= 16 * kBlock;
}

// Causal attention of the n prefill rows (QKV rows in c->pf_qkv, K/V already
// in the layer's cache) into c->pf_att.  From 64 rows on: the MFMA kernels
// (scores, softmax, P.V; Q3T_PF_ATT_MFMA=0 keeps the row kernel), exact on f64
// MFMA or, fast, on fp16 (bfloat16) MFMA with fp32 accumulation; below, or
// when the scores would not fit 4 GiB, one workgroup per row.
int pf_attention(q3t_dev * c, const LayerDev & L, const uint16_t * kc, const uint16_t * vc, int n, int n_past,
                 bool fast) {
    const q3t_config & g = c->cfg;
    const int qd = g.n_head * g.head_dim, qkvd = qd + 2 * g.n_kv_head * g.head_dim;
    const float scale = 1.0f / std::sqrt((float) g.head_dim);
    const int bf = c->kv_bf16 ? 1 : 0;
    static const bool off = [] { const char * e = std::getenv("Q3T_PF_ATT_MFMA"); return e && e[0] == '0'; }();
    const int ls = (n_past + n + pf::kAT - 1) / pf::kAT * pf::kAT;
    const size_t cells = (size_t) g.n_head * n * ls;
    if (off || n < pf::kAT || cells * 6 > ((size_t) 4 << 30)) {
        hipLaunchKernelGGL(pf::k_attn_rows, dim3(g.n_head, n), dim3(kBlock), pf::attn_rows_lds_bytes(n_past + n),
                           c->stream, (const float *) c->pf_qkv, qkvd, L.q_norm, g.rms_eps, (const float *) c->rope_cos,
                           (const float *) c->rope_sin, kc, vc, c->n_ctx, g.n_head, g.n_kv_head, n_past, scale,
                           c->pf_att, qd, bf);
        return 0;
    }
    // the probabilities buffer also holds the q rows [n_head][n][128] first
    const size_t need = std::max(cells, (size_t) g.n_head * n * g.head_dim);
    if (need > c->pf_sp_cap) {
        dev_free(c, c->pf_s); dev_free(c, c->pf_p);
        c->pf_s = nullptr; c->pf_p = nullptr; c->pf_sp_cap = 0;
        if (dev_alloc_t(c, &c->pf_s, need) || dev_alloc_t(c, &c->pf_p, need)) return -1;
        c->pf_sp_cap = need;
    }
    const int nt = (n + pf::kAT - 1) / pf::kAT;
    // grid: heads x tile pairs x position / dim halves; an odd count's middle
    // tile dealt out over the pairs' workgroups by both kernels
    // (Q3T_PF_ATT_SPREAD=0 gives it a workgroup of its own)
    const char * se = std::getenv("Q3T_PF_ATT_SPREAD");  // read per call (tests switch it)
    const bool no_spread = se && se[0] == '0';
    const dim3 tiles(g.n_head, (nt % 2 && nt >= 3 && !no_spread) ? nt / 2 : (nt + 1) / 2, 2);
    // q rows into the probabilities buffer's head (they are consumed before it is written)
    uint16_t * qh = c->pf_p;
    hipLaunchKernelGGL(pf::k_att_q, dim3(n, (g.n_head + 3) / 4), dim3(kBlock), 0, c->stream, (const float *) c->pf_qkv,
                       qkvd, L.q_norm, g.rms_eps, (const float *) c->rope_cos, (const float *) c->rope_sin, n, n_past,
                       g.n_head, qh, bf);
    hipLaunchKernelGGL(fast ? pf::k_att_scores_fast : pf::k_att_scores, tiles, dim3(pf::kAttT), 0, c->stream,
                       (const uint16_t *) qh, kc, c->n_ctx, g.n_head, g.n_kv_head, n, n_past, scale, c->pf_s, ls, bf);
    hipLaunchKernelGGL(pf::k_att_softmax, dim3((n + 3) / 4, g.n_head), dim3(kBlock), 0, c->stream,
                       (const float *) c->pf_s, n, n_past, ls, c->pf_p, bf);
    hipLaunchKernelGGL(fast ? pf::k_att_pv_fast : pf::k_att_pv, tiles, dim3(pf::kAttT), 0, c->stream,
                       (const uint16_t *) c->pf_p, ls, vc, c->n_ctx, g.n_head, g.n_kv_head, n, n_past, c->pf_att, qd, bf);
    return 0;
}

// Talker prefill of n tokens (rows in c->stage) with F16 layers: by default on
// the fast fp16-MFMA GEMMs (fp32 accumulation, the inputs written as fp16
// rows by the RMSNorm, a rounding pass over the attention rows, and the
// SwiGLU's two-plane form for the widened ffn_down); with Q3T_PF_EXACT=1
// on the exact f64-MFMA GEMMs, whose rows equal the GEMV path's.  Same layer
// program and buffers as prefill_mfma (c->pf_f holds the RMSNorm'd rows of
// the exact form until SwiGLU overwrites it).
int prefill_f16(q3t_dev * c, int n, int n_past) {
    const q3t_config & g = c->cfg;
    const int d = g.hidden_size, qd = g.n_head * g.head_dim, kd = g.n_kv_head * g.head_dim, qkvd = qd + 2 * kd;
    const int ffn = g.ffn_size;
    const size_t lstride = (size_t) g.n_kv_head * c->n_ctx * g.head_dim;
    const float scale = 1.0f / std::sqrt((float) g.head_dim);
    const float * x = c->stage;
    const bool fast = pf_f16_fast(g);
    for (int il = 0; il < g.n_layers && fast; ++il) {
        const LayerDev & L = c->talker[il];
        uint16_t * kc = c->kc + il * lstride;
        uint16_t * vc = c->vc + il * lstride;
        hipLaunchKernelGGL(pf::k_rmsnorm_rows_h16, dim3(n), dim3(kBlock), 0, c->stream, x, L.attn_norm, g.rms_eps, d,
                           c->pf_h);
        pf_gemm_h16(c, L.qkv, qkvd, d, n, c->pf_h, nullptr, d, nullptr, c->pf_qkv, nullptr, 0);
        hipLaunchKernelGGL(pf::k_kv_rows, dim3(n, (g.n_kv_head + 3) / 4), dim3(kBlock), 0, c->stream, (const float *) c->pf_qkv,
                           qkvd, qd, kd, L.k_norm, g.rms_eps, (const float *) c->rope_cos, (const float *) c->rope_sin,
                           kc, vc, c->n_ctx, n_past, c->kv_bf16 ? 1 : 0);
        if (pf_attention(c, L, kc, vc, n, n_past, true)) return -1;
        const size_t na = (size_t) n * qd;
        hipLaunchKernelGGL(pf::k_rows_h16, dim3((unsigned) std::min<size_t>((na + kBlock - 1) / kBlock, 4096)),
                           dim3(kBlock), 0, c->stream, (const float *) c->pf_att, qd, qd, n, c->pf_h);
        pf_gemm_h16(c, L.wo, d, qd, n, c->pf_h, nullptr, qd, nullptr, c->pf_xb, x, d);
        hipLaunchKernelGGL(pf::k_rmsnorm_rows_h16, dim3(n), dim3(kBlock), 0, c->stream, (const float *) c->pf_xb,
                           L.ffn_norm, g.rms_eps, d, c->pf_h);
        pf_gemm_h16(c, L.wg, ffn, d, n, c->pf_h, nullptr, d, nullptr, c->pf_g, nullptr, 0);
        pf_gemm_h16(c, L.wu, ffn, d, n, c->pf_h, nullptr, d, nullptr, c->pf_u, nullptr, 0);
        hipLaunchKernelGGL(pf::k_swiglu_h16, dim3(n), dim3(kBlock), 0, c->stream, (const float *) c->pf_g,
                           (const float *) c->pf_u, ffn, c->pf_h, c->pf_l, c->pf_sc);
        pf_gemm_h16(c, L.wd, d, ffn, n, c->pf_h, c->pf_l, ffn, c->pf_sc, c->pf_xa, c->pf_xb, d);
        x = c->pf_xa;
    }
    for (int il = 0; il < g.n_layers && !fast; ++il) {
        const LayerDev & L = c->talker[il];
        uint16_t * kc = c->kc + il * lstride;
        uint16_t * vc = c->vc + il * lstride;
        hipLaunchKernelGGL(k_rmsnorm_rows, dim3(n), dim3(kBlock), 0, c->stream, x, L.attn_norm, g.rms_eps, d, c->pf_f);
        pf_gemm_f16(c, L.qkv, qkvd, d, n, c->pf_f, d, false, c->pf_qkv, nullptr, 0);
        hipLaunchKernelGGL(pf::k_kv_rows, dim3(n, (g.n_kv_head + 3) / 4), dim3(kBlock), 0, c->stream, (const float *) c->pf_qkv,
                           qkvd, qd, kd, L.k_norm, g.rms_eps, (const float *) c->rope_cos, (const float *) c->rope_sin,
                           kc, vc, c->n_ctx, n_past, c->kv_bf16 ? 1 : 0);
        if (pf_attention(c, L, kc, vc, n, n_past, false)) return -1;
        pf_gemm_f16(c, L.wo, d, qd, n, c->pf_att, qd, false, c->pf_xb, x, d);
        hipLaunchKernelGGL(k_rmsnorm_rows, dim3(n), dim3(kBlock), 0, c->stream, (const float *) c->pf_xb, L.ffn_norm,
                           g.rms_eps, d, c->pf_f);
        pf_gemm_f16(c, L.wg, ffn, d, n, c->pf_f, d, false, c->pf_g, nullptr, 0);
        pf_gemm_f16(c, L.wu, ffn, d, n, c->pf_f, d, false, c->pf_u, nullptr, 0);
        const size_t cnt = (size_t) n * ffn;
        hipLaunchKernelGGL(pf::k_swiglu_rows, dim3((unsigned) std::min<size_t>((cnt + kBlock - 1) / kBlock, 4096)),
                           dim3(kBlock), 0, c->stream, (const float *) c->pf_g, (const float *) c->pf_u, c->pf_f, cnt);
        pf_gemm_f16(c, L.wd, d, ffn, n, c->pf_f, ffn, true, c->pf_xa, c->pf_xb, d);
        x = c->pf_xa;
    }
    GemvSpec h{};
    h.w = weight_of(c->codec_head); h.rows = g.codec_vocab; h.K = d;
    h.x = c->pf_xa + (size_t) (n - 1) * d; h.x_stride = d; h.norm_w = (const float *) c->out_norm.data;
    h.hidden_out = c->hidden; h.hidden_stride = d; h.y = c->logits; h.y_stride = g.codec_vocab;
    gemv(c, h, 1);
    return 0;
}

// Talker prefill of n tokens (rows in c->stage) on the MFMA path; the output
// rows end in c->pf_xa, the last row's head output in c->hidden / c->logits.
int prefill_mfma(q3t_dev * c, int n, int n_past) {
    const q3t_config & g = c->cfg;
    const int d = g.hidden_size, qd = g.n_head * g.head_dim, kd = g.n_kv_head * g.head_dim, qkvd = qd + 2 * kd;
    const int ffn = g.ffn_size;
    const size_t lstride = (size_t) g.n_kv_head * c->n_ctx * g.head_dim;
    const float scale = 1.0f / std::sqrt((float) g.head_dim);
    const float * x = c->stage;
    for (int il = 0; il < g.n_layers; ++il) {
        const LayerDev & L = c->talker[il];
        uint16_t * kc = c->kc + il * lstride;
        uint16_t * vc = c->vc + il * lstride;
        pf_quant(c, x, n, d, L.attn_norm);
        pf_gemm(c, L.qkv, qkvd, d, n, c->pf_qkv, nullptr);
        hipLaunchKernelGGL(pf::k_kv_rows, dim3(n, (g.n_kv_head + 3) / 4), dim3(kBlock), 0, c->stream, (const float *) c->pf_qkv,
                           qkvd, qd, kd, L.k_norm, g.rms_eps, (const float *) c->rope_cos, (const float *) c->rope_sin,
                           kc, vc, c->n_ctx, n_past, c->kv_bf16 ? 1 : 0);
        if (pf_attention(c, L, kc, vc, n, n_past, false)) return -1;
        pf_quant(c, c->pf_att, n, qd, nullptr);
        pf_gemm(c, L.wo, d, qd, n, c->pf_xb, x);
        pf_quant(c, c->pf_xb, n, d, L.ffn_norm);
        pf_gemm(c, L.wg, ffn, d, n, c->pf_g, nullptr);
        pf_gemm(c, L.wu, ffn, d, n, c->pf_u, nullptr);
        pf_quant(c, c->pf_g, n, ffn, nullptr, -1, nullptr, nullptr, c->pf_u);   // SwiGLU fused into the quantisation
        pf_gemm(c, L.wd, d, ffn, n, c->pf_xa, c->pf_xb);
        x = c->pf_xa;
    }
    GemvSpec h{};
    h.w = weight_of(c->codec_head); h.rows = g.codec_vocab; h.K = d;
    h.x = c->pf_xa + (size_t) (n - 1) * d; h.x_stride = d; h.norm_w = (const float *) c->out_norm.data;
    h.hidden_out = c->hidden; h.hidden_stride = d; h.y = c->logits; h.y_stride = g.codec_vocab;
    gemv(c, h, 1);
    return 0;
}

// y [n][N] = x [n][K] . W^T + bias on the tiled GEMMs (Q8_0: quantised rows on
// int8 MFMA; F16: the exact VALU GEMM, x rounded to fp16): the GEMV's
// EPI_BIAS, with the bias as a residual of row stride 0.
// q, dx: room for the n quantised rows of x (Q8_0 weights).
void pf_linear_bias(q3t_dev * c, const Slot & w, int N, int K, int n, const float * x, const Slot & bias, float * y,
                    int8_t * q, float * dx) {
    if (w.type == Q3T_TYPE_Q8_0) {
        pf_quant(c, x, n, K, nullptr, K, q, dx);
        pf_gemm(c, w, N, K, n, y, (const float *) bias.data, 0, q, dx);
    } else {
        pf_gemm_f16(c, w, N, K, n, x, K, false, y, (const float *) bias.data, 0);
    }
}

bool text_proj_tiled(const q3t_dev * c, int n) {
    const char * e = std::getenv("Q3T_PREFILL_MFMA");
    if (e && e[0] == '0') return false;
    if (!(e && e[0] == '1') && n < 16) return false;
    const int te = c->cfg.text_embd_dim, d = c->cfg.hidden_size;
    const auto ok = [](const Slot & s) { return s.type == Q3T_TYPE_Q8_0 || s.type == Q3T_TYPE_F16; };
    return ok(c->fc1) && ok(c->fc2) && te % 128 == 0 && d % pf::kTile == 0;
}

// project_text_tokens (src/tts_transformer.cpp:963-1028) of n ids into the
// device rows dst [n][d]: text_embd rows -> fc1 + bias -> SiLU -> fc2 + bias.
// n >= 16 runs the tiled GEMMs, fewer rows the GEMV in chunks of up to 4;
// rows are independent and both forms keep one numerics contract, so a row's
// result does not depend on n.  ids are range-checked by the caller.
// Work buffers of one text projection of n ids: the ids on the device,
// the gathered text_embd rows [n][te], the fc1 output (tiled: [n][te]; GEMV:
// [4][te]) and the Q8_0 copies of the tiled GEMMs' input rows ([n][te] int8,
// [n][te/32] scales).
struct ProjWork {
    const int32_t * ids; float * rows; float * h; int8_t * q; float * dx;
};

int proj_tensors_ok(q3t_dev * c) {
    if (!c->text_embd.data || !c->fc1.data || !c->fc1_b.data || !c->fc2.data || !c->fc2_b.data)
        return fail(c, "text projection tensors missing");
    if (c->text_embd.type != Q3T_TYPE_F16) return fail(c, "talker.text_embd must be F16");
    return 0;
}

// The kernels of project_text_tokens on n ids already on the device.
void project_rows_core(q3t_dev * c, int32_t n, const ProjWork & w, float * dst) {
    const q3t_config & g = c->cfg;
    const int te = g.text_embd_dim, d = g.hidden_size;
    hipLaunchKernelGGL(k_gather_rows, dim3((te + 255) / 256, n), dim3(256), 0, c->stream,
                       (const uint16_t *) c->text_embd.data, (int64_t) te, w.ids, n, w.rows);
    if (text_proj_tiled(c, n)) {
        pf_linear_bias(c, c->fc1, te, te, n, w.rows, c->fc1_b, w.h, w.q, w.dx);
        const size_t cnt = (size_t) n * te;
        hipLaunchKernelGGL(k_silu_rows, dim3((unsigned) std::min<size_t>((cnt + 255) / 256, 4096)), dim3(256), 0,
                           c->stream, w.h, cnt);
        pf_linear_bias(c, c->fc2, d, te, n, w.h, c->fc2_b, dst, w.q, w.dx);
    } else {
        for (int t0 = 0; t0 < n;) {
            const int left = n - t0;
            const int nt = left >= 4 ? 4 : left >= 2 ? 2 : 1;
            GemvSpec a{};
            a.w = weight_of(c->fc1); a.rows = te; a.K = te; a.x = w.rows + (size_t) t0 * te; a.x_stride = te;
            a.y = w.h; a.y_stride = te; a.bias = (const float *) c->fc1_b.data; a.epi = EPI_BIAS_SILU;
            a.no_done = true;
            gemv(c, a, nt);
            GemvSpec b{};
            b.w = weight_of(c->fc2); b.rows = d; b.K = te; b.x = w.h; b.x_stride = te;
            b.y = dst + (size_t) t0 * d; b.y_stride = d; b.bias = (const float *) c->fc2_b.data; b.epi = EPI_BIAS;
            b.no_done = true;
            gemv(c, b, nt);
            t0 += nt;
        }
    }
}

int project_rows(q3t_dev * c, const int32_t * tokens, int32_t n, float * dst) {
    const q3t_config & g = c->cfg;
    if (proj_tensors_ok(c)) return -1;
    if (n > c->ids_cap) {
        dev_free(c, c->ids);
        c->ids = nullptr;
        if (dev_alloc_t(c, &c->ids, (size_t) n)) return -1;
        c->ids_cap = n;
    }
    if (ensure_stage(c, n)) return -1;
    const int te = g.text_embd_dim;
    HIP_OK(hipMemcpyAsync(c->ids, tokens, (size_t) n * 4, hipMemcpyHostToDevice, c->stream));
    ProjWork w{c->ids, c->stage, c->tp_a, nullptr, nullptr};
    if (text_proj_tiled(c, n)) {
        if (n > c->bp_rows) {
            for (void * p : {(void *) c->bp_q, (void *) c->bp_dx, (void *) c->bp_h}) dev_free(c, p);
            c->bp_q = nullptr; c->bp_dx = nullptr; c->bp_h = nullptr; c->bp_rows = 0;
            if (dev_alloc_t(c, &c->bp_q, (size_t) n * te) || dev_alloc_t(c, &c->bp_dx, (size_t) n * (te / kQK)) ||
                dev_alloc_t(c, &c->bp_h, (size_t) n * te))
                return -1;
            c->bp_rows = n;
        }
        w.h = c->bp_h; w.q = c->bp_q; w.dx = c->bp_dx;
    }
    project_rows_core(c, n, w, dst);
    HIP_OK(hipGetLastError());
    return 0;
}

// Room for m projected rows, r assembled rows and f reference frames.
int ensure_build(q3t_dev * c, int m, int r, int f) {
    const int d = c->cfg.hidden_size;
    if (m + r > c->bp_out_rows) {
        for (void * p : {(void *) c->bp_proj, (void *) c->bp_out, (void *) c->bp_spec}) dev_free(c, p);
        c->bp_proj = nullptr; c->bp_out = nullptr; c->bp_spec = nullptr; c->bp_out_rows = 0;
        const int cap = std::max(m + r, 64);
        if (dev_alloc_t(c, &c->bp_proj, (size_t) cap * d) || dev_alloc_t(c, &c->bp_out, (size_t) cap * d) ||
            dev_alloc_t(c, &c->bp_spec, (size_t) cap))
            return -1;
        c->bp_out_rows = cap;
    }
    if (!c->bp_spk && dev_alloc_t(c, &c->bp_spk, (size_t) d)) return -1;
    if (f > c->bp_frames_cap) {
        dev_free(c, c->bp_frames);
        c->bp_frames = nullptr; c->bp_frames_cap = 0;
        if (dev_alloc_t(c, &c->bp_frames, (size_t) f * 16)) return -1;
        c->bp_frames_cap = f;
    }
    return 0;
}

// Projects ids, assembles specs.size() rows and copies them out: rows
// [0, n_pre) to prefill_out, the next n_trail to trailing_out, the last to
// pad_out.  frames: ICL reference codes (n_frames x 16) or null.
int build_rows(q3t_dev * c, const std::vector<int32_t> & ids, const std::vector<RowSpec> & specs,
               const float * speaker, const int32_t * frames, int32_t n_frames, int32_t n_pre, int32_t n_trail,
               float * prefill_out, float * trailing_out, float * pad_out) {
    const q3t_config & g = c->cfg;
    const int d = g.hidden_size, m = (int) ids.size(), r = (int) specs.size();
    if (!c->codec_embd.data || c->codec_embd.type != Q3T_TYPE_F16) return fail(c, "talker.codec_embd must be F16");
    for (int i = 0; frames && i < g.n_codebooks - 1; ++i)
        if (!c->cp_embd[i].data || c->cp_embd[i].type != Q3T_TYPE_F16 || c->cp_embd[i].ne0 != d)
            return fail(c, "code_pred.codec_embd tables must be F16 rows of hidden_size");
    if (ensure_build(c, m, r, n_frames)) return -1;
    if (project_rows(c, ids.data(), m, c->bp_proj)) return -1;
    HIP_OK(hipMemcpyAsync(c->bp_spec, specs.data(), (size_t) r * sizeof(RowSpec), hipMemcpyHostToDevice, c->stream));
    if (speaker)
        HIP_OK(hipMemcpyAsync(c->bp_spk, speaker, (size_t) d * 4, hipMemcpyHostToDevice, c->stream));
    if (n_frames > 0)
        HIP_OK(hipMemcpyAsync(c->bp_frames, frames, (size_t) n_frames * 16 * 4, hipMemcpyHostToDevice, c->stream));
    RowTables T{};
    T.proj = c->bp_proj; T.codec_embd = (const uint16_t *) c->codec_embd.data;
    for (int i = 0; frames && i < g.n_codebooks - 1; ++i) T.cp_embd[i] = (const uint16_t *) c->cp_embd[i].data;
    T.speaker = c->bp_spk; T.frames = c->bp_frames; T.n_cb = g.n_codebooks; T.d = d;
    hipLaunchKernelGGL(k_prefill_rows, dim3((d + 255) / 256, r), dim3(256), 0, c->stream, T,
                       (const RowSpec *) c->bp_spec, c->bp_out);
    HIP_OK(hipGetLastError());
    HIP_OK(hipMemcpyAsync(prefill_out, c->bp_out, (size_t) n_pre * d * 4, hipMemcpyDeviceToHost, c->stream));
    if (n_trail > 0)
        HIP_OK(hipMemcpyAsync(trailing_out, c->bp_out + (size_t) n_pre * d, (size_t) n_trail * d * 4,
                              hipMemcpyDeviceToHost, c->stream));
    HIP_OK(hipMemcpyAsync(pad_out, c->bp_out + (size_t) (n_pre + n_trail) * d, (size_t) d * 4, hipMemcpyDeviceToHost,
                          c->stream));
    return sync(c);
}

}  // namespace

extern "C" {

int q3t_dev_prefill(q3t_dev * c, const float * embd, int32_t n, int32_t n_past, float * hidden_out, float * logits_out) {
    if (!c || !embd) return -1;
    if (n <= 0) return fail(c, "n_tokens must be > 0");
    HIP_OK(hipSetDevice(c->device));
    if (check_ready(c)) return -1;
    if (n_past < 0 || n_past + n > c->n_ctx) return fail(c, "Context length exceeded");
    const q3t_config & g = c->cfg;
    const int d = g.hidden_size;
    if (ensure_stage(c, n)) return -1;
    if (hidden_out && n > c->hidden_all_rows) {
        dev_free(c, c->hidden_all);
        c->hidden_all = nullptr;
        if (dev_alloc_t(c, &c->hidden_all, (size_t) n * d)) return -1;
        c->hidden_all_rows = n;
    }
    FrameState s{};
    if (set_state(c, s)) return -1;
    HIP_OK(hipMemcpyAsync(c->stage, embd, (size_t) n * d * 4, hipMemcpyHostToDevice, c->stream));
    if (const int tp = tiled_prefill(c, n)) {
        if (ensure_pf(c, n)) return -1;
        if (tp == 1 ? prefill_mfma(c, n, n_past) : prefill_f16(c, n, n_past)) return -1;
        if (hidden_out)
            hipLaunchKernelGGL(k_rmsnorm_rows, dim3(n), dim3(kBlock), 0, c->stream, (const float *) c->pf_xa,
                               (const float *) c->out_norm.data, g.rms_eps, d, c->hidden_all);
        if (hidden_out) HIP_OK(hipMemcpyAsync(hidden_out, c->hidden_all, (size_t) n * d * 4, hipMemcpyDeviceToHost, c->stream));
        if (logits_out) HIP_OK(hipMemcpyAsync(logits_out, c->logits, (size_t) g.codec_vocab * 4, hipMemcpyDeviceToHost, c->stream));
        return sync(c);
    }
    for (int t0 = 0; t0 < n;) {
        const int left = n - t0;
        const int nt = left >= 4 ? 4 : left >= 2 ? 2 : 1;
        const bool last = t0 + nt == n;
        talker_chunk(c, c->stage + (size_t) t0 * d, nt, nullptr, n_past + t0, last);
        if (hidden_out)
            hipLaunchKernelGGL(k_rmsnorm_rows, dim3(nt), dim3(kBlock), 0, c->stream, c->xa,
                               (const float *) c->out_norm.data, g.rms_eps, d, c->hidden_all + (size_t) t0 * d);
        t0 += nt;
    }
    if (hidden_out) HIP_OK(hipMemcpyAsync(hidden_out, c->hidden_all, (size_t) n * d * 4, hipMemcpyDeviceToHost, c->stream));
    if (logits_out) HIP_OK(hipMemcpyAsync(logits_out, c->logits, (size_t) g.codec_vocab * 4, hipMemcpyDeviceToHost, c->stream));
    return sync(c);
}

}  // extern "C"

namespace {

// The pinned staging buffer of the single-step calls, grown to `need` bytes.
int ensure_pin(q3t_dev * c, size_t need) {
    if (c->pin_bytes >= need) return 0;
    if (c->pin) (void) hipHostFree(c->pin);
    c->pin = nullptr; c->pin_bytes = 0;
    HIP_OK(hipHostMalloc((void **) &c->pin, need, hipHostMallocDefault));
    c->pin_bytes = need;
    return 0;
}

}  // namespace

extern "C" {

int q3t_dev_talker_step(q3t_dev * c, const float * embd, int32_t n_past, float * logits_out, float * hidden_out) {
    if (!c || !embd) return fail(c, "step_embd is null");
    HIP_OK(hipSetDevice(c->device));
    if (check_ready(c)) return -1;
    if (n_past < 0 || n_past + 1 > c->n_ctx) return fail(c, "Context length exceeded");
    const q3t_config & g = c->cfg;
    const size_t d4 = (size_t) g.hidden_size * 4, v4 = (size_t) g.codec_vocab * 4;
    // staging layout: [FrameState | pad to 256][embd d][logits vocab][hidden d][err]
    static_assert(sizeof(FrameState) <= 256, "FrameState outgrew its staging slot");
    const size_t o_embd = 256, o_logits = o_embd + d4, o_hidden = o_logits + v4, o_err = o_hidden + d4;
    if (ensure_pin(c, o_err + 256)) return -1;
    FrameState s{};
    s.talker_pos = n_past;
    std::memcpy(c->pin, &s, sizeof s);
    std::memcpy(c->pin + o_embd, embd, d4);
    HIP_OK(hipMemcpyAsync(c->st, c->pin, sizeof s, hipMemcpyHostToDevice, c->stream));
    HIP_OK(hipMemcpyAsync(c->stage, c->pin + o_embd, d4, hipMemcpyHostToDevice, c->stream));
    bool ran = false;
    if (fk_step(c, 0, fk::MODE_TALKER_STEP, ran)) return -1;
    if (!ran) talker_chunk(c, c->stage, 1, &c->st->talker_pos, 0, true, true);
    if (logits_out) HIP_OK(hipMemcpyAsync(c->pin + o_logits, c->logits, v4, hipMemcpyDeviceToHost, c->stream));
    if (hidden_out) HIP_OK(hipMemcpyAsync(c->pin + o_hidden, c->hidden, d4, hipMemcpyDeviceToHost, c->stream));
    if (ran) HIP_OK(hipMemcpyAsync(c->pin + o_err, c->fk_err, 4, hipMemcpyDeviceToHost, c->stream));
    if (sync(c)) return -1;
    if (!ran && c->attn_layer >= 0 && keep_attn_row(c, n_past + 1)) return -1;
    if (logits_out) std::memcpy(logits_out, c->pin + o_logits, v4);
    if (hidden_out) std::memcpy(hidden_out, c->pin + o_hidden, d4);
    if (ran) {
        int32_t err = 0;
        std::memcpy(&err, c->pin + o_err, 4);
        if (err) return fail(c, fk_err_msg(err));
    }
    return 0;
}

int q3t_dev_predict_codes(q3t_dev * c, const float * hidden, const int32_t * prev_codes, float * logits_out) {
    if (!c || !hidden || !logits_out) return -1;
    HIP_OK(hipSetDevice(c->device));
    if (resolve(c)) return -1;
    const q3t_config & g = c->cfg;
    const int ng = g.n_codebooks - 1;
    SingleInArgs in{};
    in.n = prev_codes ? ng : 0;
    for (int i = 0; i < in.n; ++i) {
        if (prev_codes[i] < 0 || prev_codes[i] >= g.cp_vocab) return fail(c, "Embedding token ID out of range");
        in.codes[i] = prev_codes[i];
        in.embd[i] = (const uint16_t *) c->cp_embd[i].data;
    }
    const size_t d4 = (size_t) g.hidden_size * 4, l4 = (size_t) ng * g.cp_vocab * 4;
    if (ensure_pin(c, d4 + l4)) return -1;
    std::memcpy(c->pin, hidden, d4);
    HIP_OK(hipMemcpyAsync(c->stage, c->pin, d4, hipMemcpyHostToDevice, c->stream));
    code_pred_single(c, in);
    HIP_OK(hipMemcpyAsync(c->pin + d4, c->cp_logits, l4, hipMemcpyDeviceToHost, c->stream));
    if (sync(c)) return -1;
    std::memcpy(logits_out, c->pin + d4, l4);
    return 0;
}

int q3t_dev_code_pred(q3t_dev * c, const float * hidden, int32_t cb0, const q3t_sampling * sampling, uint32_t frame,
                      int32_t * codes_out, float * logits_out) {
    if (!c || !hidden || !codes_out) return -1;
    HIP_OK(hipSetDevice(c->device));
    if (resolve(c)) return -1;
    if (!c->cpk) return fail(c, "KV cache not reserved");
    const q3t_config & g = c->cfg;
    if (cb0 < 0 || cb0 >= g.codec_vocab) return fail(c, "Embedding token ID out of range");
    // pinned staging: [SampleParams][FrameState in][hidden d][FrameState out][logits 15 x vocab][err]
    static_assert(sizeof(SampleParams) <= 256 && sizeof(FrameState) <= 256, "staging slots");
    const size_t d4 = (size_t) g.hidden_size * 4, l4 = (size_t) (g.n_codebooks - 1) * g.cp_vocab * 4;
    const size_t o_st = 256, o_hid = 512, o_out = o_hid + d4, o_log = o_out + 256, o_err = o_log + l4;
    if (ensure_pin(c, o_err + 256)) return -1;
    SampleParams p{};
    p.temperature = sampling ? sampling->temperature : 0.0f;
    p.top_k = sampling ? sampling->top_k : 0;
    p.rep_penalty = 1.0f;
    p.seed = sampling ? sampling->seed : 0;
    FrameState s{};
    s.codes[0] = cb0;
    s.frame = (int32_t) frame;
    std::memcpy(c->pin, &p, sizeof p);
    std::memcpy(c->pin + o_st, &s, sizeof s);
    std::memcpy(c->pin + o_hid, hidden, d4);
    HIP_OK(hipMemcpyAsync(c->params, c->pin, sizeof p, hipMemcpyHostToDevice, c->stream));
    HIP_OK(hipMemcpyAsync(c->st, c->pin + o_st, sizeof s, hipMemcpyHostToDevice, c->stream));
    HIP_OK(hipMemcpyAsync(c->hidden, c->pin + o_hid, d4, hipMemcpyHostToDevice, c->stream));
    // the persistent kernel needs the talker KV reservation for its tables
    bool ran = false;
    if (c->kc && fk_step(c, (int32_t) frame, fk::MODE_CODE_PRED, ran)) return -1;
    if (ran) {
        if (logits_out) {
            // arena slots of one code-predictor pass (the input row, the
            // mtp_proj output in the 1.7B layout, the layers, the head): the
            // head's logits sit in its last slot
            const int mtp = g.cp_hidden != g.hidden_size ? 1 : 0;
            const int stride = 2 + mtp + (fk_xcd(c->fk_variant) ? 15 : 5) * g.cp_layers, n = g.n_codebooks - 1;
            hipLaunchKernelGGL(k_untag_heads, dim3((n * g.cp_vocab + 255) / 256), dim3(256), 0, c->stream,
                               c->fk_arena, stride - 1, stride, n, g.cp_vocab, c->cp_logits);
        }
    } else {
        hipLaunchKernelGGL(k_cp_input, dim3((g.hidden_size + 255) / 256), dim3(256), 0, c->stream, c->st, c->hidden,
                           (const uint16_t *) c->codec_embd.data, g.hidden_size, c->stage);
        code_pred_seq(c, false);
    }
    HIP_OK(hipMemcpyAsync(c->pin + o_out, c->st, sizeof(FrameState), hipMemcpyDeviceToHost, c->stream));
    if (logits_out) HIP_OK(hipMemcpyAsync(c->pin + o_log, c->cp_logits, l4, hipMemcpyDeviceToHost, c->stream));
    if (ran) HIP_OK(hipMemcpyAsync(c->pin + o_err, c->fk_err, 4, hipMemcpyDeviceToHost, c->stream));
    if (sync(c)) return -1;
    if (ran) {
        int32_t err = 0;
        std::memcpy(&err, c->pin + o_err, 4);
        if (err) return fail(c, fk_err_msg(err));
    }
    FrameState r{};
    std::memcpy(&r, c->pin + o_out, sizeof r);
    if (logits_out) std::memcpy(logits_out, c->pin + o_log, l4);
    for (int i = 0; i < g.n_codebooks - 1; ++i) codes_out[i] = r.codes[i + 1];
    return 0;
}

int q3t_dev_text_proj(q3t_dev * c, const int32_t * tokens, int32_t n, float * out) {
    if (!c || !tokens || !out) return -1;
    if (n <= 0) return 0;
    HIP_OK(hipSetDevice(c->device));
    const q3t_config & g = c->cfg;
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= g.text_vocab) return fail(c, "Embedding token ID out of range");
    if (ensure_build(c, n, 0, 0)) return -1;
    if (project_rows(c, tokens, n, c->bp_proj)) return -1;
    HIP_OK(hipMemcpyAsync(out, c->bp_proj, (size_t) n * g.hidden_size * 4, hipMemcpyDeviceToHost, c->stream));
    return sync(c);
}

int q3t_dev_text_proj_noalloc(q3t_dev * c, const int32_t * tokens, int32_t n, float * out) {
    if (!c || !tokens || !out) return -1;
    if (n <= 0) return 0;
    if (n > kNoAllocMaxIds) return fail(c, "text_proj_noalloc: at most 64 ids per call");
    HIP_OK(hipSetDevice(c->device));
    const q3t_config & g = c->cfg;
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= g.text_vocab) return fail(c, "Embedding token ID out of range");
    if (proj_tensors_ok(c)) return -1;
    if (!c->scratch) return fail(c, "text_proj_noalloc: device scratch not set up");
    const int te = g.text_embd_dim, d = g.hidden_size;
    // carve the scratch: every region 256-byte aligned
    size_t off = 0;
    auto take = [&](size_t bytes) {
        unsigned char * p = c->scratch + off;
        off += (bytes + 255) & ~(size_t) 255;
        return p;
    };
    const size_t rows = (size_t) std::max(n, 4);   // the GEMV form writes fc1 rows in chunks of 4
    int32_t * ids = (int32_t *) take((size_t) n * 4);
    ProjWork w{ids, (float *) take(rows * te * 4), (float *) take(rows * te * 4), (int8_t *) take((size_t) n * te),
               (float *) take((size_t) n * (te / kQK) * 4)};
    float * res = (float *) take((size_t) n * d * 4);
    if (off > kScratchBytes) return fail(c, "text_proj_noalloc: widths too large for the device scratch");
    HIP_OK(hipMemcpyAsync(ids, tokens, (size_t) n * 4, hipMemcpyHostToDevice, c->stream));
    project_rows_core(c, n, w, res);
    HIP_OK(hipGetLastError());
    HIP_OK(hipMemcpyAsync(out, res, (size_t) n * d * 4, hipMemcpyDeviceToHost, c->stream));
    return sync(c);
}

int q3t_dev_build_prefill(q3t_dev * c, const int32_t * text_tokens, int32_t n_tokens, const float * speaker_embd,
                          int32_t language_id, const int32_t * instruct_tokens, int32_t n_instruct,
                          float * prefill_out, int32_t * n_prefill_out, float * trailing_out,
                          int32_t * n_trailing_out, float * tts_pad_out) {
    if (!c || !n_prefill_out || !n_trailing_out) return -1;
    if (!text_tokens) return fail(c, "text_tokens is null");
    if (n_tokens < 4) return fail(c, "Need at least 4 text tokens for prefill");
    const q3t_config & g = c->cfg;
    if (!instruct_tokens || n_instruct < 0) n_instruct = 0;
    const int n_codec_tok = language_id < 0 ? 3 : 4;
    const int in_len = n_codec_tok + (speaker_embd ? 1 : 0) + 2, ov_len = in_len - 1;
    const int n_trail = std::max(0, n_tokens - 9);
    const int n_pre = n_instruct + 3 + ov_len + 1;
    *n_prefill_out = n_pre;
    *n_trailing_out = n_trail + 1;
    if (!prefill_out) return 0;
    if (!trailing_out || !tts_pad_out) return fail(c, "output buffers are null");
    HIP_OK(hipSetDevice(c->device));
    // projected ids: bos, eos, pad, text[0..3], instruct, text[4 .. 4 + n_trail)
    std::vector<int32_t> ids = {g.tts_bos_id, g.tts_eos_id, g.tts_pad_id, text_tokens[0], text_tokens[1],
                                text_tokens[2], text_tokens[3]};
    ids.insert(ids.end(), instruct_tokens, instruct_tokens + n_instruct);
    ids.insert(ids.end(), text_tokens + 4, text_tokens + 4 + n_trail);
    for (int32_t t : ids)
        if (t < 0 || t >= g.text_vocab) return fail(c, "Embedding token ID out of range");
    std::vector<RowSpec> cin;   // the codec input rows as sources
    const int32_t think[4] = {language_id < 0 ? g.codec_nothink_id : g.codec_think_id, g.codec_think_bos_id,
                              language_id, g.codec_think_eos_id};
    for (int k = 0; k < 4; ++k) {
        if (language_id < 0 && k == 2) continue;
        cin.push_back({0, RS_CODEC, think[k], 0, 0});
    }
    if (speaker_embd) cin.push_back({0, RS_SPEAKER, 0, 0, 0});
    cin.push_back({0, RS_CODEC, g.codec_pad_id, 0, 0});
    cin.push_back({0, RS_CODEC, g.codec_bos_id, 0, 0});
    for (const RowSpec & r : cin)
        if (r.a_src == RS_CODEC && (r.a_idx < 0 || r.a_idx >= g.codec_vocab))
            return fail(c, "Embedding token ID out of range");
    const int P_BOS = 0, P_EOS = 1, P_PAD = 2, P_ROLE = 3, P_FIRST = 6, P_INSTR = 7, P_TRAIL = 7 + n_instruct;
    std::vector<RowSpec> sp;
    for (int i = 0; i < n_instruct; ++i) sp.push_back({RO_COPY, RS_PROJ, P_INSTR + i, 0, 0});
    for (int i = 0; i < 3; ++i) sp.push_back({RO_COPY, RS_PROJ, P_ROLE + i, 0, 0});
    for (int t = 0; t < ov_len; ++t)
        sp.push_back({RO_ADD, RS_PROJ, t == ov_len - 1 ? P_BOS : P_PAD, cin[t].a_src, cin[t].a_idx});
    sp.push_back({RO_ADD, RS_PROJ, P_FIRST, cin[in_len - 1].a_src, cin[in_len - 1].a_idx});
    for (int j = 0; j < n_trail; ++j) sp.push_back({RO_COPY, RS_PROJ, P_TRAIL + j, 0, 0});
    sp.push_back({RO_COPY, RS_PROJ, P_EOS, 0, 0});
    sp.push_back({RO_COPY, RS_PROJ, P_PAD, 0, 0});
    return build_rows(c, ids, sp, speaker_embd, nullptr, 0, n_pre, n_trail + 1, prefill_out, trailing_out,
                      tts_pad_out);
}

int q3t_dev_build_prefill_icl(q3t_dev * c, const int32_t * text_tokens, int32_t n_tokens,
                              const int32_t * ref_text_tokens, int32_t n_ref_text, const int32_t * ref_codec_tokens,
                              int32_t n_ref_frames, const float * speaker_embd, float * prefill_out,
                              int32_t * n_prefill_out, float * trailing_out, int32_t * n_trailing_out,
                              float * tts_pad_out) {
    if (!c || !n_prefill_out || !n_trailing_out) return -1;
    if (!text_tokens || n_tokens < 4) return fail(c, "ICL: need at least 4 target text tokens");
    if (!ref_codec_tokens || n_ref_frames < 1) return fail(c, "ICL: need at least 1 reference codec frame");
    if (!ref_text_tokens || n_ref_text < 0) n_ref_text = 0;
    const q3t_config & g = c->cfg;
    // text stream: ref_text[3:-5] ++ target[3:-5] ++ tts_eos
    std::vector<int32_t> stream;
    for (int32_t i = 3; i < std::max(3, n_ref_text - 5) && i < n_ref_text; ++i) stream.push_back(ref_text_tokens[i]);
    for (int32_t i = 3; i < std::max(3, n_tokens - 5) && i < n_tokens; ++i) stream.push_back(text_tokens[i]);
    stream.push_back(g.tts_eos_id);
    const int n_text = (int) stream.size(), n_codec = n_ref_frames + 1;
    const int in_len = 3 + (speaker_embd ? 1 : 0) + 2, ov_len = in_len - 1;
    const int n_pre = 3 + ov_len + n_codec, n_trail = std::max(0, n_text - n_codec);
    *n_prefill_out = n_pre;
    *n_trailing_out = n_trail;
    if (!prefill_out) return 0;
    if ((n_trail > 0 && !trailing_out) || !tts_pad_out) return fail(c, "output buffers are null");
    HIP_OK(hipSetDevice(c->device));
    std::vector<int32_t> ids = {g.tts_bos_id, g.tts_eos_id, g.tts_pad_id, text_tokens[0], text_tokens[1],
                                text_tokens[2]};
    ids.insert(ids.end(), stream.begin(), stream.end());
    for (int32_t t : ids)
        if (t < 0 || t >= g.text_vocab) return fail(c, "Embedding token ID out of range");
    for (int32_t f = 0; f < n_ref_frames; ++f)
        for (int cb = 0; cb < 16 && cb < g.n_codebooks; ++cb) {
            const int32_t t = ref_codec_tokens[(size_t) f * 16 + cb];
            if (t < 0 || t >= (cb == 0 ? g.codec_vocab : g.cp_vocab)) return fail(c, "Embedding token ID out of range");
        }
    std::vector<RowSpec> cin = {{0, RS_CODEC, g.codec_nothink_id, 0, 0}, {0, RS_CODEC, g.codec_think_bos_id, 0, 0},
                                {0, RS_CODEC, g.codec_think_eos_id, 0, 0}};
    if (speaker_embd) cin.push_back({0, RS_SPEAKER, 0, 0, 0});
    cin.push_back({0, RS_CODEC, g.codec_pad_id, 0, 0});
    cin.push_back({0, RS_CODEC, g.codec_bos_id, 0, 0});
    for (const RowSpec & r : cin)
        if (r.a_src == RS_CODEC && (r.a_idx < 0 || r.a_idx >= g.codec_vocab))
            return fail(c, "Embedding token ID out of range");
    const int P_BOS = 0, P_PAD = 2, P_ROLE = 3, P_STREAM = 6;
    std::vector<RowSpec> sp;
    for (int i = 0; i < 3; ++i) sp.push_back({RO_COPY, RS_PROJ, P_ROLE + i, 0, 0});
    for (int t = 0; t < ov_len; ++t)
        sp.push_back({RO_ADD, RS_PROJ, t == ov_len - 1 ? P_BOS : P_PAD, cin[t].a_src, cin[t].a_idx});
    for (int i = 0; i < n_codec; ++i)
        sp.push_back({RO_ZERO_ADD, RS_PROJ, i < n_text ? P_STREAM + i : P_PAD, i == 0 ? RS_CODEC : RS_FRAME,
                      i == 0 ? g.codec_bos_id : i - 1});
    for (int j = 0; j < n_trail; ++j) sp.push_back({RO_COPY, RS_PROJ, P_STREAM + n_codec + j, 0, 0});
    sp.push_back({RO_COPY, RS_PROJ, P_PAD, 0, 0});
    return build_rows(c, ids, sp, speaker_embd, ref_codec_tokens, n_ref_frames, n_pre, n_trail, prefill_out,
                      trailing_out, tts_pad_out);
}

int q3t_dev_embed_rows(q3t_dev * c, int32_t table, int32_t index, const int32_t * tokens, int32_t n, float * out) {
    if (!c || !tokens || !out) return -1;
    if (n <= 0) return 0;
    HIP_OK(hipSetDevice(c->device));
    const q3t_config & g = c->cfg;
    const Slot * s = nullptr;
    int64_t vocab = 0;
    if (table == 0) { s = &c->codec_embd; vocab = g.codec_vocab; }
    else if (table == 1) {
        if (index < 0 || index >= g.n_codebooks - 1) return fail(c, "codebook index out of range");
        s = &c->cp_embd[index]; vocab = g.cp_vocab;
    } else { s = &c->text_embd; vocab = g.text_vocab; }
    if (!s->data) return fail(c, "Embedding tensor not found");
    if (s->type != Q3T_TYPE_F16) return fail(c, "embedding tables must be F16");
    for (int i = 0; i < n; ++i)
        if (tokens[i] < 0 || tokens[i] >= vocab) return fail(c, "Embedding token ID out of range");
    if (n > c->ids_cap) {
        dev_free(c, c->ids);
        c->ids = nullptr;
        if (dev_alloc_t(c, &c->ids, (size_t) n)) return -1;
        c->ids_cap = n;
    }
    const int64_t dim = s->ne0;
    float * tmp = nullptr;
    HIP_OK(hipMalloc(&tmp, (size_t) n * dim * 4));
    HIP_OK(hipMemcpyAsync(c->ids, tokens, (size_t) n * 4, hipMemcpyHostToDevice, c->stream));
    hipLaunchKernelGGL(k_gather_rows, dim3((unsigned) ((dim + 255) / 256), n), dim3(256), 0, c->stream,
                       (const uint16_t *) s->data, dim, c->ids, n, tmp);
    hipError_t e = hipMemcpyAsync(out, tmp, (size_t) n * dim * 4, hipMemcpyDeviceToHost, c->stream);
    hipError_t e2 = hipStreamSynchronize(c->stream);
    (void) hipFree(tmp);
    if (e != hipSuccess || e2 != hipSuccess) return fail(c, "embedding lookup failed");
    return 0;
}

int q3t_dev_frames_begin(q3t_dev * c, const q3t_frame_args * a) {
    if (!c || !a) return -1;
    HIP_OK(hipSetDevice(c->device));
    if (check_ready(c)) return -1;
    const q3t_config & g = c->cfg;
    const int d = g.hidden_size;
    if (!a->tts_pad) return fail(c, "tts_pad row is null");
    if (a->n_trailing < 0 || (a->n_trailing > 0 && !a->trailing)) return fail(c, "bad trailing rows");
    if (a->max_len < 0) return fail(c, "max_len must be >= 0");
    if (a->n_past < 1 || a->n_past + a->max_len > c->n_ctx) return fail(c, "Context length exceeded");
    if (a->max_len > c->codes_cap) {
        dev_free(c, c->codes_out);
        c->codes_out = nullptr;
        if (dev_alloc_t(c, &c->codes_out, (size_t) a->max_len * g.n_codebooks)) return -1;
        c->codes_cap = a->max_len;
        drop_graph(c);
    }
    if (a->n_trailing > c->trailing_cap) {
        dev_free(c, c->trailing);
        c->trailing = nullptr;
        if (dev_alloc_t(c, &c->trailing, (size_t) a->n_trailing * d)) return -1;
        c->trailing_cap = a->n_trailing;
        drop_graph(c);
    }
    if (c->n_trailing != a->n_trailing) drop_graph(c);
    c->n_trailing = a->n_trailing;
    if (a->n_trailing)
        HIP_OK(hipMemcpyAsync(c->trailing, a->trailing, (size_t) a->n_trailing * d * 4, hipMemcpyHostToDevice, c->stream));
    HIP_OK(hipMemcpyAsync(c->pad, a->tts_pad, (size_t) d * 4, hipMemcpyHostToDevice, c->stream));
    SampleParams p{};
    p.temperature = a->sampling.temperature;
    p.top_k = a->sampling.top_k;
    p.rep_penalty = a->repetition_penalty;
    p.eos_bias = a->eos_bias;
    p.target_frames = a->target_frames;
    p.seed = a->sampling.seed;
    HIP_OK(hipMemcpyAsync(c->params, &p, sizeof p, hipMemcpyHostToDevice, c->stream));
    FrameState s{};
    s.base_pos = a->n_past;
    s.talker_pos = a->n_past;
    s.max_frames = a->max_len;
    if (set_state(c, s)) return -1;
    HIP_OK(hipMemsetAsync(c->seen, 0, (size_t) g.codec_vocab, c->stream));
    if (a->max_len >= (1 << 19)) return fail(c, "max_len too large");
    if (fk_prepare(c)) return -1;
    if (c->fk_ok) {
        HIP_OK(hipMemsetAsync(c->fk_arena, 0, c->fk_arena_bytes, c->stream));
        HIP_OK(hipMemsetAsync(c->fk_err, 0, sizeof(int32_t), c->stream));
        c->fk_epoch = 0;
        if (fk_upload_args(c)) return -1;
    }
    if (sync(c)) return -1;
    if (!c->fk_ok && ensure_frame_graph(c)) return -1;
    c->host_emitted = 0;
    c->attn_emitted = 0;
    c->frames_launched = 0;
    c->run_us = 0.0;
    c->run_frames = 0;
    c->frames_max = a->max_len;
    c->frames_ready = true;
    c->codes_begun = true;
    c->stats_streams = false;
    return 0;
}

const int32_t * q3t_dev_frame_codes(const q3t_dev * c) {
    return c && c->codes_begun ? c->codes_out : nullptr;
}

int q3t_dev_frames_run(q3t_dev * c, int32_t n_frames, int32_t * codes_out, int32_t * n_emitted_out, int32_t * eos_out) {
    if (!c) return -1;
    if (!c->frames_ready) return fail(c, "frames_begin not called");
    HIP_OK(hipSetDevice(c->device));
    n_frames = std::max(0, std::min(n_frames, c->frames_max - c->frames_launched));
    // Q3T_NO_GRAPH=1 enqueues the frame's kernels directly (for tracers that
    // do not follow graph launches); the kernels and results are the same.
    static const bool no_graph = [] { const char * e = std::getenv("Q3T_NO_GRAPH"); return e && e[0] == '1'; }();
    if (!c->run_ev[0]) {
        HIP_OK(hipEventCreate(&c->run_ev[0]));
        HIP_OK(hipEventCreate(&c->run_ev[1]));
    }
    // on the XCD-parallel program, keep the carried state: a wait timeout
    // there is re-checked below and the batch run again on the row-parallel
    // program if the workgroup dealing has changed
    const bool xcd_run = c->fk_ok && fk_xcd(c->fk_variant) && n_frames > 0;
    if (xcd_run && fk_snapshot(c, false)) return -1;
    if (n_frames > 0) HIP_OK(hipEventRecord(c->run_ev[0], c->stream));
    for (int i = 0; i < n_frames; ++i) {
        if (c->fk_ok) {
            const hipError_t e = fk_launch(c, c->frames_launched + i, fk::MODE_FRAME);
            if (e == hipSuccess) continue;
            // The cooperative launch can be refused while another process holds
            // the device's cooperative-launch resources.  Nothing was enqueued:
            // continue this context on the captured multi-kernel frame, which
            // shares the frame state and gives the same codes.
            (void) hipGetLastError();
            std::fprintf(stderr, "q3t: cooperative frame-kernel launch refused (%s); using the multi-kernel frame\n",
                         hipGetErrorString(e));
            c->fk_ok = false;
            c->fk_refused = true;
            if (ensure_frame_graph(c)) return -1;
        }
        if (no_graph) frame_seq(c);
        else HIP_OK(hipGraphLaunch(c->frame_exec, c->stream));
        if (c->attn_layer >= 0) {
            // attention capture: a frame that emitted codes (no EOS) ran its
            // talker step, whose row covers positions 0..talker_pos; the
            // reference takes no step after the last frame
            // (src/tts_transformer.cpp:3259-3261), so that row is not kept
            FrameState f{};
            HIP_OK(hipMemcpyAsync(&f, c->st, sizeof f, hipMemcpyDeviceToHost, c->stream));
            if (sync(c)) return -1;
            const bool last = c->frames_launched + i + 1 >= c->frames_max;
            if (f.n_emitted > c->attn_emitted && !last && keep_attn_row(c, f.talker_pos + 1)) return -1;
            c->attn_emitted = f.n_emitted;
        }
    }
    if (n_frames > 0) HIP_OK(hipEventRecord(c->run_ev[1], c->stream));
    c->frames_launched += n_frames;
    FrameState r{};
    HIP_OK(hipMemcpyAsync(&r, c->st, sizeof r, hipMemcpyDeviceToHost, c->stream));
    int32_t fk_err = 0;
    if (c->fk_ok) HIP_OK(hipMemcpyAsync(&fk_err, c->fk_err, sizeof fk_err, hipMemcpyDeviceToHost, c->stream));
    if (sync(c)) return -1;
    const bool forced = xcd_run && c->fk_ok && fk_xcd(c->fk_variant) && test_reprobe_fail();
    if ((fk_err || forced) && xcd_run && c->fk_ok && fk_xcd(c->fk_variant)) {
        // A wait of the XCD-parallel program timed out.  Its hand-offs inside
        // an XCD rely on the workgroups of each class b % 8 sharing one XCD;
        // check the dealing again, and if it changed, rerun this batch from
        // the kept state on the row-parallel program (fresh launches), which
        // gives the same codes.
        c->xcd_map = -1;
        bool ok = false;
        if (xcd_map_ok(c, c->fk_grid, ok, forced)) return -1;
        if (!ok) {
            if (fk_snapshot(c, true)) return -1;
            c->frames_launched -= n_frames;
            c->fk_no_xcd = true;
            c->fk_ok = false;
            if (fk_prepare(c)) return -1;
            if (c->fk_ok) {
                HIP_OK(hipMemsetAsync(c->fk_arena, 0, c->fk_arena_bytes, c->stream));
                HIP_OK(hipMemsetAsync(c->fk_err, 0, sizeof(int32_t), c->stream));
                c->fk_epoch = 0;
                if (fk_upload_args(c)) return -1;
            } else if (ensure_frame_graph(c)) {
                return -1;
            }
            if (sync(c)) return -1;
            return q3t_dev_frames_run(c, n_frames, codes_out, n_emitted_out, eos_out);
        }
    }
    if (fk_err) return fail(c, fk_err_msg(fk_err));
    if (n_frames > 0) {
        float ms = 0.0f;
        HIP_OK(hipEventElapsedTime(&ms, c->run_ev[0], c->run_ev[1]));
        c->run_us += 1e3 * ms;
        c->run_frames += n_frames;
    }
    const int ncb = c->cfg.n_codebooks;
    const int fresh = r.n_emitted - c->host_emitted;
    if (fresh > 0 && codes_out)
        HIP_OK(hipMemcpy(codes_out, c->codes_out + (size_t) c->host_emitted * ncb, (size_t) fresh * ncb * 4,
                         hipMemcpyDeviceToHost));
    c->host_emitted = r.n_emitted;
    if (n_emitted_out) *n_emitted_out = fresh;
    if (eos_out) *eos_out = r.eos;
    return 0;
}

}  // extern "C"

namespace {

// ------------------------------------------------------------ multi-stream
// nb independent utterances share the weights: every GEMV of the frame
// becomes an (nb x nt)-row GEMM on the int8 MFMA kernel, attention and the
// samplers run one block per stream (grid z / x), each stream keeps its own
// KV caches, frame state, sampler state and trailing text.

// F16 / Q8 GEMV over n rows in launches of 4, 2 or 1 rows.
static void gemv_rows(q3t_dev * c, const GemvSpec & s, int n) {
    const bool wide = s.w.kind == W_F16 && s.epi != EPI_SWIGLU;   // 8 / 16 rows per launch (F16 heads)
    for (int r = 0; r < n;) {
        const int nt = wide && n - r >= 16 ? 16 : wide && n - r >= 8 ? 8 : n - r >= 4 ? 4 : n - r >= 2 ? 2 : 1;
        GemvSpec t = s;
        t.x = s.x + (size_t) r * s.x_stride;
        t.y = s.y + (size_t) r * s.y_stride;
        if (s.hidden_out) t.hidden_out = s.hidden_out + (size_t) r * s.hidden_stride;
        gemv(c, t, nt);
        r += nt;
    }
}

struct StreamKV {
    uint16_t * kc; uint16_t * vc;   // stream 0, this layer
    int64_t stream;                 // elements per stream
    int n_ctx;
    const float * rc; const float * rs;
    const int32_t * pos_ptr; int pos_const;
    bool f32_prefill;               // the code predictor's 2-token prefill: F32 q, K, V, P
};

// The three shapes of decode GEMM a layer needs (ms::k_gemm_sk):
//   QKV      RMSNorm'd fp32 rows quantised in registers, fp32 out
//   PROJ     pre-quantised rows in (attention / SwiGLU output), + residual
//   GATE_UP  RMSNorm'd rows, gate and up matrices, SwiGLU, Q8_0 out
enum GemmKind { G_QKV = 0, G_PROJ = 1, G_GATE_UP = 2 };
// preferred K splits and the Q8_0 blocks per wave they leave (QKV and gate/up:
// 32 blocks / (4 waves x 2); Wo / down: 64 or 96 / (4 x 4)).  Measured with
// 16 streams on one box: {2, 4, 2} 2,567 aggregate frames/s, {2, 2, 2} 2,500,
// the former {4, 8, 4} 2,340, no split {1, 1, 1} 2,051.
constexpr int kGemmKB[3] = {4, 6, 4};       // max Q8_0 blocks per wave
constexpr int kGemmMT[3] = {1, 1, 2};       // 16-row tiles per workgroup
constexpr int kGemmS[3] = {2, 4, 2};        // preferred K splits

template <int NT, int KIND>
const void * gemm_kernel() {
    if (KIND == G_QKV) return (const void *) ms::k_gemm_sk<NT, 1, false, ms::IN_NORM, ms::OUT_F32, kGemmKB[G_QKV]>;
    if (KIND == G_PROJ) return (const void *) ms::k_gemm_sk<NT, 1, false, ms::IN_Q8, ms::OUT_RESID, kGemmKB[G_PROJ]>;
    return (const void *) ms::k_gemm_sk<NT, 2, true, ms::IN_NORM, ms::OUT_SWIGLU_Q8, kGemmKB[G_GATE_UP]>;
}

template <int KIND>
const void * gemm_kernel_nt(int nt) {
    switch (nt) {
        case 1: return gemm_kernel<1, KIND>();
        case 2: return gemm_kernel<2, KIND>();
        case 3: return gemm_kernel<3, KIND>();
        default: return gemm_kernel<4, KIND>();
    }
}

const void * gemm_fn(int kind, int nt) {
    return kind == G_QKV ? gemm_kernel_nt<G_QKV>(nt) : kind == G_PROJ ? gemm_kernel_nt<G_PROJ>(nt)
                                                                      : gemm_kernel_nt<G_GATE_UP>(nt);
}

// K splits for a contraction of nb Q8_0 blocks: the largest S <= the kind's
// preference with nb % (4 S) == 0 and at most KB blocks per wave; 0 if none.
int gemm_splits(int kind, int nb) {
    for (int S = kGemmS[kind]; S >= 1; S >>= 1)
        if (nb % (ms::kWaves * S) == 0 && nb / (ms::kWaves * S) <= kGemmKB[kind]) return S;
    return 0;
}

size_t gemm_lds(int kind, int nt, int K) {
    const int S = gemm_splits(kind, K / kQK);
    return ms::gemm_sk_lds_bytes(nt, kGemmMT[kind], kind == G_GATE_UP, S ? K / kQK / S : 0);
}

// tagged words of the partials one launch may store: tiles x S x 2 per value x values per lane x 64 lanes
size_t gemm_part_words(int kind, int nt, int N, int K) {
    const int mt = kGemmMT[kind], nw = kind == G_GATE_UP ? 2 : 1;
    return (size_t) (N / (ms::kRows * mt)) * gemm_splits(kind, K / kQK) * 2 * nw * mt * nt * 4 * 64;
}

// call types sharing a ticket/partial set
enum GemmSite { S_QKV = 0, S_WO = 1, S_GATE_UP = 2, S_DOWN = 3 };

void gemm_rows(q3t_dev * c, int kind, int site, ms::GemmArgs a) {
    const int nt = (a.n + 15) / 16;
    const int S = gemm_splits(kind, a.K / kQK);
    a.part = c->spart[site]; a.cnt = c->scnt[site]; a.err = c->serr;
    void * args[] = {(void *) &a};
    (void) hipLaunchKernel(gemm_fn(kind, nt), dim3(a.N / (ms::kRows * kGemmMT[kind]), S), dim3(ms::kThreads), args,
                           gemm_lds(kind, nt, a.K), c->stream);
}

// F16 layers: the four decode GEMMs of a layer on ms::k_gemm_h, 16-row tiles,
// K split up to 8 ways (kHKB chunks of 32 per wave at most).
enum HKind { H_QKV = 0, H_WO = 1, H_GATE_UP = 2, H_DOWN = 3 };
constexpr int kHKB[4] = {1, 2, 1, 3};

template <int NT, int KIND, bool HM>
const void * hgemm_kernel() {
    if (KIND == H_QKV) return (const void *) ms::k_gemm_h<NT, 1, false, ms::IN_NORM, ms::OUT_F32, kHKB[H_QKV], HM>;
    if (KIND == H_WO) return (const void *) ms::k_gemm_h<NT, 1, false, ms::IN_ROUND, ms::OUT_RESID, kHKB[H_WO], HM>;
    if (KIND == H_GATE_UP)
        return (const void *) ms::k_gemm_h<NT, 1, true, ms::IN_NORM, ms::OUT_SWIGLU_F32, kHKB[H_GATE_UP], HM>;
    return (const void *) ms::k_gemm_h<NT, 1, false, ms::IN_WIDE, ms::OUT_RESID, kHKB[H_DOWN], HM>;
}

template <int KIND, bool HM>
const void * hgemm_kernel_nt(int nt) {
    switch (nt) {
        case 1: return hgemm_kernel<1, KIND, HM>();
        case 2: return hgemm_kernel<2, KIND, HM>();
        case 3: return hgemm_kernel<3, KIND, HM>();
        default: return hgemm_kernel<4, KIND, HM>();
    }
}

template <bool HM>
const void * hgemm_fn_form(int kind, int nt) {
    switch (kind) {
        case H_QKV: return hgemm_kernel_nt<H_QKV, HM>(nt);
        case H_WO: return hgemm_kernel_nt<H_WO, HM>(nt);
        case H_GATE_UP: return hgemm_kernel_nt<H_GATE_UP, HM>(nt);
        default: return hgemm_kernel_nt<H_DOWN, HM>(nt);
    }
}

// hm: the fp16-MFMA form (fp32 accumulation), else the exact f64-MFMA form
const void * hgemm_fn(int kind, int nt, bool hm) {
    return hm ? hgemm_fn_form<true>(kind, nt) : hgemm_fn_form<false>(kind, nt);
}

// Q3T_MS_EXACT=1: the multi-stream decode of F16 layers on the exact f64-MFMA
// GEMMs, whose codes equal each stream's batch-1 run; by default the
// fp16-MFMA GEMMs with fp32 accumulation (read at q3t_dev_streams_begin).
bool ms_exact() {
    const char * e = std::getenv("Q3T_MS_EXACT");
    return e && e[0] == '1';
}

// K splits of an F16 contraction of nb 32-element chunks: the largest S <= 8
// with nb % (4 S) == 0 and at most kHKB chunks per wave; 0 if none.
int hgemm_splits(int kind, int nb) {
    for (int S = 8; S >= 1; S >>= 1)
        if (nb % (ms::kWaves * S) == 0 && nb / (ms::kWaves * S) <= kHKB[kind]) return S;
    return 0;
}

size_t hgemm_part_words(int kind, int nt, int N, int K) {
    const int nw = kind == H_GATE_UP ? 2 : 1;
    return (size_t) (N / ms::kRows) * hgemm_splits(kind, K / kQK) * 2 * nw * nt * 4 * 64;
}

void hgemm_rows(q3t_dev * c, int kind, int site, ms::GemmArgs a) {
    const int nt = (a.n + 15) / 16;
    const int S = hgemm_splits(kind, a.K / kQK);
    a.part = c->spart[site]; a.cnt = c->scnt[site]; a.err = c->serr;
    void * args[] = {(void *) &a};
    (void) hipLaunchKernel(hgemm_fn(kind, nt, c->s_hm), dim3(a.N / ms::kRows, S), dim3(ms::kThreads), args,
                           ms::gemm_h_lds_bytes(nt, 1, kind == H_GATE_UP), c->stream);
}

// Contraction length of each decode GEMM kind: the normed inputs are model
// rows (d), the projections read attention or SwiGLU rows.
int gemm_k(int kind, int d, int kproj) { return kind == G_PROJ ? kproj : d; }

// Allows each decode GEMM its dynamic LDS.
hipError_t allow_gemm_lds(int d, int kproj) {
    for (int kind = 0; kind < 3; ++kind)
        for (int nt = 1; nt <= 4; ++nt) {
            const hipError_t e = hipFuncSetAttribute(gemm_fn(kind, nt), hipFuncAttributeMaxDynamicSharedMemorySize,
                                                     (int) gemm_lds(kind, nt, gemm_k(kind, d, kproj)));
            if (e != hipSuccess) return e;
        }
    return hipSuccess;
}

// RMSNorm row scales of n rows of width K into c->srs.
void row_scales(q3t_dev * c, const float * x, int xs, int K, int n) {
    hipLaunchKernelGGL(ms::k_row_scale, dim3(n), dim3(kBlock), 0, c->stream, x, xs, K, c->cfg.rms_eps, c->srs);
}

void attn_gqa(q3t_dev * c, const LayerDev & L, const StreamKV & kv) {
    const q3t_config & g = c->cfg;
    const int qd = g.n_head * g.head_dim, qkvd = qd + 2 * g.n_kv_head * g.head_dim, G = g.n_head / g.n_kv_head;
    ms::GqaArgs a{};
    a.qkv = c->bqkv; a.qkv_stride = qkvd;
    a.q_norm = L.q_norm; a.k_norm = L.k_norm; a.eps = g.rms_eps;
    a.rope_cos = kv.rc; a.rope_sin = kv.rs;
    a.kc = kv.kc; a.vc = kv.vc; a.kv_stream = kv.stream;
    a.n_ctx = kv.n_ctx; a.n_head = g.n_head; a.n_kv_head = g.n_kv_head;
    a.pos = kv.pos_ptr; a.pos_stream = (int32_t) (sizeof(FrameState) / 4);
    a.done = &c->sst[0].done; a.done_stream = (int32_t) (sizeof(FrameState) / 4);
    a.out = c->batt; a.out_stride = qd;
    a.out_q = c->bq8; a.out_dx = c->bdx8;
    a.scale = 1.0f / std::sqrt((float) g.head_dim);
    // one query head per workgroup: twice the workgroups of one per KV head,
    // each streaming its KV head's cache (the two of a group share it in L2)
    (void) G;
    const dim3 grid(g.n_head, c->nb), block(ms::kAThreads);
    hipLaunchKernelGGL(ms::k_attn_gqa<1>, grid, block, ms::attn_gqa_lds_bytes(1, kv.n_ctx), c->stream, a);
}

// Code-predictor layer 0 of step s (1..14) for every stream: the QKV row of
// the stream's input code (sampled into its frame state by the previous
// step) copied from the per-code table, in place of RMSNorm + the QKV GEMM
// (the table rows equal the GEMM's bit for bit).
__global__ __launch_bounds__(256) void k_cp_tab_rows(const float * __restrict__ tab, int32_t V, int32_t qkvd,
                                                      int32_t step, const FrameState * __restrict__ st,
                                                      float * __restrict__ out) {
    const int b = blockIdx.x;
    int code = st[b].codes[step];
    code = code < 0 ? 0 : code >= V ? V - 1 : code;     // a finished stream's row is never used
    const float4 * src = (const float4 *) (tab + ((size_t) (step - 1) * V + code) * qkvd);
    float4 * dst = (float4 *) (out + (size_t) b * qkvd);
    for (int i = threadIdx.x; i < qkvd / 4; i += 256) dst[i] = src[i];
}

static void cp_tab_rows(q3t_dev * c, int step) {
    const q3t_config & g = c->cfg;
    const int qkvd = (g.n_head + 2 * g.n_kv_head) * g.head_dim;
    hipLaunchKernelGGL(k_cp_tab_rows, dim3(c->nb), dim3(256), 0, c->stream, (const float *) c->cp_tab, g.cp_vocab,
                       qkvd, step, (const FrameState *) c->sst, c->bqkv);
}

// The layer's attention over the QKV rows in c->bqkv: the talker's GQA kernel
// for one token per stream; for the code predictor's 16-position cache the
// per-head kernel over nt tokens.  Output rows (fp32) in c->batt, Q8_0 copies
// in c->bq8 / c->bdx8.
static void stream_attention(q3t_dev * c, const LayerDev & L, int nt, const StreamKV & kv) {
    const q3t_config & g = c->cfg;
    const int qd = g.n_head * g.head_dim, qkvd = qd + 2 * g.n_kv_head * g.head_dim;
    if (kv.pos_ptr && nt == 1) {
    attn_gqa(c, L, kv);
    return;
    }
    AttnArgs a{};
    a.qkv = c->bqkv; a.qkv_stride = qkvd; a.qkv_stream = nt * qkvd;
    a.q_norm = L.q_norm; a.k_norm = L.k_norm; a.eps = g.rms_eps;
    a.rope_cos = kv.rc; a.rope_sin = kv.rs;
    a.kc = kv.kc; a.vc = kv.vc; a.n_ctx = kv.n_ctx; a.kv_stream = kv.stream;
    a.n_head = g.n_head; a.n_kv_head = g.n_kv_head;
    a.pos_ptr = kv.pos_ptr; a.pos_const = kv.pos_const; a.pos_stream = (int32_t) (sizeof(FrameState) / 4);
    a.out = c->batt; a.out_stride = qd; a.out_stream = nt * qd;
    a.out_q = c->bq8; a.out_dx = c->bdx8;
    a.done = &c->sst[0].done; a.done_stream = (int32_t) (sizeof(FrameState) / 4);
    a.scale = 1.0f / std::sqrt((float) g.head_dim);
    a.nt = nt;
    a.f32_new = kv.f32_prefill ? 1 : 0;
    hipLaunchKernelGGL(k_attention, dim3(g.n_head, nt, c->nb), dim3(kBlock), attn_lds_bytes(kv.n_ctx), c->stream, a);
}

// One decoder layer over n = nb * nt rows (stream-major); output rows in c->bxa.
// The residual-producing GEMMs (Wo, down) also leave per-tile sums of squares
// of their output rows, from which the next normed GEMM forms its RMSNorm
// scales; only a layer's first input (x_ss false: gathered rows) needs the
// row-scale kernel.
// Four decode-shaped GEMMs and one attention launch (the talker's GQA kernel
// for one token per stream; for the code predictor's 16-position cache the
// per-head kernel over nt tokens).  Activations pass between them as fp32
// residual rows (RMSNorm + quantisation inside the consuming GEMM) or as
// Q8_0 rows quantised by the producer (attention output, SwiGLU output).
static void stream_layer(q3t_dev * c, const LayerDev & L, const float * x, bool x_ss, int nt, const StreamKV & kv,
                        int tab_step = 0) {
    const q3t_config & g = c->cfg;
    const int d = g.hidden_size, qd = g.n_head * g.head_dim, kd = g.n_kv_head * g.head_dim, qkvd = qd + 2 * kd;
    const int ffn = g.ffn_size, n = c->nb * nt, tiles = d / ms::kRows;
    const bool fuse = tiles / 4 <= ms::kSsPer;   // row scales from the producer's per-tile sums
    x_ss = x_ss && fuse;
    if (tab_step > 0) {
        cp_tab_rows(c, tab_step);
    } else {
        if (!x_ss) row_scales(c, x, d, d, n);
        ms::GemmArgs q{};
        q.W = (const int8_t *) L.qkv.data; q.Wd = L.qkv.scales; q.N = qkvd; q.K = d;
        q.x = x; q.xs = d; q.rscale = c->srs; q.norm_w = L.attn_norm; q.n = n; q.y = c->bqkv; q.ys = qkvd;
        if (x_ss) { q.ss_in = c->sss[1]; q.ss_tiles = tiles; q.eps = g.rms_eps; }
        gemm_rows(c, G_QKV, S_QKV, q);
    }
    stream_attention(c, L, nt, kv);
    ms::GemmArgs o{};
    o.W = (const int8_t *) L.wo.data; o.Wd = L.wo.scales; o.N = d; o.K = qd;
    o.q = c->bq8; o.qdx = c->bdx8; o.n = n; o.y = c->bxb; o.ys = d; o.res = x; o.rs = d;
    if (fuse) o.ss_out = c->sss[0];
    gemm_rows(c, G_PROJ, S_WO, o);
    if (!fuse) row_scales(c, c->bxb, d, d, n);
    ms::GemmArgs f{};
    f.W = (const int8_t *) L.wg.data; f.Wd = L.wg.scales; f.W2 = (const int8_t *) L.wu.data; f.W2d = L.wu.scales;
    f.N = ffn; f.K = d; f.x = c->bxb; f.xs = d; f.rscale = c->srs; f.norm_w = L.ffn_norm; f.n = n;
    if (fuse) { f.ss_in = c->sss[0]; f.ss_tiles = tiles; f.eps = g.rms_eps; }
    f.yq = c->bq8; f.ydx = c->bdx8;
    gemm_rows(c, G_GATE_UP, S_GATE_UP, f);
    ms::GemmArgs dn{};
    dn.W = (const int8_t *) L.wd.data; dn.Wd = L.wd.scales; dn.N = d; dn.K = ffn;
    dn.q = c->bq8; dn.qdx = c->bdx8; dn.n = n; dn.y = c->bxa; dn.ys = d; dn.res = c->bxb; dn.rs = d;
    if (fuse) dn.ss_out = c->sss[1];
    gemm_rows(c, G_PROJ, S_DOWN, dn);
}

// The same layer with F16 weights on the f64-MFMA decode GEMMs: inputs rounded
// to fp16 as the batch-1 F16 GEMVs round them (the widened ffn_down takes the
// fp32 SwiGLU rows in c->bff), row scales fused the same way.
static void stream_layer_h(q3t_dev * c, const LayerDev & L, const float * x, bool x_ss, int nt, const StreamKV & kv,
                        int tab_step = 0) {
    const q3t_config & g = c->cfg;
    const int d = g.hidden_size, qd = g.n_head * g.head_dim, kd = g.n_kv_head * g.head_dim, qkvd = qd + 2 * kd;
    const int ffn = g.ffn_size, n = c->nb * nt, tiles = d / ms::kRows;
    const bool fuse = tiles / 4 <= ms::kSsPer;
    x_ss = x_ss && fuse;
    if (tab_step > 0) {
        cp_tab_rows(c, tab_step);
    } else {
        if (!x_ss) row_scales(c, x, d, d, n);
        ms::GemmArgs q{};
        q.H = (const uint16_t *) L.qkv.data; q.N = qkvd; q.K = d;
        q.x = x; q.xs = d; q.rscale = c->srs; q.norm_w = L.attn_norm; q.n = n; q.y = c->bqkv; q.ys = qkvd;
        if (x_ss) { q.ss_in = c->sss[1]; q.ss_tiles = tiles; q.eps = g.rms_eps; }
        hgemm_rows(c, H_QKV, S_QKV, q);
    }
    stream_attention(c, L, nt, kv);
    ms::GemmArgs o{};
    o.H = (const uint16_t *) L.wo.data; o.N = d; o.K = qd;
    o.x = c->batt; o.xs = qd; o.n = n; o.y = c->bxb; o.ys = d; o.res = x; o.rs = d;
    if (fuse) o.ss_out = c->sss[0];
    hgemm_rows(c, H_WO, S_WO, o);
    if (!fuse) row_scales(c, c->bxb, d, d, n);
    ms::GemmArgs f{};
    f.H = (const uint16_t *) L.wg.data; f.H2 = (const uint16_t *) L.wu.data; f.N = ffn; f.K = d;
    f.x = c->bxb; f.xs = d; f.rscale = c->srs; f.norm_w = L.ffn_norm; f.n = n; f.y = c->bff; f.ys = ffn;
    if (fuse) { f.ss_in = c->sss[0]; f.ss_tiles = tiles; f.eps = g.rms_eps; }
    hgemm_rows(c, H_GATE_UP, S_GATE_UP, f);
    ms::GemmArgs dn{};
    dn.H = (const uint16_t *) L.wd.data; dn.N = d; dn.K = ffn;
    dn.x = c->bff; dn.xs = ffn; dn.n = n; dn.y = c->bxa; dn.ys = d; dn.res = c->bxb; dn.rs = d;
    if (fuse) dn.ss_out = c->sss[1];
    hgemm_rows(c, H_DOWN, S_DOWN, dn);
}

static SampleArgs stream_sample_args(q3t_dev * c, int mode, int group) {
    const q3t_config & g = c->cfg;
    const int d = g.hidden_size;
    SampleArgs sa{};
    sa.mode = mode; sa.group = group;
    sa.vocab = mode == 0 ? g.codec_vocab : g.cp_vocab;
    sa.logits = mode == 0 ? c->slogits : c->scplogits;
    sa.logits_stream = sa.vocab;
    sa.params = c->sparams; sa.st = c->sst; sa.seen = c->sseen; sa.seen_stream = g.codec_vocab;
    sa.eos_id = g.codec_eos_id;
    sa.stage = c->sstage; sa.stage_stream = mode == 0 ? 2 * d : d;
    sa.hidden = c->shidden; sa.hidden_stream = d;
    sa.codec_embd = (const uint16_t *) c->codec_embd.data;
    for (int i = 0; i < g.n_codebooks - 1; ++i) sa.cp_embd[i] = (const uint16_t *) c->cp_embd[i].data;
    sa.trailing = c->strail; sa.trailing_stream = c->strail_cap * d; sa.n_trailing_arr = c->sntrail;
    sa.pad = c->spad; sa.pad_stream = d;
    sa.d = d;
    return sa;
}

// One frame of every stream: codebook-0 samplers, code predictor (2-token
// prefill + 14 steps), talker step; each stream's frame state advances
// unless it is done.
static void streams_frame_seq(q3t_dev * c) {
    const q3t_config & g = c->cfg;
    const int d = g.hidden_size, B = c->nb;
    SampleArgs sa = stream_sample_args(c, 0, 0);
    sa.open_frame = 1;
    hipLaunchKernelGGL(k_sample, dim3(B), dim3(kSampleThreads), 0, c->stream, sa);
    const int64_t cp_lstride = (int64_t) g.n_kv_head * 16 * g.head_dim;
    for (int step = 0; step < g.n_codebooks - 1; ++step) {
        const int nt = step == 0 ? 2 : 1;
        const int pos = step == 0 ? 0 : step + 1;
        const float * x = c->sstage;
        for (int il = 0; il < g.cp_layers; ++il) {
            StreamKV kv{c->scpk + il * cp_lstride, c->scpv + il * cp_lstride, cp_lstride * g.cp_layers, 16,
                        c->cp_rope_cos, c->cp_rope_sin, nullptr, pos, step == 0};
            (c->s_f16 ? stream_layer_h : stream_layer)(c, c->cp[il], x, il > 0, nt, kv,
                                                       c->s_tab && il == 0 && step > 0 ? step : 0);
            x = c->bxa;
        }
        GemvSpec h{};
        h.w = weight_of(c->cp_head[step]); h.rows = g.cp_vocab; h.K = d;
        h.x = c->bxa + (size_t) (nt - 1) * d; h.x_stride = nt * d; h.norm_w = (const float *) c->cp_out_norm.data;
        h.y = c->scplogits; h.y_stride = g.cp_vocab; h.no_done = true;
        gemv_rows(c, h, B);
        SampleArgs sc = stream_sample_args(c, 1, step + 1);
        if (step + 1 == 15) { sc.codes_out = c->scodes; sc.codes_stream = c->scodes_cap * 16; }
        hipLaunchKernelGGL(k_sample, dim3(B), dim3(kSampleThreads), 0, c->stream, sc);
    }
    const int64_t lstride = (int64_t) g.n_kv_head * c->sb_ctx * g.head_dim;
    const float * x = c->sstage;
    for (int il = 0; il < g.n_layers; ++il) {
        StreamKV kv{c->skc + il * lstride, c->svc + il * lstride, lstride * g.n_layers, c->sb_ctx, c->rope_cos,
                    c->rope_sin, &c->sst[0].talker_pos, 0, false};
        (c->s_f16 ? stream_layer_h : stream_layer)(c, c->talker[il], x, il > 0, 1, kv, 0);
        x = c->bxa;
    }
    GemvSpec h{};
    h.w = weight_of(c->codec_head); h.rows = g.codec_vocab; h.K = d;
    h.x = c->bxa; h.x_stride = d; h.norm_w = (const float *) c->out_norm.data;
    h.hidden_out = c->shidden; h.hidden_stride = d; h.y = c->slogits; h.y_stride = g.codec_vocab; h.no_done = true;
    gemv_rows(c, h, B);
}

}  // namespace

extern "C" {

int q3t_dev_streams_reserve(q3t_dev * c, int32_t n_streams, int32_t n_ctx) {
    if (!c) return -1;
    HIP_OK(hipSetDevice(c->device));
    if (resolve(c)) return -1;
    const q3t_config & g = c->cfg;
    if (n_streams < 1 || n_streams > 32) return fail(c, "n_streams must be in [1, 32]");
    if (n_ctx < 1) return fail(c, "n_ctx must be > 0");
    if (c->kv_bf16) return fail(c, "multi-stream decode keeps an F16 talker cache (q3t_dev_kv_set_type F16 first)");
    bool all_q8 = true, all_f16 = true;
    for (int i = 0; i < g.n_layers + g.cp_layers; ++i) {
        const LayerDev & L = i < g.n_layers ? c->talker[i] : c->cp[i - g.n_layers];
        for (const Slot * w : {&L.qkv, &L.wo, &L.wg, &L.wu, &L.wd}) {
            all_q8 = all_q8 && w->type == Q3T_TYPE_Q8_0;
            all_f16 = all_f16 && w->type == Q3T_TYPE_F16;
        }
    }
    if (!all_q8 && !all_f16)
        return fail(c, "multi-stream decode needs all layer weights Q8_0 (int8 MFMA GEMMs) or all F16 (f64 MFMA GEMMs)");
    const int d = g.hidden_size, qd = g.n_head * g.head_dim, qkvd = qd + 2 * g.n_kv_head * g.head_dim;
    const int G = g.n_kv_head > 0 ? g.n_head / g.n_kv_head : 0;
    // decode GEMMs: every contraction splits into 4-wave slices of at most KB
    // blocks (32-element chunks) per wave; N a multiple of 16 (Q8_0 gate/up: 32)
    const bool splits_ok = all_q8 ? gemm_splits(G_QKV, d / kQK) && gemm_splits(G_GATE_UP, d / kQK) &&
                                        gemm_splits(G_PROJ, qd / kQK) && gemm_splits(G_PROJ, g.ffn_size / kQK)
                                  : hgemm_splits(H_QKV, d / kQK) && hgemm_splits(H_GATE_UP, d / kQK) &&
                                        hgemm_splits(H_WO, qd / kQK) && hgemm_splits(H_DOWN, g.ffn_size / kQK);
    if (g.head_dim != 128 || d % kQK || qd % kQK || g.ffn_size % kQK || !splits_ok || qkvd % ms::kRows ||
        d % ms::kRows || g.ffn_size % (2 * ms::kRows) || g.cp_ffn != g.ffn_size || g.cp_hidden != d ||
        g.n_head % g.n_kv_head || !(G == 1 || G == 2 || G == 4))
        return fail(c, "multi-stream decode: unsupported model widths");
    int max_lds = 0;
    HIP_OK(hipDeviceGetAttribute(&max_lds, hipDeviceAttributeMaxSharedMemoryPerBlock, c->device));
    const size_t al = ms::attn_gqa_lds_bytes(1, n_ctx);
    const int kproj = std::max(qd, g.ffn_size);
    size_t gl = 0;
    for (int kind = 0; kind < 3; ++kind) gl = std::max(gl, gemm_lds(kind, 4, gemm_k(kind, d, kproj)));
    if (gl > (size_t) max_lds) return fail(c, "multi-stream decode: GEMM LDS exceeds the device limit");
    if (al > (size_t) max_lds) return fail(c, "multi-stream decode: n_ctx too large for the attention kernel's LDS");
    HIP_OK(allow_gemm_lds(d, kproj));
    HIP_OK(hipFuncSetAttribute((const void *) ms::k_attn_gqa<1>, hipFuncAttributeMaxDynamicSharedMemorySize, (int) al));
    // the streams' talker caches share the context's RoPE tables and KV layout stride
    if (c->n_ctx != n_ctx && q3t_dev_kv_reserve(c, n_ctx)) return -1;
    HIP_OK(hipStreamSynchronize(c->stream));
    drop_stream_graph(c);
    for (void * p : {(void *) c->skc, (void *) c->svc, (void *) c->scpk, (void *) c->scpv, (void *) c->sst,
                     (void *) c->sparams, (void *) c->sseen, (void *) c->sntrail, (void *) c->spad, (void *) c->shidden,
                     (void *) c->slogits, (void *) c->scplogits, (void *) c->sstage, (void *) c->bxa, (void *) c->bxb,
                     (void *) c->bqkv, (void *) c->batt, (void *) c->bq8, (void *) c->bdx8, (void *) c->bff, (void *) c->srs,
                     (void *) c->serr, (void *) c->scodes, (void *) c->strail, (void *) c->sss[0], (void *) c->sss[1]})
        if (p) dev_free(c, p);
    for (int i = 0; i < 4; ++i) {
        if (c->spart[i]) dev_free(c, c->spart[i]);
        if (c->scnt[i]) dev_free(c, c->scnt[i]);
        c->spart[i] = nullptr; c->scnt[i] = nullptr;
    }
    c->scodes = nullptr; c->strail = nullptr; c->scodes_cap = 0; c->strail_cap = 0;
    const size_t B = (size_t) n_streams, rows = 2 * B;
    const size_t kv = (size_t) g.n_layers * g.n_kv_head * n_ctx * g.head_dim;
    const size_t ckv = (size_t) g.cp_layers * g.n_kv_head * 16 * g.head_dim;
    if (dev_alloc_t(c, &c->skc, B * kv) || dev_alloc_t(c, &c->svc, B * kv) || dev_alloc_t(c, &c->scpk, B * ckv) ||
        dev_alloc_t(c, &c->scpv, B * ckv) || dev_alloc_t(c, &c->sst, B) || dev_alloc_t(c, &c->sparams, B) ||
        dev_alloc_t(c, &c->sseen, B * g.codec_vocab) || dev_alloc_t(c, &c->sntrail, B) ||
        dev_alloc_t(c, &c->spad, B * d) || dev_alloc_t(c, &c->shidden, B * d) ||
        dev_alloc_t(c, &c->slogits, B * g.codec_vocab) || dev_alloc_t(c, &c->scplogits, B * g.cp_vocab) ||
        dev_alloc_t(c, &c->sstage, B * 2 * d) || dev_alloc_t(c, &c->bxa, rows * d) || dev_alloc_t(c, &c->bxb, rows * d) ||
        dev_alloc_t(c, &c->bqkv, rows * qkvd) || dev_alloc_t(c, &c->batt, rows * qd) ||
        dev_alloc_t(c, &c->bq8, rows * std::max(qd, g.ffn_size)) || dev_alloc_t(c, &c->bff, rows * g.ffn_size) ||
        dev_alloc_t(c, &c->bdx8, rows * (std::max(qd, g.ffn_size) / kQK)) || dev_alloc_t(c, &c->srs, rows) ||
        dev_alloc_t(c, &c->sss[0], rows * (d / ms::kRows)) || dev_alloc_t(c, &c->sss[1], rows * (d / ms::kRows)))
        return -1;
    {
        // tickets and tags start at 0 (a tag is >= 1), zeroed here, outside any graph
        const int nt = (int) ((rows + 15) / 16);
        const size_t words[4] = {all_q8 ? gemm_part_words(G_QKV, nt, qkvd, d) : hgemm_part_words(H_QKV, nt, qkvd, d),
                                 all_q8 ? gemm_part_words(G_PROJ, nt, d, qd) : hgemm_part_words(H_WO, nt, d, qd),
                                 all_q8 ? gemm_part_words(G_GATE_UP, nt, g.ffn_size, d)
                                        : hgemm_part_words(H_GATE_UP, nt, g.ffn_size, d),
                                 all_q8 ? gemm_part_words(G_PROJ, nt, d, g.ffn_size)
                                        : hgemm_part_words(H_DOWN, nt, d, g.ffn_size)};
        const size_t tiles = (size_t) std::max(qkvd, std::max(d, g.ffn_size)) / ms::kRows;
        for (int i = 0; i < 4; ++i) {
            const size_t nw = std::max(words[i], (size_t) 64);
            if (dev_alloc_t(c, &c->spart[i], nw) || dev_alloc_t(c, &c->scnt[i], tiles)) return -1;
            HIP_OK(hipMemsetAsync(c->spart[i], 0, nw * 8, c->stream));
            HIP_OK(hipMemsetAsync(c->scnt[i], 0, tiles * sizeof(uint32_t), c->stream));
        }
        if (dev_alloc_t(c, &c->serr, 1)) return -1;
        HIP_OK(hipMemsetAsync(c->serr, 0, sizeof(int32_t), c->stream));
    }
    HIP_OK(hipMemsetAsync(c->skc, 0, B * kv * 2, c->stream));
    HIP_OK(hipMemsetAsync(c->svc, 0, B * kv * 2, c->stream));
    HIP_OK(hipMemsetAsync(c->scpk, 0, B * ckv * 2, c->stream));
    HIP_OK(hipMemsetAsync(c->scpv, 0, B * ckv * 2, c->stream));
    c->nb = n_streams;
    c->s_f16 = all_f16;
    // code-predictor layer 0 of steps 1..14 from the per-code QKV table
    // (built or refreshed at streams_begin; Q3T_CP_QKV_TABLE=0 turns it off)
    c->s_tab = true;
    if (const char * e = std::getenv("Q3T_CP_QKV_TABLE")) if (e[0] == '0') c->s_tab = false;
    c->sb_ctx = n_ctx;
    c->s_emitted.assign(B, 0);
    return sync(c);
}

}  // extern "C"

namespace {

// Runs fn with the context's cache pointers set to stream b's cache slice.
template <class F>
int with_stream_cache(q3t_dev * c, int32_t stream, F fn) {
    if (stream < 0 || stream >= c->nb) return fail(c, "stream index out of range (q3t_dev_streams_reserve first)");
    if (c->n_ctx != c->sb_ctx) return fail(c, "KV cache re-reserved since q3t_dev_streams_reserve; reserve the streams again");
    const q3t_config & g = c->cfg;
    const size_t kv = (size_t) g.n_layers * g.n_kv_head * c->sb_ctx * g.head_dim;
    uint16_t * kc0 = c->kc, * vc0 = c->vc;
    c->kc = c->skc + stream * kv;
    c->vc = c->svc + stream * kv;
    const int rc = fn();
    c->kc = kc0;
    c->vc = vc0;
    return rc;
}

}  // namespace

extern "C" {

int q3t_dev_stream_kv_write(q3t_dev * c, int32_t stream, int32_t layer, int32_t n_pos, const uint16_t * k,
                            const uint16_t * v) {
    if (!c || !k || !v) return -1;
    return with_stream_cache(c, stream, [&] { return q3t_dev_kv_write(c, layer, n_pos, k, v); });
}

int q3t_dev_stream_prefill_at(q3t_dev * c, int32_t stream, const float * embd, int32_t n, int32_t n_past) {
    if (!c || !embd) return -1;
    if (n < 1 || n_past < 0 || n_past + n > c->sb_ctx) return fail(c, "Context length exceeded");
    HIP_OK(hipSetDevice(c->device));
    const q3t_config & g = c->cfg;
    // the single-stream prefill against this stream's cache
    const int rc = with_stream_cache(c, stream, [&] { return q3t_dev_prefill(c, embd, n, n_past, nullptr, nullptr); });
    if (rc) return rc;
    HIP_OK(hipMemcpyAsync(c->slogits + (size_t) stream * g.codec_vocab, c->logits, (size_t) g.codec_vocab * 4,
                          hipMemcpyDeviceToDevice, c->stream));
    HIP_OK(hipMemcpyAsync(c->shidden + (size_t) stream * g.hidden_size, c->hidden, (size_t) g.hidden_size * 4,
                          hipMemcpyDeviceToDevice, c->stream));
    return sync(c);
}

int q3t_dev_stream_prefill(q3t_dev * c, int32_t stream, const float * embd, int32_t n) {
    return q3t_dev_stream_prefill_at(c, stream, embd, n, 0);
}

int q3t_dev_streams_begin(q3t_dev * c, const q3t_frame_args * args) {
    if (!c || !args) return -1;
    if (c->nb < 1) return fail(c, "q3t_dev_streams_reserve first");
    if (c->n_ctx != c->sb_ctx) return fail(c, "KV cache re-reserved since q3t_dev_streams_reserve; reserve the streams again");
    HIP_OK(hipSetDevice(c->device));
    // the table keeps its address when rebuilt, so a captured frame graph stays valid
    if (c->s_tab && (!c->cp_tab || c->cp_tab_stale) && build_cp_tab(c)) return -1;
    const q3t_config & g = c->cfg;
    const int d = g.hidden_size, B = c->nb;
    int max_len = 0, max_trail = 1;
    for (int b = 0; b < B; ++b) {
        const q3t_frame_args & a = args[b];
        if (!a.tts_pad) return fail(c, "tts_pad row is null");
        if (a.n_trailing < 0 || (a.n_trailing > 0 && !a.trailing)) return fail(c, "bad trailing rows");
        if (a.max_len < 0 || a.max_len >= (1 << 19)) return fail(c, "max_len out of range");
        if (a.n_past < 1 || a.n_past + a.max_len > c->sb_ctx) return fail(c, "Context length exceeded");
        max_len = std::max(max_len, a.max_len);
        max_trail = std::max(max_trail, a.n_trailing);
    }
    if (max_len > c->scodes_cap || max_trail > c->strail_cap) {
        if (c->scodes) dev_free(c, c->scodes);
        if (c->strail) dev_free(c, c->strail);
        c->scodes = nullptr; c->strail = nullptr;
        const int cap = std::max(max_len, c->scodes_cap), tcap = std::max(max_trail, c->strail_cap);
        if (dev_alloc_t(c, &c->scodes, (size_t) B * std::max(cap, 1) * 16) ||
            dev_alloc_t(c, &c->strail, (size_t) B * tcap * d))
            return -1;
        c->scodes_cap = std::max(cap, 1);
        c->strail_cap = tcap;
        drop_stream_graph(c);
    }
    std::vector<FrameState> st(B);
    std::vector<SampleParams> sp(B);
    std::vector<int32_t> ntr(B);
    for (int b = 0; b < B; ++b) {
        const q3t_frame_args & a = args[b];
        st[b] = FrameState{};
        st[b].base_pos = a.n_past; st[b].talker_pos = a.n_past; st[b].max_frames = a.max_len;
        sp[b] = SampleParams{};
        sp[b].temperature = a.sampling.temperature; sp[b].top_k = a.sampling.top_k;
        sp[b].rep_penalty = a.repetition_penalty; sp[b].eos_bias = a.eos_bias;
        sp[b].target_frames = a.target_frames; sp[b].seed = a.sampling.seed;
        ntr[b] = a.n_trailing;
        if (a.n_trailing)
            HIP_OK(hipMemcpyAsync(c->strail + (size_t) b * c->strail_cap * d, a.trailing, (size_t) a.n_trailing * d * 4,
                                  hipMemcpyHostToDevice, c->stream));
        HIP_OK(hipMemcpyAsync(c->spad + (size_t) b * d, a.tts_pad, (size_t) d * 4, hipMemcpyHostToDevice, c->stream));
    }
    HIP_OK(hipMemcpyAsync(c->sst, st.data(), sizeof(FrameState) * B, hipMemcpyHostToDevice, c->stream));
    HIP_OK(hipMemcpyAsync(c->sparams, sp.data(), sizeof(SampleParams) * B, hipMemcpyHostToDevice, c->stream));
    HIP_OK(hipMemcpyAsync(c->sntrail, ntr.data(), sizeof(int32_t) * B, hipMemcpyHostToDevice, c->stream));
    HIP_OK(hipMemsetAsync(c->sseen, 0, (size_t) B * g.codec_vocab, c->stream));
    if (sync(c)) return -1;
    // the F16 GEMM form is fixed in the captured graph: recapture on a change
    const bool hm = !ms_exact();
    if (c->s_exec && hm != c->s_hm) drop_stream_graph(c);
    c->s_hm = hm;
    if (!c->s_exec) {
        HIP_OK(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
        streams_frame_seq(c);
        hipGraph_t graph = nullptr;
        HIP_OK(hipStreamEndCapture(c->stream, &graph));
        c->s_graph = graph;
        HIP_OK(hipGraphInstantiate(&c->s_exec, graph, nullptr, nullptr, 0));
    }
    c->s_emitted.assign(B, 0);
    c->s_launched = 0;
    c->s_max = max_len;
    c->s_ready = true;
    c->run_us = 0.0;
    c->run_frames = 0;
    c->stats_streams = true;
    return 0;
}

int q3t_dev_streams_run(q3t_dev * c, int32_t n_frames, int32_t * codes_out, int32_t * n_emitted_out, int32_t * eos_out) {
    if (!c) return -1;
    if (!c->s_ready) return fail(c, "q3t_dev_streams_begin not called");
    HIP_OK(hipSetDevice(c->device));
    const int B = c->nb;
    const int n = std::max(0, std::min(n_frames, c->s_max - c->s_launched));
    static const bool no_graph = [] { const char * e = std::getenv("Q3T_NO_GRAPH"); return e && e[0] == '1'; }();
    if (!c->run_ev[0]) {
        HIP_OK(hipEventCreate(&c->run_ev[0]));
        HIP_OK(hipEventCreate(&c->run_ev[1]));
    }
    if (n > 0) HIP_OK(hipEventRecord(c->run_ev[0], c->stream));
    for (int i = 0; i < n; ++i) {
        if (no_graph) streams_frame_seq(c);
        else HIP_OK(hipGraphLaunch(c->s_exec, c->stream));
    }
    if (n > 0) HIP_OK(hipEventRecord(c->run_ev[1], c->stream));
    c->s_launched += n;
    std::vector<FrameState> st(B);
    int32_t err = 0;
    HIP_OK(hipMemcpyAsync(st.data(), c->sst, sizeof(FrameState) * B, hipMemcpyDeviceToHost, c->stream));
    HIP_OK(hipMemcpyAsync(&err, c->serr, sizeof err, hipMemcpyDeviceToHost, c->stream));
    if (sync(c)) return -1;
    if (err) {
        c->s_ready = false;
        return fail(c, "multi-stream decode: a split-K partial never arrived (device wait timed out)");
    }
    if (n > 0) {
        float ms = 0.0f;
        HIP_OK(hipEventElapsedTime(&ms, c->run_ev[0], c->run_ev[1]));
        c->run_us += 1e3 * ms;
        c->run_frames += n;
    }
    for (int b = 0; b < B; ++b) {
        const int fresh = st[b].n_emitted - c->s_emitted[b];
        if (fresh > 0 && codes_out)
            HIP_OK(hipMemcpy(codes_out + (size_t) b * std::max(n_frames, 1) * 16,
                             c->scodes + ((size_t) b * c->scodes_cap + c->s_emitted[b]) * 16, (size_t) fresh * 16 * 4,
                             hipMemcpyDeviceToHost));
        if (n_emitted_out) n_emitted_out[b] = std::max(fresh, 0);
        if (eos_out) eos_out[b] = st[b].eos;
        c->s_emitted[b] = st[b].n_emitted;
    }
    return 0;
}

int q3t_dev_stream_logits(q3t_dev * c, int32_t stream, float * out) {
    if (!c || !out) return -1;
    HIP_OK(hipSetDevice(c->device));
    if (!c->slogits || stream < 0 || stream >= c->nb) return fail(c, "stream_logits: no such stream");
    const size_t n = (size_t) c->cfg.codec_vocab;
    HIP_OK(hipMemcpyAsync(out, c->slogits + (size_t) stream * n, n * 4, hipMemcpyDeviceToHost, c->stream));
    return sync(c);
}

int q3t_dev_frames_stats(q3t_dev * c, double * gpu_us_out, int64_t * frames_out, int32_t * path_out) {
    if (!c) return -1;
    if (gpu_us_out) *gpu_us_out = c->run_us;
    if (frames_out) *frames_out = c->run_frames;
    if (path_out) *path_out = c->stats_streams ? 2 : c->fk_ok ? (fk_xcd(c->fk_variant) ? 3 : 1) : 0;
    return 0;
}

int q3t_dev_sync(q3t_dev * c) {
    if (!c) return -1;
    HIP_OK(hipSetDevice(c->device));
    return sync(c);
}

int q3t_dev_time_kernel(q3t_dev * c, int32_t which, int32_t iters, double * avg_us_out, double * bytes_out) {
    if (!c || iters <= 0) return -1;
    HIP_OK(hipSetDevice(c->device));
    if (check_ready(c)) return -1;
    const q3t_config & g = c->cfg;
    const int d = g.hidden_size, qd = g.n_head * g.head_dim, kd = g.n_kv_head * g.head_dim;
    const LayerDev & L = c->talker[0];
    auto wbytes = [](const Slot & s) { return (double) type_bytes(s.type, s.ne0, s.ne1); };
    double bytes = 0.0;
    GemvSpec s{};
    const int pos = std::min(c->n_ctx - 1, 512);
    if (which < 0 || which > 5) return fail(c, "unknown kernel class");
    if (which == 5 && !c->copy_buf) {
        // 64 MiB source + 64 MiB destination for the copy-kernel calibration
        if (dev_alloc(c, (void **) &c->copy_buf, (size_t) 2 * kCopyBytes)) return -1;
        HIP_OK(hipMemsetAsync(c->copy_buf, 0, (size_t) 2 * kCopyBytes, c->stream));
    }
    {
        FrameState st{};
        st.talker_pos = pos;
        if (set_state(c, st)) return -1;
    }
    auto enqueue = [&]() {
        switch (which) {
            case 0:
                s = GemvSpec{}; s.w = weight_of(L.wg); s.w2 = weight_of(L.wu); s.rows = g.ffn_size; s.K = d;
                s.x = c->xb; s.x_stride = d; s.norm_w = L.ffn_norm; s.y = c->ffn; s.y_stride = g.ffn_size; s.epi = EPI_SWIGLU;
                gemv(c, s, 1);
                bytes = wbytes(L.wg) + wbytes(L.wu);
                break;
            case 1:
                s = GemvSpec{}; s.w = weight_of(L.qkv); s.rows = qd + 2 * kd; s.K = d; s.x = c->xa; s.x_stride = d;
                s.norm_w = L.attn_norm; s.y = c->qkv; s.y_stride = qd + 2 * kd;
                gemv(c, s, 1);
                bytes = wbytes(L.qkv);
                break;
            case 2:
                s = GemvSpec{}; s.w = weight_of(L.wd, true); s.rows = d; s.K = g.ffn_size; s.x = c->ffn; s.x_stride = g.ffn_size;
                s.y = c->xa; s.y_stride = d; s.resid = c->xb; s.resid_stride = d; s.epi = EPI_RESID;
                gemv(c, s, 1);
                bytes = wbytes(L.wd);
                break;
            case 3:
                s = GemvSpec{}; s.w = weight_of(L.wo); s.rows = d; s.K = qd; s.x = c->attn; s.x_stride = qd;
                s.y = c->xb; s.y_stride = d; s.resid = c->xa; s.resid_stride = d; s.epi = EPI_RESID;
                gemv(c, s, 1);
                bytes = wbytes(L.wo);
                break;
            case 4: {
                AttnSpec as{c->qkv, &L, c->kc, c->vc, c->n_ctx, c->rope_cos, c->rope_sin, &c->st->talker_pos, 0};
                attention(c, as, 1);
                bytes = 2.0 * (double) (pos + 1) * kd * 2;   // K and V rows read
                break;
            }
            case 5: {
                const size_t n16 = kCopyBytes / 16;
                hipLaunchKernelGGL(k_copy16, dim3(4096), dim3(256), 0, c->stream, (const int4 *) c->copy_buf,
                                   (int4 *) (c->copy_buf + kCopyBytes), n16);
                bytes = 2.0 * (double) kCopyBytes;   // read + write
                break;
            }
            default:
                break;
        }
    };
    enqueue();   // warm-up
    if (sync(c)) return -1;
    hipEvent_t e0, e1;
    HIP_OK(hipEventCreate(&e0));
    HIP_OK(hipEventCreate(&e1));
    HIP_OK(hipEventRecord(e0, c->stream));
    for (int i = 0; i < iters; ++i) enqueue();
    HIP_OK(hipEventRecord(e1, c->stream));
    HIP_OK(hipEventSynchronize(e1));
    float ms = 0.0f;
    HIP_OK(hipEventElapsedTime(&ms, e0, e1));
    (void) hipEventDestroy(e0);
    (void) hipEventDestroy(e1);
    if (avg_us_out) *avg_us_out = (double) ms * 1000.0 / iters;
    if (bytes_out) *bytes_out = bytes;
    return sync(c);
}

}  // extern "C"
