// CPU emulation of the sampler's kernels (test infrastructure only).
//
// Runs the unchanged kernel sources (compiled as host C++ against
// tests/emu/include/hip/hip_runtime.h) one workgroup at a time: every lane
// is a cooperative fiber on its own stack.  A lane runs until it reaches a
// synchronising operation, then the next lane runs.  When every live lane
// of the block waits:
//   * the lanes of a wave that wait at one wave operation (same source site
//     and kind) complete it with exact wave64 semantics over those lanes,
//     the wave's other lanes being inactive, as under an EXEC mask (a
//     shuffle that reads an inactive lane aborts the run);
//   * otherwise, when every live lane of the block waits at a barrier, the
//     barrier opens;
//   * anything else (a barrier some live lane never reaches) is reported
//     and aborts.
// Built with AddressSanitizer and -fsanitize=bounds, a run also checks
// every global-memory access (each buffer is its own allocation) and every
// LDS array index (each __shared__ object is a redzoned static).
//
// main(): reads a case (logits, params) from a binary file, calls the real
// C ABI entry mis_sample() and writes ids, status, probabilities and the
// keep bitmask to another file for the Python side to compare with the
// oracle.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <sys/mman.h>

#include <vector>

#include "mis_sampler.h"

#if defined(__has_feature)
#if __has_feature(address_sanitizer)
#define EMU_ASAN 1
#endif
#endif
#ifdef EMU_ASAN
#include <sanitizer/asan_interface.h>
#include <sanitizer/common_interface_defs.h>
#endif

// x86-64 (System V) fiber switch: saves the callee-saved registers, MXCSR
// and the x87 control word on the current stack, stores the stack pointer
// in *from and resumes the fiber whose stack pointer is `to`.  No system
// calls (ucontext's swapcontext makes two per switch).
extern "C" void emu_ctx_switch(void **from, void *to);
asm(R"(
    .text
    .globl emu_ctx_switch
    .type emu_ctx_switch, @function
emu_ctx_switch:
    pushq %rbp
    pushq %rbx
    pushq %r12
    pushq %r13
    pushq %r14
    pushq %r15
    subq $8, %rsp
    stmxcsr (%rsp)
    fnstcw 4(%rsp)
    movq %rsp, (%rdi)
    movq %rsi, %rsp
    ldmxcsr (%rsp)
    fldcw 4(%rsp)
    addq $8, %rsp
    popq %r15
    popq %r14
    popq %r13
    popq %r12
    popq %rbx
    popq %rbp
    ret
    .size emu_ctx_switch, .-emu_ctx_switch
)");

namespace emu {

namespace {

enum State : int { RUN = 0, BAR = 1, WAVE = 2, DONE = 3 };

struct Lane {
    void *sp = nullptr;              // saved stack pointer while switched out
    void *stack = nullptr;
    dim3 tid;
    int lin = 0;
    State st = RUN;
    const char *site = nullptr;
    int kind = 0, arg = 0, width = 64;
    uint64_t in = 0, out = 0;
};

constexpr size_t STACK = 256 * 1024;

struct Block {
    std::vector<Lane> lanes;
    int n = 0;
    dim3 bidx, bdim, gdim;
    void *sched_sp = nullptr;
    Lane *cur = nullptr;
    const std::function<void()> *fn = nullptr;
    const char *kernel = "";
    void *fake_stack = nullptr;  // ASan fiber bookkeeping of the scheduler
};

Block g_blk;
const dim3 g_zero(0, 0, 0);
const void *g_main_bottom = nullptr;  // the scheduler's (main thread's) stack, for ASan
size_t g_main_size = 0;

[[noreturn]] void die(const char *what, const char *a = "", const char *b = "")
{
    fprintf(stderr, "[emu] %s: %s %s (kernel %s, block %u,%u)\n", what, a, b, g_blk.kernel, g_blk.bidx.x, g_blk.bidx.y);
    fflush(stderr);
    abort();
}

void switch_to_sched(Lane *l)
{
#ifdef EMU_ASAN
    void *fs = nullptr;
    __sanitizer_start_switch_fiber(l->st == DONE ? nullptr : &fs, g_main_bottom, g_main_size);
#endif
    emu_ctx_switch(&l->sp, g_blk.sched_sp);
#ifdef EMU_ASAN
    __sanitizer_finish_switch_fiber(fs, &g_main_bottom, &g_main_size);
#endif
}

void lane_entry()
{
#ifdef EMU_ASAN
    __sanitizer_finish_switch_fiber(nullptr, &g_main_bottom, &g_main_size);
#endif
    (*g_blk.fn)();
    Lane *l = g_blk.cur;
    l->st = DONE;
    switch_to_sched(l);
    die("a finished lane was resumed");
}

void block_until_resumed(State st, const char *site)
{
    Lane *l = g_blk.cur;
    l->st = st;
    l->site = site;
    switch_to_sched(l);
}

void resume(Lane &l)
{
    g_blk.cur = &l;
#ifdef EMU_ASAN
    __sanitizer_start_switch_fiber(&g_blk.fake_stack, l.stack, STACK);
#endif
    emu_ctx_switch(&g_blk.sched_sp, l.sp);
#ifdef EMU_ASAN
    __sanitizer_finish_switch_fiber(g_blk.fake_stack, nullptr, nullptr);
#endif
    g_blk.cur = nullptr;
}

// one wave's operation: every live lane in `w` waits at it
void complete_wave(std::vector<Lane *> &w)
{
    const int kind = w[0]->kind;
    uint64_t present = 0;
    uint64_t val[64];
    for (Lane *l : w) { const int ln = l->lin & 63; present |= 1ull << ln; val[ln] = l->in; }
    if (kind == OP_BALLOT) {
        uint64_t m = 0;
        for (Lane *l : w) if (l->in) m |= 1ull << (l->lin & 63);
        for (Lane *l : w) l->out = m;
    } else if (kind == OP_FIRST) {
        const int f = __builtin_ctzll(present);
        for (Lane *l : w) l->out = val[f];
    } else {
        for (Lane *l : w) {
            const int ln = l->lin & 63, wd = l->width, base = ln & ~(wd - 1);
            int src = ln;
            if (kind == OP_SHFL) src = base + (l->arg & (wd - 1));
            else if (kind == OP_XOR) src = ln ^ l->arg;
            else if (kind == OP_UP) src = (ln - base) >= l->arg ? ln - l->arg : ln;
            else if (kind == OP_DOWN) src = (ln - base) + l->arg < wd ? ln + l->arg : ln;
            if (src < 0 || src > 63 || !((present >> src) & 1ull))
                die("shuffle reads a lane that is not active", l->site);
            l->out = val[src];
        }
    }
    for (Lane *l : w) l->st = RUN;
}

void run_block()
{
    Block &b = g_blk;
    for (;;) {
        bool any = false;
        for (int i = 0; i < b.n; ++i) {
            if (b.lanes[i].st == RUN) { resume(b.lanes[i]); any = true; }
        }
        if (any) continue;
        // every lane waits or is done
        int live = 0, atbar = 0;
        for (int i = 0; i < b.n; ++i) {
            if (b.lanes[i].st != DONE) ++live;
            if (b.lanes[i].st == BAR) ++atbar;
        }
        if (live == 0) return;
        bool progressed = false;
        for (int w0 = 0; w0 < b.n; w0 += 64) {
            // lanes of this wave waiting at wave operations, grouped by
            // (site, kind): each group is one set of active lanes, the
            // others being inactive (at a barrier, at another operation of
            // a divergent branch, or exited), as under an EXEC mask
            std::vector<Lane *> pend;
            for (int i = w0; i < w0 + 64 && i < b.n; ++i)
                if (b.lanes[i].st == WAVE) pend.push_back(&b.lanes[i]);
            while (!pend.empty()) {
                std::vector<Lane *> grp, rest;
                for (Lane *l : pend)
                    (l->site == pend[0]->site && l->kind == pend[0]->kind ? grp : rest).push_back(l);
                complete_wave(grp);
                pend.swap(rest);
                progressed = true;
            }
        }
        if (progressed) continue;
        if (atbar == live) {
            for (int i = 0; i < b.n; ++i) if (b.lanes[i].st == BAR) b.lanes[i].st = RUN;
            continue;
        }
        die("deadlock: lanes wait at operations that cannot complete");
    }
}

}  // namespace

uint64_t clock_tick()
{
    static uint64_t t = 0;
    return ++t;
}

const dim3 &thread_idx() { return g_blk.cur ? g_blk.cur->tid : g_zero; }
const dim3 &block_idx() { return g_blk.bidx; }
const dim3 &block_dim() { return g_blk.bdim; }
const dim3 &grid_dim() { return g_blk.gdim; }

void syncthreads(const char *site)
{
    if (!g_blk.cur) die("__syncthreads outside a kernel", site);
    block_until_resumed(BAR, site);
}

uint64_t wave_op(int kind, uint64_t v, int arg, int width, const char *site)
{
    Lane *l = g_blk.cur;
    if (!l) die("wave operation outside a kernel", site);
    if (width <= 0 || width > 64 || (width & (width - 1))) die("bad shuffle width", site);
    l->kind = kind; l->in = v; l->arg = arg; l->width = width;
    block_until_resumed(WAVE, site);
    return l->out;
}

void launch(dim3 grid, dim3 block, const std::function<void()> &fn, const char *name)
{
    const int n = (int)(block.x * block.y * block.z);
    if (n <= 0 || n > 1024) die("bad block size", name);
    Block &b = g_blk;
    if ((int)b.lanes.size() < n) {
        b.lanes.resize(n);
        for (auto &l : b.lanes)
            if (!l.stack) {
                l.stack = mmap(nullptr, STACK, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
                if (l.stack == MAP_FAILED) die("mmap of a lane stack failed");
            }
    }
    b.n = n; b.bdim = block; b.gdim = grid; b.fn = &fn; b.kernel = name;
    for (unsigned z = 0; z < grid.z; ++z)
        for (unsigned y = 0; y < grid.y; ++y)
            for (unsigned x = 0; x < grid.x; ++x) {
                b.bidx = dim3(x, y, z);
                for (int i = 0; i < n; ++i) {
                    Lane &l = b.lanes[i];
                    l.lin = i;
                    l.tid = dim3(i % block.x, (i / block.x) % block.y, i / (block.x * block.y));
                    l.st = RUN;
                    l.site = nullptr;
#ifdef EMU_ASAN
                    // the previous fiber's frames on this stack left their
                    // redzones poisoned
                    __asan_unpoison_memory_region(l.stack, STACK);
#endif
                    // initial frame: control words, six callee-saved
                    // registers, then lane_entry as the return address
                    uint64_t *top = (uint64_t *)((char *)l.stack + STACK);
                    uint64_t *sp = top - 9;
                    sp[0] = 0x037f00001f80ull;  // MXCSR default, x87 control word default
                    for (int r = 1; r <= 6; ++r) sp[r] = 0;
                    sp[7] = (uint64_t)(uintptr_t)&lane_entry;
                    sp[8] = 0;  // lane_entry never returns
                    l.sp = sp;
                }
                run_block();
            }
}

}  // namespace emu

// ---------------------------------------------------------------- driver
//
// case file (little endian):
//   i32 magic 0x4d495345, i32 dtype, i64 B, i64 V, i32 want_debug, i32 kinds
//   logits  B*V elements (4 or 2 bytes each)
//   params  B * 16 bytes (mis_row_params)
// output file:
//   ids B*i64, status B*i32, then (want_debug) probs B*V*f32, keep B*ceil(V/32)*u32

template <class T> static std::vector<T> alloc_exact(size_t n) { return std::vector<T>(n); }

int main(int argc, char **argv)
{
    if (argc != 3) { fprintf(stderr, "usage: %s case.bin out.bin\n", argv[0]); return 2; }
    FILE *f = fopen(argv[1], "rb");
    if (!f) { perror("case"); return 2; }
    int32_t magic, dtype, want, kinds;
    int64_t B, V;
    if (fread(&magic, 4, 1, f) != 1 || magic != 0x4d495345 || fread(&dtype, 4, 1, f) != 1 || fread(&B, 8, 1, f) != 1 ||
        fread(&V, 8, 1, f) != 1 || fread(&want, 4, 1, f) != 1 || fread(&kinds, 4, 1, f) != 1) {
        fprintf(stderr, "bad case header\n");
        return 2;
    }
    const size_t esz = dtype == MIS_DTYPE_F32 ? 4 : 2;
    // every buffer is its own exact-size heap allocation, so AddressSanitizer
    // flags any access past its end
    char *logits = (char *)malloc((size_t)B * V * esz);
    mis_row_params *params = (mis_row_params *)malloc((size_t)B * sizeof(mis_row_params));
    if (fread(logits, esz, (size_t)B * V, f) != (size_t)(B * V) || fread(params, sizeof(mis_row_params), (size_t)B, f) != (size_t)B) {
        fprintf(stderr, "short case file\n");
        return 2;
    }
    fclose(f);
    const size_t ws_bytes = mis_workspace_bytes(B, V, dtype);
    // a MIS_TRACE build writes a [B][32] u64 timestamp table past the workspace
    const char *trace_out = getenv("EMU_TRACE_OUT");
    const size_t tr_bytes = trace_out ? (size_t)B * 32 * 8 : 0;
    void *ws = aligned_alloc(256, (ws_bytes + tr_bytes + 255) & ~(size_t)255);
    memset(ws, 0xa5, ws_bytes);  // nothing may depend on the workspace's prior contents
    if (tr_bytes) memset((char *)ws + ws_bytes, 0, tr_bytes);
    int64_t *ids = (int64_t *)malloc((size_t)B * 8);
    int32_t *status = (int32_t *)malloc((size_t)B * 4);
    const int64_t W = (V + 31) / 32;
    float *probs = want ? (float *)malloc((size_t)B * V * 4) : nullptr;
    uint32_t *keep = want ? (uint32_t *)malloc((size_t)B * W * 4) : nullptr;
    if (want) { for (int64_t i = 0; i < B * V; ++i) probs[i] = -1.0f; memset(keep, 0, (size_t)B * W * 4); }
    // EMU_SIDE=1: with a context (the split schedule), else one stream
    mis_context *ctx = nullptr;
    if (getenv("EMU_SIDE") && atoi(getenv("EMU_SIDE")) && mis_context_create(&ctx) != MIS_OK) {
        fprintf(stderr, "mis_context_create failed\n");
        return 3;
    }
    // EMU_NOALLOC=1: through mis_sample_noalloc (its static scratch, one stream)
    const bool noalloc = getenv("EMU_NOALLOC") && atoi(getenv("EMU_NOALLOC"));
    const int rc = noalloc ? mis_sample_noalloc(logits, dtype, B, V, V, params, ids, status, probs, keep, nullptr,
                                                (unsigned)kinds)
                           : mis_sample_ex(logits, dtype, B, V, V, params, ids, status, probs, keep, ws, ws_bytes,
                                           nullptr, (unsigned)kinds, nullptr, ctx);
    mis_context_destroy(ctx);
    if (rc != MIS_OK) { fprintf(stderr, "mis_sample: %s\n", mis_strerror(rc)); return 3; }
    FILE *o = fopen(argv[2], "wb");
    if (!o) { perror("out"); return 2; }
    fwrite(ids, 8, (size_t)B, o);
    fwrite(status, 4, (size_t)B, o);
    if (want) { fwrite(probs, 4, (size_t)(B * V), o); fwrite(keep, 4, (size_t)(B * W), o); }
    fclose(o);
    if (const char *wo = getenv("EMU_WS_OUT")) {  // the workspace after the call
        FILE *t = fopen(wo, "wb");
        if (t) { fwrite(ws, 1, ws_bytes, t); fclose(t); }
    }
    if (trace_out) {
        FILE *t = fopen(trace_out, "wb");
        if (t) { fwrite((char *)ws + ws_bytes, 1, tr_bytes, t); fclose(t); }
    }
    free(logits); free(params); free(ws); free(ids); free(status); free(probs); free(keep);
    return 0;
}
