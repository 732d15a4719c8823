/* Fiber scheduler of the SIMT emulator (see simt.h).
 *
 * Fibers switch through a six-register x86-64 context switch (no signal-mask syscall per switch).
 * SIMT_ORDER=fwd|rev|rand picks the order in which the fibers of a workgroup run between two
 * barriers: a kernel whose output changes with the order has a race between barriers. With
 * SIMT_POISON_LDS defined at build time every `__shared__` variable is filled with 0xA5 bytes before
 * each workgroup (LDS holds stale data on the device, not zeros). */
#include "simt.h"

#include <stdio.h>

#if defined(__SANITIZE_ADDRESS__)
extern "C" void __sanitizer_start_switch_fiber(void **fake_stack_save, const void *bottom, size_t size);
extern "C" void __sanitizer_finish_switch_fiber(void *fake_stack_save, const void **bottom_old, size_t *size_old);
#define SIMT_ASAN 1
#else
#define SIMT_ASAN 0
#endif

extern "C" void simt_switch(void **save_sp, void *new_sp);
asm(R"(
.text
.globl simt_switch
.type simt_switch,@function
simt_switch:
  pushq %rbp
  pushq %rbx
  pushq %r12
  pushq %r13
  pushq %r14
  pushq %r15
  movq %rsp, (%rdi)
  movq %rsi, %rsp
  popq %r15
  popq %r14
  popq %r13
  popq %r12
  popq %rbx
  popq %rbp
  ret
.size simt_switch,.-simt_switch
)");

#if defined(SIMT_POISON_LDS)
extern "C" char __start_simt_lds[], __stop_simt_lds[];
#endif

namespace simt {

static const size_t STACK = 256 << 10;

struct Fiber {
  void *sp = nullptr;
  char *stack = nullptr;
  bool done = false;
  const char *file = nullptr; /* site of the wave operation in progress */
  int line = 0;
};

struct Block {
  dim3 bid, bdim, gdim;
  int n = 0;
  std::vector<Fiber> f;
  void *sched_sp = nullptr;
  int block_gen = 0, block_arrived = 0;
  const char *block_site = nullptr;
  int block_line = 0;
  std::vector<int> wave_gen, wave_arrived;
  std::vector<const char *> wave_file;
  std::vector<int> wave_line;
  std::vector<std::vector<uint64_t>> slots;
  const std::function<void()> *body = nullptr;
  long progress = 0;
};

static Block *g_blk = nullptr;
static int g_tid = 0;
static int g_order = -1; /* 0 fwd, 1 rev, 2 rand */
static uint64_t g_rand = 0x9E3779B97F4A7C15ull;

dim3 tidx() {
  unsigned x = g_tid % g_blk->bdim.x;
  unsigned y = (g_tid / g_blk->bdim.x) % g_blk->bdim.y;
  return dim3(x, y, 0);
}
dim3 bidx() { return g_blk->bid; }
dim3 bdim() { return g_blk->bdim; }
dim3 gdim() { return g_blk->gdim; }
int lane_id() { return g_tid & 63; }
uint64_t *wave_slots() { return g_blk->slots[g_tid >> 6].data(); }

static void to_sched() {
  Fiber &me = g_blk->f[g_tid];
#if SIMT_ASAN
  void *fake = nullptr;
  __sanitizer_start_switch_fiber(&fake, nullptr, 0);
#endif
  simt_switch(&me.sp, g_blk->sched_sp);
#if SIMT_ASAN
  __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
#endif
}

static int live_in_block() {
  int k = 0;
  for (auto &x : g_blk->f) k += !x.done;
  return k;
}
static int live_in_wave(int w) {
  int k = 0;
  for (int i = w * 64; i < std::min(g_blk->n, w * 64 + 64); i++) k += !g_blk->f[i].done;
  return k;
}

void sync_block_at(const char *file, int line) {
  Block &b = *g_blk;
  int gen = b.block_gen;
  if (b.block_arrived == 0) {
    b.block_site = file;
    b.block_line = line;
  } else if (b.block_site != file || b.block_line != line) {
    fprintf(stderr, "simt: block (%u,%u) thread %d reached the barrier at %s:%d while others wait at %s:%d\n",
            b.bid.x, b.bid.y, g_tid, file, line, b.block_site, b.block_line);
    abort();
  }
  b.block_arrived++;
  b.progress++;
  if (b.block_arrived == live_in_block()) {
    b.block_arrived = 0;
    b.block_gen++;
    return;
  }
  while (b.block_gen == gen) to_sched();
}

/* Called before the wave operation's first rendezvous. A site is recorded by the first lane of the
 * wave to arrive at a new rendezvous and checked against every other lane's. */
void wave_site(const char *file, int line) {
  g_blk->f[g_tid].file = file;
  g_blk->f[g_tid].line = line;
}

void sync_wave() {
  Block &b = *g_blk;
  int w = g_tid >> 6;
  int gen = b.wave_gen[w];
  const char *t_file = b.f[g_tid].file;
  const int t_line = b.f[g_tid].line;
  if (b.wave_arrived[w] == 0) {
    b.wave_file[w] = t_file;
    b.wave_line[w] = t_line;
  } else if (b.wave_file[w] != t_file || b.wave_line[w] != t_line) {
    fprintf(stderr, "simt: block (%u,%u) wave %d: lane %d at the wave operation %s:%d, others at %s:%d\n", b.bid.x,
            b.bid.y, w, g_tid & 63, t_file, t_line, b.wave_file[w], b.wave_line[w]);
    abort();
  }
  b.wave_arrived[w]++;
  b.progress++;
  if (b.wave_arrived[w] == live_in_wave(w)) {
    b.wave_arrived[w] = 0;
    b.wave_gen[w]++;
    return;
  }
  while (b.wave_gen[w] == gen) to_sched();
}

static void trampoline() {
#if SIMT_ASAN
  __sanitizer_finish_switch_fiber(nullptr, nullptr, nullptr);
#endif
  int tid = g_tid;
  (*g_blk->body)();
  Block &b = *g_blk;
  b.f[tid].done = true;
  b.progress++;
  /* a finished fiber may complete a barrier the others wait on */
  if (b.block_arrived > 0 && b.block_arrived == live_in_block()) {
    b.block_arrived = 0;
    b.block_gen++;
  }
  int w = tid >> 6;
  if (b.wave_arrived[w] > 0 && b.wave_arrived[w] == live_in_wave(w)) {
    b.wave_arrived[w] = 0;
    b.wave_gen[w]++;
  }
#if SIMT_ASAN
  __sanitizer_start_switch_fiber(nullptr, nullptr, 0);
#endif
  void *dead;
  simt_switch(&dead, b.sched_sp);
  abort();
}

static void init_fiber(Fiber &x) {
  x.stack = (char *)malloc(STACK);
  uintptr_t top = ((uintptr_t)x.stack + STACK) & ~(uintptr_t)15;
  void **sp = (void **)top;
  *--sp = nullptr;              /* trampoline's return address slot (never used) */
  *--sp = (void *)&trampoline;  /* popped by simt_switch's ret */
  for (int i = 0; i < 6; i++) *--sp = nullptr;
  x.sp = sp;
}

__attribute__((no_sanitize_address)) static void poison_lds() {
#if defined(SIMT_POISON_LDS)
  for (char *p = __start_simt_lds; p < __stop_simt_lds; p++) *(volatile char *)p = (char)0xA5;
#endif
}

void launch(dim3 grid, dim3 block, const std::function<void()> &body) {
  if (g_order < 0) {
    const char *o = getenv("SIMT_ORDER");
    g_order = !o ? 0 : !strcmp(o, "rev") ? 1 : !strcmp(o, "rand") ? 2 : 0;
  }
  int n = (int)(block.x * block.y * block.z);
  int nw = (n + 63) / 64;
  std::vector<int> order(n);
  for (unsigned bz = 0; bz < grid.z; bz++)
    for (unsigned by = 0; by < grid.y; by++)
      for (unsigned bx = 0; bx < grid.x; bx++) {
        Block b;
        b.bid = dim3(bx, by, bz);
        b.bdim = block;
        b.gdim = grid;
        b.n = n;
        b.f.resize(n);
        b.wave_gen.assign(nw, 0);
        b.wave_arrived.assign(nw, 0);
        b.wave_file.assign(nw, nullptr);
        b.wave_line.assign(nw, 0);
        b.slots.assign(nw, std::vector<uint64_t>(64, 0));
        b.body = &body;
        Block *prev = g_blk;
        int prev_tid = g_tid;
        g_blk = &b;
        poison_lds();
        for (int t = 0; t < n; t++) init_fiber(b.f[t]);
        for (int t = 0; t < n; t++) order[t] = g_order == 1 ? n - 1 - t : t;
        while (true) {
          if (g_order == 2)
            for (int t = n - 1; t > 0; t--) {
              g_rand ^= g_rand << 13, g_rand ^= g_rand >> 7, g_rand ^= g_rand << 17;
              std::swap(order[t], order[g_rand % (uint64_t)(t + 1)]);
            }
          bool any = false;
          long before = b.progress;
          for (int q = 0; q < n; q++) {
            int t = order[q];
            Fiber &x = b.f[t];
            if (x.done) continue;
            any = true;
            g_tid = t;
#if SIMT_ASAN
            void *fake = nullptr;
            __sanitizer_start_switch_fiber(&fake, x.stack, STACK);
#endif
            simt_switch(&b.sched_sp, x.sp);
#if SIMT_ASAN
            __sanitizer_finish_switch_fiber(fake, nullptr, nullptr);
#endif
          }
          if (!any) break;
          if (b.progress == before) {
            fprintf(stderr, "simt: deadlock in block (%u,%u,%u): %d live threads wait forever\n", bx, by, bz,
                    live_in_block());
            abort();
          }
        }
        for (auto &x : b.f) free(x.stack);
        g_blk = prev;
        g_tid = prev_tid;
      }
}

}  // namespace simt
