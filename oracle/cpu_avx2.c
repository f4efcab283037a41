/*
 * The CPU baseline: golem's x86 path for the quantised products -- its AVX2
 * kernels and its worker pool -- restated in C with intrinsics.
 *
 * TEST AND BENCHMARK INFRASTRUCTURE ONLY.  bench.py's cpu_baseline leg times
 * it on the GPU host's cores, and tests/ check it against the generic
 * restatement in oracle.c.  Nothing in golem_amd/ links or calls it.
 *
 * What is restated, and from where:
 *   - the worker pool: nn/parallel.go:36-191 (persistent workers as many as the
 *     threads allowed, spin 200,000 rounds of eight PAUSE then park, ranges
 *     handed out ceil(n / (4 chunks)) at a time, the caller takes ranges too,
 *     one section at a time), with the work threshold of nn/kernel.go:24;
 *   - dotQ6_KAVX2 (nn/dot_q6_k_amd64.s:62-125): the same integer steps, so the
 *     result is bit-identical to dotQ6_KGo (nn/dot_q6_k_test.go:51-75 holds
 *     golem to that), and matVecQ6_KRows' single-column loop
 *     (nn/dot_q6_k.go:77-103);
 *   - dotQ4_0AVX2 / x4 / x8 (nn/dot_q4_0_amd64.s:63-398) with their Begin /
 *     Finish state (nn/dot_q4_0.go:99-114), and matVecQ4_0Rows' tiling
 *     (nn/dot_q4_0.go:147-270): eight columns, then four, then one; stretches
 *     of 2048 inputs; row tiles of 24 KiB of weights, at most 64 rows.
 *
 * Build: gcc -O2 -mavx2 -mfma -mf16c -ffp-contract=off -pthread (oracle/build.py).
 */
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- the worker pool (nn/parallel.go) --------------------------------- */

#define SPIN_ROUNDS 200000           /* nn/parallel.go:38 */
#define PARALLEL_THRESHOLD (1 << 19) /* nn/kernel.go:24 */

typedef void (*cpu_work)(void *arg, int start, int end);

/* A worker's wake-up: a flag under a mutex, set at most once before it is
 * taken, like the one-slot channel a Go worker blocks on. */
struct slot {
    pthread_mutex_t mu;
    pthread_cond_t cv;
    int pending;
    atomic_int sleeping;
};

static struct {
    int count;
    cpu_work work;
    void *arg;
    int n, grain;
    atomic_long cursor;
    atomic_ulong sequence;
    atomic_long remaining;
    atomic_int spin;
    struct slot *slots;
    pthread_mutex_t section;
} pool = {.section = PTHREAD_MUTEX_INITIALIZER};

static pthread_mutex_t pool_init_mu = PTHREAD_MUTEX_INITIALIZER;

static void spin_pause(void) {
    for (int i = 0; i < 8; i++)
        _mm_pause();
}

static void consume(void) {
    for (;;) {
        const long start = atomic_fetch_add(&pool.cursor, pool.grain);
        if (start >= pool.n)
            return;
        const long end = start + pool.grain < pool.n ? start + pool.grain : pool.n;
        pool.work(pool.arg, (int)start, (int)end);
    }
}

static void park(struct slot *s) {
    pthread_mutex_lock(&s->mu);
    while (!s->pending)
        pthread_cond_wait(&s->cv, &s->mu);
    s->pending = 0;
    pthread_mutex_unlock(&s->mu);
}

static void wake(struct slot *s) {
    pthread_mutex_lock(&s->mu);
    s->pending = 1;
    pthread_cond_signal(&s->cv);
    pthread_mutex_unlock(&s->mu);
}

static void *serve(void *p) {
    struct slot *s = &pool.slots[(intptr_t)p];
    unsigned long last = 0;
    for (;;) {
        int spins = 0;
        while (atomic_load(&pool.sequence) == last) {
            spins++;
            if (spins > SPIN_ROUNDS || !atomic_load(&pool.spin)) {
                atomic_store(&s->sleeping, 1);
                /* a section published between the test and the flag */
                if (atomic_load(&pool.sequence) != last) {
                    atomic_store(&s->sleeping, 0);
                    break;
                }
                park(s);
                atomic_store(&s->sleeping, 0);
                spins = 0;
            }
            spin_pause();
        }
        last = atomic_load(&pool.sequence);
        consume();
        atomic_fetch_sub(&pool.remaining, 1);
    }
    return NULL;
}

/* Starts `threads` - 1 workers; the caller is the last one.  Once per process;
 * a later call with another count fails. */
int cpu_pool_init(int threads) {
    int rc = 0;
    pthread_mutex_lock(&pool_init_mu);
    if (pool.count) {
        rc = pool.count == threads ? 0 : -1;
    } else if (threads < 1) {
        rc = -2;
    } else {
        pool.slots = calloc((size_t)threads, sizeof(struct slot));
        for (int i = 0; i < threads; i++) {
            pthread_mutex_init(&pool.slots[i].mu, NULL);
            pthread_cond_init(&pool.slots[i].cv, NULL);
        }
        pool.count = threads;
        for (int i = 1; i < threads; i++) {
            pthread_t t;
            pthread_attr_t a;
            pthread_attr_init(&a);
            pthread_attr_setdetachstate(&a, PTHREAD_CREATE_DETACHED);
            if (pthread_create(&t, &a, serve, (void *)(intptr_t)i) != 0)
                rc = -3;
            pthread_attr_destroy(&a);
        }
    }
    pthread_mutex_unlock(&pool_init_mu);
    return rc;
}

int cpu_pool_threads(void) { return pool.count; }

static void pool_run(int n, int chunks, cpu_work work, void *arg) {
    int grain = (n + chunks * 4 - 1) / (chunks * 4);
    if (grain < 1)
        grain = 1;
    pool.work = work;
    pool.arg = arg;
    pool.n = n;
    pool.grain = grain;
    atomic_store(&pool.cursor, 0);
    atomic_store(&pool.spin, chunks >= pool.count);
    atomic_store(&pool.remaining, pool.count - 1);
    atomic_fetch_add(&pool.sequence, 1);
    for (int i = 1; i < pool.count; i++)
        if (atomic_load(&pool.slots[i].sleeping))
            wake(&pool.slots[i]);
    consume();
    while (atomic_load(&pool.remaining) != 0) {
        if (atomic_load(&pool.spin))
            spin_pause();
        else
            sched_yield();
    }
    pool.work = NULL;
}

/* InParallel (nn/parallel.go:177-191), with `limit` playing GOMAXPROCS: the
 * number of threads a call may use, so one pool times 1 and all threads. */
static void in_parallel(int n, long total_work, int limit, cpu_work work, void *arg) {
    int chunks = pool.count < limit ? pool.count : limit;
    if (chunks > n)
        chunks = n;
    if (total_work < PARALLEL_THRESHOLD)
        chunks = 1;
    if (chunks <= 1) {
        work(arg, 0, n);
        return;
    }
    pthread_mutex_lock(&pool.section);
    pool_run(n, chunks, work, arg);
    pthread_mutex_unlock(&pool.section);
}

/* ---- Q6_K (nn/dot_q6_k_amd64.s:62-125) -------------------------------- */

/* One chunk of 32 six-bit magnitudes against 32 activations: int16 pair sums,
 * then the two group scales (bytes 0..15 and 16..31) into int32 lanes. */
static inline __m256i q6_chunk(__m256i acc, __m256i mag, const int8_t *a, int16_t s_lo, int16_t s_hi) {
    const __m256i sc = _mm256_blend_epi32(_mm256_set1_epi16(s_lo), _mm256_set1_epi16(s_hi), 0xF0);
    const __m256i pairs = _mm256_maddubs_epi16(mag, _mm256_loadu_si256((const __m256i *)a));
    return _mm256_add_epi32(acc, _mm256_madd_epi16(pairs, sc));
}

static float dot_q6_k_avx2(const uint8_t *w, const int8_t *q, const int16_t *bsums, const float *kscales, int n) {
    const __m256i m4 = _mm256_set1_epi8(0x0F), m2 = _mm256_set1_epi8(0x03);
    float total = 0.0f;
    for (int b = 0; b < n / 256; b++, w += 210, q += 256, bsums += 16) {
        const __m256i sc = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(w + 192)));
        int16_t s[16];
        _mm256_storeu_si256((__m256i *)s, sc);
        __m256i acc = _mm256_setzero_si256();
        for (int h = 0; h < 2; h++) {
            const __m256i l0 = _mm256_loadu_si256((const __m256i *)(w + 64 * h));
            const __m256i l1 = _mm256_loadu_si256((const __m256i *)(w + 64 * h + 32));
            const __m256i hb = _mm256_loadu_si256((const __m256i *)(w + 128 + 32 * h));
            const int8_t *a = q + 128 * h;
            const int16_t *g = s + 8 * h;
            __m256i m;
            m = _mm256_or_si256(_mm256_and_si256(l0, m4), _mm256_slli_epi16(_mm256_and_si256(hb, m2), 4));
            acc = q6_chunk(acc, m, a, g[0], g[1]);
            m = _mm256_or_si256(_mm256_and_si256(l1, m4),
                                _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 2), m2), 4));
            acc = q6_chunk(acc, m, a + 32, g[2], g[3]);
            m = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l0, 4), m4),
                                _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 4), m2), 4));
            acc = q6_chunk(acc, m, a + 64, g[4], g[5]);
            m = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(l1, 4), m4),
                                _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 6), m2), 4));
            acc = q6_chunk(acc, m, a + 96, g[6], g[7]);
        }
        /* recentring: 32 x sum over groups of scale x sum(q) */
        const __m256i rc = _mm256_madd_epi16(_mm256_loadu_si256((const __m256i *)bsums), sc);
        acc = _mm256_sub_epi32(acc, _mm256_slli_epi32(rc, 5));
        __m128i t = _mm_add_epi32(_mm256_extracti128_si256(acc, 1), _mm256_castsi256_si128(acc));
        t = _mm_add_epi32(t, _mm_shuffle_epi32(t, 0x4E));
        t = _mm_add_epi32(t, _mm_shuffle_epi32(t, 0xB1));
        uint16_t dh;
        memcpy(&dh, w + 208, 2);
        float f = (float)_mm_cvtsi128_si32(t);
        f = f * _cvtsh_ss(dh);
        f = f * kscales[b];
        total = total + f;
    }
    return total;
}

struct q6_args {
    const uint8_t *w;
    const int8_t *qk;
    const int16_t *bsums;
    const float *kscales;
    int cols, size, ldy;
    float *y;
};

static void q6_rows(void *p, int start, int end) {
    const struct q6_args *a = p;
    const size_t stride = (size_t)a->cols / 256 * 210;
    for (int r = start; r < end; r++)
        for (int c = 0; c < a->size; c++)
            a->y[(size_t)c * a->ldy + r] =
                dot_q6_k_avx2(a->w + r * stride, a->qk + (size_t)c * a->cols, a->bsums + (size_t)c * a->cols / 16,
                              a->kscales + (size_t)c * a->cols / 256, a->cols);
}

/* MatVecQ6_K (nn/dot_q6_k.go:64-74) on at most `threads` threads.  QK, KScales
 * and BSums in golem's layout ([column][...]); y is [size][ldy]. */
int cpu_mat_vec_q6_k(const uint8_t *w, const int8_t *qk, const int16_t *bsums, const float *kscales, int rows,
                     int cols, int size, float *y, int ldy, int threads) {
    if (cols % 256 || !pool.count)
        return -1;
    struct q6_args a = {w, qk, bsums, kscales, cols, size, ldy, y};
    in_parallel(rows, (long)rows * cols * size, threads, q6_rows, &a);
    return 0;
}

/* ---- Q4_0 (nn/dot_q4_0_amd64.s) ---------------------------------------- */

enum { BEGIN = 1, FINISH = 2 }; /* nn/dot_q4_0.go:99-104 */

/* The 32 nibbles of a block, unsigned: weights 0..15 then 16..31. */
static inline __m256i q4_unpack(const uint8_t *blk) {
    const __m128i m4 = _mm_set1_epi8(0x0F);
    const __m128i x = _mm_loadu_si128((const __m128i *)(blk + 2));
    const __m128i lo = _mm_and_si128(x, m4);
    const __m128i hi = _mm_and_si128(_mm_srli_epi16(x, 4), m4);
    return _mm256_inserti128_si256(_mm256_castsi128_si256(lo), hi, 1);
}

static inline float q4_scale(const uint8_t *blk) {
    uint16_t h;
    memcpy(&h, blk, 2);
    return _cvtsh_ss(h);
}

/* The eight int32 sums of one block against one column. */
static inline __m256 q4_column(__m256i nib, const int8_t *q) {
    const __m256i pairs = _mm256_maddubs_epi16(nib, _mm256_loadu_si256((const __m256i *)q));
    return _mm256_cvtepi32_ps(_mm256_madd_epi16(pairs, _mm256_set1_epi16(1)));
}

/* Eight lanes and a correction to one product: ((l0+l4)+(l2+l6)) +
 * ((l1+l5)+(l3+l7)) - corr (REDUCE; nn/dot_q4_0.go:108-114). */
static inline float q4_reduce(__m256 acc, float corr) {
    __m128 lo = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    lo = _mm_add_ps(lo, _mm_movehl_ps(lo, lo));
    const float s = _mm_cvtss_f32(lo) + _mm_cvtss_f32(_mm_shuffle_ps(lo, lo, 0x01));
    return s - corr;
}

/* dotQ4_0AVX2: state = 8 lanes + 1 correction. */
static void dot_q4_0_x1(const uint8_t *w, const int8_t *q, const float *scales, const float *corr, int n,
                        int stride, float *state, int mode) {
    __m256 acc = (mode & BEGIN) ? _mm256_setzero_ps() : _mm256_loadu_ps(state);
    float c = (mode & BEGIN) ? 0.0f : state[8];
    for (int b = 0; b < n / 32; b++) {
        const __m256i nib = q4_unpack(w);
        const float d = q4_scale(w);
        const __m256 s = _mm256_set1_ps(d * scales[0]);
        acc = _mm256_fmadd_ps(s, q4_column(nib, q), acc);
        c = c + d * corr[0];
        w += 18;
        q += (size_t)stride * 32;
        scales += stride;
        corr += stride;
    }
    if (mode & FINISH) {
        state[0] = q4_reduce(acc, c);
    } else {
        _mm256_storeu_ps(state, acc);
        state[8] = c;
    }
}

/* dotQ4_0x4AVX2 / dotQ4_0x8AVX2: `cols` consecutive columns, state = cols x 8
 * lanes then cols corrections.  The row is unpacked once per block. */
static inline void dot_q4_0_xn(const uint8_t *w, const int8_t *q, const float *scales, const float *corr, int n,
                               int stride, float *state, int mode, const int cols) {
    __m256 acc[8];
    float c[8];
    for (int j = 0; j < cols; j++) {
        acc[j] = (mode & BEGIN) ? _mm256_setzero_ps() : _mm256_loadu_ps(state + 8 * j);
        c[j] = (mode & BEGIN) ? 0.0f : state[8 * cols + j];
    }
    for (int b = 0; b < n / 32; b++) {
        const __m256i nib = q4_unpack(w);
        const float d = q4_scale(w);
        float sd[8];
        for (int j = 0; j < cols; j++) {
            sd[j] = d * scales[j];
            c[j] = c[j] + d * corr[j];  /* a multiply and an add, as x1 */
        }
        for (int j = 0; j < cols; j++)
            acc[j] = _mm256_fmadd_ps(_mm256_set1_ps(sd[j]), q4_column(nib, q + 32 * j), acc[j]);
        w += 18;
        q += (size_t)stride * 32;
        scales += stride;
        corr += stride;
    }
    for (int j = 0; j < cols; j++) {
        if (mode & FINISH) {
            state[j] = q4_reduce(acc[j], c[j]);
        } else {
            _mm256_storeu_ps(state + 8 * j, acc[j]);
            state[8 * cols + j] = c[j];
        }
    }
}

/* One column group of matVecQ4_0Rows: the kernel for `cols` columns starting
 * at column c, over the inputs starting at `block`. */
static void q4_kernel(const uint8_t *w, const int8_t *Q, const float *S, const float *C, int stride, int block,
                      int c, int n, float *state, int mode, int cols) {
    const size_t at = (size_t)block * stride + c;
    if (cols == 8)
        dot_q4_0_xn(w, Q + at * 32, S + at, C + at, n, stride, state, mode, 8);
    else if (cols == 4)
        dot_q4_0_xn(w, Q + at * 32, S + at, C + at, n, stride, state, mode, 4);
    else
        dot_q4_0_x1(w, Q + at * 32, S + at, C + at, n, stride, state, mode);
}

struct q4_args {
    const uint8_t *w;
    const int8_t *Q;
    const float *S, *C;
    int stride, size, inputs, ldy;
    float *y;
};

enum { K_TILE = 2048, ROW_TILE_BYTES = 24 * 1024, MAX_ROW_TILE = 64 }; /* nn/dot_q4_0.go:147-152 */

/* matVecQ4_0Rows (nn/dot_q4_0.go:168-270): rows [start, end). */
static void q4_rows(void *p, int start, int end) {
    const struct q4_args *a = p;
    const size_t row_bytes = (size_t)a->inputs / 32 * 18;
    const int widths[3] = {8, 4, 1};
    if (a->inputs <= K_TILE) {
        float state[72];
        int c = 0;
        for (int wi = 0; wi < 3; wi++) {
            const int cols = widths[wi];
            for (; c + cols <= a->size; c += cols)
                for (int r = start; r < end; r++) {
                    q4_kernel(a->w + r * row_bytes, a->Q, a->S, a->C, a->stride, 0, c, a->inputs, state,
                              BEGIN | FINISH, cols);
                    for (int j = 0; j < cols; j++)
                        a->y[(size_t)(c + j) * a->ldy + r] = state[j];
                }
        }
        return;
    }
    const int step_bytes = K_TILE / 32 * 18;
    int rows = ROW_TILE_BYTES / step_bytes;
    rows = rows < 1 ? 1 : rows > MAX_ROW_TILE ? MAX_ROW_TILE : rows;
    static __thread float states[MAX_ROW_TILE][72];
    for (int from = start; from < end; from += rows) {
        const int to = from + rows < end ? from + rows : end;
        int c = 0;
        for (int wi = 0; wi < 3; wi++) {
            const int cols = widths[wi];
            for (; c + cols <= a->size; c += cols) {
                for (int k = 0; k < a->inputs; k += K_TILE) {
                    const int block = k / 32, n = a->inputs - k < K_TILE ? a->inputs - k : K_TILE;
                    const int mode = (k == 0 ? BEGIN : 0) | (k + n >= a->inputs ? FINISH : 0);
                    for (int r = from; r < to; r++)
                        q4_kernel(a->w + r * row_bytes + (size_t)block * 18, a->Q, a->S, a->C, a->stride, block, c,
                                  n, states[r - from], mode, cols);
                }
                for (int r = from; r < to; r++)
                    for (int j = 0; j < cols; j++)
                        a->y[(size_t)(c + j) * a->ldy + r] = states[r - from][j];
            }
        }
    }
}

/* MatVecQ4_0 (nn/dot_q4_0.go:117-124) on at most `threads` threads.  Q,
 * Scales and Corr in golem's interleaved layout with stride = size; y is
 * [size][ldy]. */
int cpu_mat_vec_q4_0(const uint8_t *w, const int8_t *Q, const float *S, const float *C, int rows, int inputs,
                     int size, float *y, int ldy, int threads) {
    if (inputs % 32 || !pool.count)
        return -1;
    struct q4_args a = {w, Q, S, C, size, size, inputs, ldy, y};
    in_parallel(rows, (long)rows * inputs * size, threads, q4_rows, &a);
    return 0;
}

/* ---- the packed product (nn/pack_q4_0.go, nn/pack_q4_0_amd64.s) ----------
 *
 * Eight rows interleaved per group of blocks (144 bytes a block: the rows'
 * eight fp16 scales, then four 32-byte chunks of eight inputs; byte s*8+j of
 * chunk g holds row {0,1,4,5}[s] in its low nibble and row {2,3,6,7}[s] in
 * its high one, at input 8g+j).  dotPackedQ4_0x4AVX2 (:99-160) multiplies a
 * group against four columns: per block the nibbles are split into eight
 * registers once; per column the eight activation bytes of a chunk are
 * broadcast to its four slots, VPMADDUBSW'd against the low and the high
 * nibbles, the int16 pairs summed over the four chunks, widened by VPMADDWD
 * against ones and folded by one VPHADDD into the eight rows in order; then
 * acc += float(sums) * (act_scale * row_scale) and acc -= corr * row_scale,
 * both fused.  dotPackedQ4_0AVX2 is the same for one column. */
static inline void packed_unpack(const uint8_t *blk, __m256i nib[8], __m256 *rs) {
    *rs = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)blk));
    const __m256i mask = _mm256_set1_epi8(0x0F);
    for (int g = 0; g < 4; g++) {
        const __m256i c = _mm256_loadu_si256((const __m256i *)(blk + 16 + 32 * g));
        nib[2 * g] = _mm256_and_si256(c, mask);
        nib[2 * g + 1] = _mm256_and_si256(_mm256_srli_epi16(c, 4), mask);
    }
}

static inline __m256 packed_sums(const __m256i nib[8], const int8_t *q) {
    __m256i lo = _mm256_setzero_si256(), hi = _mm256_setzero_si256();
    for (int g = 0; g < 4; g++) {
        const __m256i a = _mm256_set1_epi64x(*(const long long *)(q + 8 * g));
        const __m256i l = _mm256_maddubs_epi16(nib[2 * g], a), h = _mm256_maddubs_epi16(nib[2 * g + 1], a);
        lo = g == 0 ? l : _mm256_add_epi16(lo, l);
        hi = g == 0 ? h : _mm256_add_epi16(hi, h);
    }
    const __m256i ones = _mm256_set1_epi16(1);
    return _mm256_cvtepi32_ps(_mm256_hadd_epi32(_mm256_madd_epi16(lo, ones), _mm256_madd_epi16(hi, ones)));
}

/* One group of eight rows against `cols` (4 or 1) columns from column c,
 * over n inputs from `block`; state: cols x 8 running sums. */
static void packed_kernel(const uint8_t *w, const int8_t *Q, const float *S, const float *C, int stride, int block,
                          int c, int n, float *state, int mode, int cols) {
    __m256 acc[4];
    for (int j = 0; j < cols; j++)
        acc[j] = (mode & BEGIN) ? _mm256_setzero_ps() : _mm256_loadu_ps(state + 8 * j);
    for (int b = 0; b < n / 32; b++) {
        __m256i nib[8];
        __m256 rs;
        packed_unpack(w + (size_t)b * 144, nib, &rs);
        const size_t at = (size_t)(block + b) * stride + c;
        for (int j = 0; j < cols; j++) {
            const __m256 sums = packed_sums(nib, Q + (at + j) * 32);
            const __m256 sc = _mm256_mul_ps(_mm256_set1_ps(S[at + j]), rs);
            acc[j] = _mm256_fmadd_ps(sums, sc, acc[j]);
            acc[j] = _mm256_fnmadd_ps(_mm256_set1_ps(C[at + j]), rs, acc[j]);
        }
    }
    for (int j = 0; j < cols; j++)
        _mm256_storeu_ps(state + 8 * j, acc[j]);
}

struct packed_args {
    const uint8_t *w;
    const int8_t *Q;
    const float *S, *C;
    int size, inputs, ldy;
    float *y;
};

enum { MAX_GROUP_TILE = 8 }; /* nn/pack_q4_0.go:147-152 */

/* matVecPackedQ4_0Rows (nn/pack_q4_0.go:153-221): rows [start, end), a
 * group computed whole and written in part. */
static void packed_rows(void *p, int start, int end) {
    const struct packed_args *a = p;
    const size_t group_bytes = (size_t)a->inputs / 32 * 144;
    const int first = start / 8, last = (end + 7) / 8;
    const int steps = K_TILE < a->inputs ? K_TILE : a->inputs;
    const int step_bytes = steps / 32 * 144;
    int tile = ROW_TILE_BYTES / step_bytes;
    tile = tile < 1 ? 1 : tile > MAX_GROUP_TILE ? MAX_GROUP_TILE : tile;
    float four[MAX_GROUP_TILE][32], one[MAX_GROUP_TILE][8];
    for (int from = first; from < last; from += tile) {
        const int to = from + tile < last ? from + tile : last;
        int c = 0;
        for (int wi = 0; wi < 2; wi++) {
            const int cols = wi == 0 ? 4 : 1;
            for (; c + cols <= a->size; c += cols) {
                for (int k = 0; k < a->inputs; k += steps) {
                    const int block = k / 32, n = a->inputs - k < steps ? a->inputs - k : steps;
                    const int mode = (k == 0 ? BEGIN : 0) | (k + n >= a->inputs ? FINISH : 0);
                    for (int g = from; g < to; g++)
                        packed_kernel(a->w + (size_t)g * group_bytes + (size_t)block * 144, a->Q, a->S, a->C,
                                      a->size, block, c, n, cols == 4 ? four[g - from] : one[g - from], mode, cols);
                }
                for (int g = from; g < to; g++)
                    for (int j = 0; j < cols; j++)
                        for (int r = 0; r < 8; r++) {
                            const int row = 8 * g + r;
                            if (row >= start && row < end)
                                a->y[(size_t)(c + j) * a->ldy + row] =
                                    (cols == 4 ? four[g - from] : one[g - from])[8 * j + r];
                        }
            }
        }
    }
}

/* The packed product of golem's loader (whole groups of eight rows) over a
 * batch in golem's interleaved layout, on at most `threads` threads. */
int cpu_mat_vec_packed_q4_0(const uint8_t *packed, const int8_t *Q, const float *S, const float *C, int rows,
                            int inputs, int size, float *y, int ldy, int threads) {
    if (inputs % 32 || rows % 8 || !pool.count)
        return -1;
    struct packed_args a = {packed, Q, S, C, size, inputs, ldy, y};
    in_parallel(rows, (long)rows * inputs * size, threads, packed_rows, &a);
    return 0;
}

/* The single kernels, for the tests: one row against columns [c, c+cols). */
void cpu_dot_q4_0(const uint8_t *w, const int8_t *Q, const float *S, const float *C, int stride, int block, int c,
                  int n, float *state, int mode, int cols) {
    q4_kernel(w, Q, S, C, stride, block, c, n, state, mode, cols);
}

float cpu_dot_q6_k(const uint8_t *w, const int8_t *q, const int16_t *bsums, const float *kscales, int n) {
    return dot_q6_k_avx2(w, q, bsums, kscales, n);
}
