// qt_noalloc.hip — the batched int8 projection (qwen_hip_op_matmat_int8's kernels) for
// callers that cannot allocate device memory: code under HIP graph capture, serving
// loops that forbid hipMalloc.  The inputs and outputs are the caller's device buffers;
// the one scratch buffer the kernels need (the exact int8 activation pieces and their
// per-stream scales, qt_batch.hip) is a file-scope device array, so no call allocates.
//
// The array's name is only a host-side stand-in: its device address is taken once per
// device with hipGetSymbolAddress (with that device current) and kept in a per-device
// table; kernels are given that address, never the name.  The device is the one the
// `stream` argument belongs to (the current device for the null stream).  Every call on a
// GPU shares that GPU's array, so calls that overlap on one GPU (two streams, two threads)
// race: callers serialise them on one stream per GPU.  The pieces kernel writes every
// byte the GEMM reads (padding streams included), so nothing needs clearing between calls.
#include <hip/hip_runtime.h>
#include <pthread.h>

#include "qt_launch.h"

#define QT_NA_MAX_COLS 8192
#define QT_NA_MAX_B 64
// pieces [cols/64][3*Bp][64] int8 + scales f32[Bp], Bp <= 64
#define QT_NA_PIECE_BYTES ((size_t)QT_NA_MAX_COLS * 3 * QT_NA_MAX_B)
#define QT_NA_BYTES (QT_NA_PIECE_BYTES + 256)
#define QT_NA_MAX_DEV 64

static __device__ __align__(256) unsigned char scratch[QT_NA_BYTES];

static pthread_mutex_t g_na_lock = PTHREAD_MUTEX_INITIALIZER;
static void *g_na_ptr[QT_NA_MAX_DEV];

// the stream's device's copy of the array (looked up once per device), NULL on error
static void *na_scratch(hipStream_t st) {
    int dev = -1;
    if (st ? hipStreamGetDevice(st, &dev) != hipSuccess : hipGetDevice(&dev) != hipSuccess) {
        qt_seterr("matmat_int8_noalloc: cannot tell the stream's device");
        return NULL;
    }
    if (dev < 0 || dev >= QT_NA_MAX_DEV) {
        qt_seterr("matmat_int8_noalloc: device index %d out of range (0..%d)", dev, QT_NA_MAX_DEV - 1);
        return NULL;
    }
    pthread_mutex_lock(&g_na_lock);
    void *p = g_na_ptr[dev];
    if (!p) {
        // the symbol's address is per device: look it up with the stream's device current
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e == hipSuccess && cur != dev) e = hipSetDevice(dev);
        if (e == hipSuccess) e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur >= 0 && cur != dev) {
            const hipError_t e2 = hipSetDevice(cur);
            if (e == hipSuccess) e = e2;
        }
        if (e != hipSuccess || !p) {
            qt_seterr("matmat_int8_noalloc: hipGetSymbolAddress of the scratch array on device %d failed: %s", dev,
                      hipGetErrorString(e));
            p = NULL;
        } else {
            g_na_ptr[dev] = p;
        }
    }
    pthread_mutex_unlock(&g_na_lock);
    return p;
}

extern "C" int qwen_hip_op_matmat_int8_noalloc(float *Y, const int8_t *W, const float *scale, const float *X, int rows,
                                               int cols, int B, void *stream) {
    if (!Y || !W || !scale || !X) {
        qt_seterr("matmat_int8_noalloc: null pointer argument");
        return -1;
    }
    if (rows <= 0 || cols <= 0 || cols % 64 != 0 || cols > QT_NA_MAX_COLS) {
        qt_seterr("matmat_int8_noalloc: bad shape %dx%d (cols must be a multiple of 64 and <= %d: the scratch "
                  "array holds %zu bytes)", rows, cols, QT_NA_MAX_COLS, (size_t)QT_NA_BYTES);
        return -1;
    }
    if (B < 1 || B > QT_NA_MAX_B) {
        qt_seterr("matmat_int8_noalloc: B %d out of range (1..%d)", B, QT_NA_MAX_B);
        return -1;
    }
    hipStream_t st = (hipStream_t)stream;
    unsigned char *base = (unsigned char *)na_scratch(st);
    if (!base) return -1;
    const int Bp = (B + 15) & ~15;
    int8_t *P = (int8_t *)base;
    float *S = (float *)(base + QT_NA_PIECE_BYTES);
    hipError_t e = qt_launch_bpieces(X, cols, NULL, 0.f, cols, B, Bp, P, S, st);
    if (e == hipSuccess)
        e = qt_launch_bgemm_i8(QT_EPI_STORE, (const uint8_t *)W, scale, rows, cols, P, S, B, Bp, Y, rows, st);
    if (e != hipSuccess) {
        qt_seterr("matmat_int8_noalloc: launch failed: %s", hipGetErrorString(e));
        return -1;
    }
    return 0;
}
