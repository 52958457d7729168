/*
 * wm_io.h -- C ABI of libwm_hip's device-direct byte streams: the payload
 * half of whitematter's WMT tensor files (reference core/serialize.cpp:
 * 36-108, and the float buffers of save_model / save_optimizer /
 * save_checkpoint) moved between a byte source or sink and device memory
 * without a host-side copy of the whole buffer.
 *
 * The caller supplies the file side as a callback (an ifstream, a file
 * descriptor, a socket); the library owns two pinned staging buffers of
 * WM_IO_CHUNK bytes and alternates between them, so that reading chunk i+1
 * overlaps the host-to-device copy of chunk i (and the device-to-host copy
 * of chunk i+1 overlaps writing chunk i).  Copies run on the library stream,
 * ordered after the kernels that produce a buffer and before the ones that
 * read it; a read returns once every chunk has been handed to the stream.
 * Conventions are those of wm_hip.h.  Calls are serialised by the library.
 */
#ifndef WM_IO_H
#define WM_IO_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WM_IO_CHUNK (8 << 20)

/* Deliver up to `bytes` bytes into buf; return how many were delivered
 * (fewer only at the end of the data or on an error). */
typedef int64_t (*wm_read_fn)(void* ctx, void* buf, int64_t bytes);
/* Accept `bytes` bytes from buf; return how many were accepted. */
typedef int64_t (*wm_write_fn)(void* ctx, const void* buf, int64_t bytes);

/* dst[0 .. bytes) = the next `bytes` bytes of `read`.  WM_ERR_IO when the
 * source ends early (the bytes that arrived are on the device).  Replaces
 * load_tensor's read into a host vector (core/serialize.cpp:90-93) and the
 * buffer reads of load_optimizer / load_checkpoint (:296, :336, :347,
 * :474, :496, :501). */
int wm_read_into_device(wm_read_fn read, void* ctx, void* dst, int64_t bytes);

/* Stream src[0 .. bytes) to `write`.  WM_ERR_IO when the sink refuses
 * bytes.  Replaces save_tensor's write of the host vector (:53) and the
 * buffer writes of save_optimizer / save_checkpoint (:200, :213, :219,
 * :371, :385, :389). */
int wm_write_from_device(wm_write_fn write, void* ctx, const void* src, int64_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* WM_IO_H */
