/*
 * scunet_image.h - PNG in, PNG out for the command-line denoiser (libscunet_hip.so).
 *
 * Replaces the reference crate's src/image.rs:17-69 (`image::read`, `image::write`),
 * which its CLI (src/main.rs:160-201) uses around `backend::run`. The I/O contract is
 * the reference's: 8-bit samples, value / 255 as float32 NCHW in [0, 1], no other
 * normalisation; RGB and RGBA read as 3 channels (alpha dropped), grayscale and
 * grayscale+alpha as 1; output is written as 8-bit RGB (c = 3) or grayscale (c = 1)
 * after clamping to [0, 1] and rounding half up.
 *
 * Status: 0 = OK, non-zero = failure with the message in scunet_image_error(), which
 * names the file and what is wrong with it. Thread-safe (the message is per thread).
 */
#ifndef SCUNET_IMAGE_H
#define SCUNET_IMAGE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* image.rs:17-43: decode an 8-bit PNG (any filter, Adam7 or not) into a newly allocated
 * float32 [c][h][w] array (*data; release it with scunet_image_free). Palette images
 * fail with "unsupported colour type Indexed" as in image.rs:31; samples of another
 * depth than 8 fail with a message saying so. */
int scunet_image_read(const char* path, float** data, size_t* c, size_t* h, size_t* w);
void scunet_image_free(float* data);

/* image.rs:45-69: write [c][h][w] float32 as an 8-bit PNG, each value clamped to [0, 1]
 * and stored as (unsigned char)(v * 255 + 0.5), NaN as 0. c must be 1 or 3. */
int scunet_image_write(const char* path, const float* data, size_t c, size_t h, size_t w);

/* Message of the last failed scunet_image_* call on this thread ("" if none). */
const char* scunet_image_error(void);

#ifdef __cplusplus
}
#endif

#endif
