/* amdc_internal.h -- declarations shared by the C sources of libamdc_q4.so
 * (not exported: hidden visibility). */
#ifndef AMDC_INTERNAL_H
#define AMDC_INTERNAL_H
#include <stdarg.h>

#define AMDC_HIDDEN __attribute__((visibility("hidden")))

/* Set the message of amdc_last_error() and return code. */
AMDC_HIDDEN int amdc_fail_v(int code, const char *fmt, va_list ap);

#endif
