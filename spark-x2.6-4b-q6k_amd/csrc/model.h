/* model.h — what the model loader needs from the forward's model object. */
#pragma once

namespace sparkmv {

/* The model frees dev_ptr (hipFree) when it is destroyed: the weights a
 * loader uploaded for it. Returns 0, or -1 with the message set. */
int model_adopt(void * model, void * dev_ptr);

}  // namespace sparkmv
