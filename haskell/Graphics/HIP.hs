{-# LANGUAGE ForeignFunctionInterface #-}
{-# LANGUAGE EmptyDataDecls #-}

{-|
Module: Graphics.HIP
Description: FFI binding of libgemma_hip (include/gemma_hip.h)

The replacement for the Graphics.WebGPU.Dawn.* modules (the webgpu-dawn
dependency, gemma.cabal:60) under gemma.hs's decode loop.  Every import
below is one C function of include/gemma_hip.h with its exact C types;
tests/test_haskell_ffi.py parses this file and checks each one (name, arity,
argument and result types) against the header.

Handles are ForeignPtrs whose finalisers are the void-typed gh_*_release
functions.  GHC runs finalisers in any order; the library keeps a context
or model alive until the last handle made from it is released, so no order
is unsafe.

Calls that run GPU work block until it is done and are imported "safe", so
the -threaded RTS (gemma.cabal:102) keeps other Haskell threads running;
the library serialises calls on one context with a mutex.
-}
module Graphics.HIP
  ( -- * Handles
    CtxS, ModelS, KvS, Q4S
  , Context, Model, Cache, Q4Tensor
  , GhConfig(..)
    -- * Errors
  , HipError(..), check
    -- * Handles with finalisers
  , newContext, newModel, loadGGUF, newCache, uploadQ4
    -- * Raw imports
  , c_lastError, c_version, c_deviceCount
  , c_ctxCreate, c_ctxDestroy, p_ctxRelease, c_ctxSync
  , c_configPreset, c_modelCreate, c_modelDestroy, p_modelRelease
  , c_modelSetTensor, c_modelCheck, c_modelConfig, c_modelPlan, c_modelLoadGGUF, c_ggufInspect
  , c_kvCreate, c_kvDestroy, p_kvRelease, c_kvReset, c_kvLength, c_kvTruncate, c_kvSetSampling, c_kvSetTopK
  , c_step, c_generate, c_prefill, c_generatePrefill
  , c_q4Upload, c_q4Free, p_q4Release, c_q4Matvec, c_q4Dequant, c_linearQ4
    -- * Constants
  , dtypeF32, dtypeF16, dtypeQ4_0
  , modeGemma3, modeRef
  , flagQKNorm, flagPostAttnNorm, flagPostFFNNorm, flagZeroCentered, flagIEEEScales
  ) where

import Control.Exception (Exception, throwIO)
import Data.Int (Int32, Int64)
import Data.Word (Word8, Word32, Word64)
import Foreign.C.String (CString, peekCString, withCString)
import Foreign.C.Types (CFloat(..), CInt(..), CSize(..))
import Foreign.ForeignPtr (FinalizerPtr, ForeignPtr, newForeignPtr, withForeignPtr)
import Foreign.Marshal.Alloc (alloca)
import Foreign.Ptr (Ptr, castPtr)
import Foreign.Storable (Storable(..))

-- | Opaque C structs (gh_ctx, gh_model, gh_kv, gh_q4).
data CtxS
data ModelS
data KvS
data Q4S

type Context = ForeignPtr CtxS
type Model = ForeignPtr ModelS
type Cache = ForeignPtr KvS
type Q4Tensor = ForeignPtr Q4S

-- | gh_config: seven int32 shape fields, max_seq, sliding_window,
-- global_every, three floats (rope_theta_local, rope_theta_global, rms_eps),
-- mode and flags -- 15 fields of 4 bytes, in this order.
data GhConfig = GhConfig
  { ghVocab, ghHidden, ghLayers, ghHeads, ghKVHeads, ghHeadDim, ghFFN :: !Int32
  , ghMaxSeq, ghSlidingWindow, ghGlobalEvery :: !Int32
  , ghThetaLocal, ghThetaGlobal, ghRmsEps :: !Float
  , ghMode, ghFlags :: !Int32
  } deriving (Show, Eq)

instance Storable GhConfig where
  sizeOf _ = 15 * 4
  alignment _ = 4
  peek p = do
    let i k = peekByteOff p (4 * k) :: IO Int32
        f k = peekByteOff p (4 * k) :: IO Float
    GhConfig <$> i 0 <*> i 1 <*> i 2 <*> i 3 <*> i 4 <*> i 5 <*> i 6
             <*> i 7 <*> i 8 <*> i 9
             <*> f 10 <*> f 11 <*> f 12
             <*> i 13 <*> i 14
  poke p c = do
    let ints = [ghVocab, ghHidden, ghLayers, ghHeads, ghKVHeads, ghHeadDim, ghFFN, ghMaxSeq, ghSlidingWindow, ghGlobalEvery]
    mapM_ (\(k, g) -> pokeByteOff p (4 * k) (g c)) (zip [0 ..] ints)
    pokeByteOff p 40 (ghThetaLocal c)
    pokeByteOff p 44 (ghThetaGlobal c)
    pokeByteOff p 48 (ghRmsEps c)
    pokeByteOff p 52 (ghMode c)
    pokeByteOff p 56 (ghFlags c)

dtypeF32, dtypeF16, dtypeQ4_0 :: CInt
dtypeF32 = 0
dtypeF16 = 1
dtypeQ4_0 = 2

modeGemma3, modeRef :: Int32
modeGemma3 = 0
modeRef = 1

flagQKNorm, flagPostAttnNorm, flagPostFFNNorm, flagZeroCentered, flagIEEEScales :: Int32
flagQKNorm = 1
flagPostAttnNorm = 2
flagPostFFNNorm = 4
flagZeroCentered = 8
flagIEEEScales = 16

-- ---------------------------------------------------------------- imports
foreign import ccall unsafe "gh_last_error" c_lastError :: IO CString
foreign import ccall unsafe "gh_version" c_version :: IO CString
foreign import ccall safe "gh_device_count" c_deviceCount :: Ptr CInt -> IO CInt

foreign import ccall safe "gh_ctx_create" c_ctxCreate :: CInt -> Ptr (Ptr CtxS) -> IO CInt
foreign import ccall safe "gh_ctx_destroy" c_ctxDestroy :: Ptr CtxS -> IO CInt
foreign import ccall safe "&gh_ctx_release" p_ctxRelease :: FinalizerPtr CtxS
foreign import ccall safe "gh_ctx_sync" c_ctxSync :: Ptr CtxS -> IO CInt

foreign import ccall unsafe "gh_config_preset" c_configPreset :: CString -> Ptr GhConfig -> IO CInt
foreign import ccall safe "gh_model_create" c_modelCreate :: Ptr CtxS -> Ptr GhConfig -> Ptr (Ptr ModelS) -> IO CInt
foreign import ccall safe "gh_model_destroy" c_modelDestroy :: Ptr ModelS -> IO CInt
foreign import ccall safe "&gh_model_release" p_modelRelease :: FinalizerPtr ModelS
foreign import ccall safe "gh_model_set_tensor"
  c_modelSetTensor :: Ptr ModelS -> CString -> CInt -> Ptr () -> CSize -> IO CInt
foreign import ccall safe "gh_model_check" c_modelCheck :: Ptr ModelS -> IO CInt
foreign import ccall safe "gh_model_config" c_modelConfig :: Ptr ModelS -> Ptr GhConfig -> IO CInt
foreign import ccall safe "gh_model_plan" c_modelPlan :: Ptr ModelS -> CString -> CSize -> Ptr CSize -> IO CInt
foreign import ccall safe "gh_model_load_gguf"
  c_modelLoadGGUF :: Ptr CtxS -> CString -> Int32 -> Ptr (Ptr ModelS) -> IO CInt
foreign import ccall safe "gh_gguf_inspect" c_ggufInspect :: CString -> Ptr GhConfig -> IO CInt

foreign import ccall safe "gh_kv_create" c_kvCreate :: Ptr ModelS -> Int32 -> Ptr (Ptr KvS) -> IO CInt
foreign import ccall safe "gh_kv_destroy" c_kvDestroy :: Ptr KvS -> IO CInt
foreign import ccall safe "&gh_kv_release" p_kvRelease :: FinalizerPtr KvS
foreign import ccall safe "gh_kv_reset" c_kvReset :: Ptr KvS -> IO CInt
foreign import ccall safe "gh_kv_length" c_kvLength :: Ptr KvS -> Ptr Int32 -> IO CInt
foreign import ccall safe "gh_kv_truncate" c_kvTruncate :: Ptr KvS -> Int32 -> IO CInt
foreign import ccall safe "gh_kv_set_sampling" c_kvSetSampling :: Ptr KvS -> CFloat -> Word64 -> IO CInt
foreign import ccall safe "gh_kv_set_top_k" c_kvSetTopK :: Ptr KvS -> Int32 -> IO CInt

foreign import ccall safe "gh_step"
  c_step :: Ptr ModelS -> Ptr KvS -> Int32 -> Ptr CFloat -> Ptr CFloat -> Ptr Int32 -> IO CInt
foreign import ccall safe "gh_generate"
  c_generate :: Ptr ModelS -> Ptr KvS -> Ptr Int32 -> Int32 -> Int32 -> Ptr Int32 -> IO CInt
foreign import ccall safe "gh_prefill"
  c_prefill :: Ptr ModelS -> Ptr KvS -> Ptr Int32 -> Int32 -> Ptr CFloat -> Ptr CFloat -> Ptr Int32 -> IO CInt
foreign import ccall safe "gh_generate_prefill"
  c_generatePrefill :: Ptr ModelS -> Ptr KvS -> Ptr Int32 -> Int32 -> Int32 -> Ptr Int32 -> IO CInt

foreign import ccall safe "gh_q4_0_upload"
  c_q4Upload :: Ptr CtxS -> Ptr Word8 -> Int64 -> Int64 -> CInt -> Ptr (Ptr Q4S) -> IO CInt
foreign import ccall safe "gh_q4_0_free" c_q4Free :: Ptr Q4S -> IO CInt
foreign import ccall safe "&gh_q4_0_release" p_q4Release :: FinalizerPtr Q4S
foreign import ccall safe "gh_q4_0_matvec" c_q4Matvec :: Ptr Q4S -> Ptr CFloat -> Ptr CFloat -> CInt -> CFloat -> IO CInt
foreign import ccall safe "gh_q4_0_dequant" c_q4Dequant :: Ptr Q4S -> Ptr CFloat -> IO CInt
foreign import ccall safe "gh_linear_q4"
  c_linearQ4 :: Ptr CtxS -> Ptr Word32 -> CSize -> Ptr CFloat -> CInt -> CInt -> CInt -> CFloat -> Ptr CFloat -> IO CInt

-- ---------------------------------------------------------------- errors
-- | A negative GH_ERR_* code and gh_last_error's message.  The reference
-- fails with 'error' where these codes arise (for example
-- src/Gemma/KVCache.hs:109-116); the rewired modules throw this instead.
data HipError = HipError !Int !String deriving Show
instance Exception HipError

check :: IO CInt -> IO ()
check act = do
  rc <- act
  if rc == 0
    then pure ()
    else do
      msg <- c_lastError >>= peekCString
      throwIO (HipError (fromIntegral rc) msg)

-- | Run a creating call that writes a handle to its out pointer and wrap
-- the handle with its finaliser.
created :: FinalizerPtr a -> (Ptr (Ptr a) -> IO CInt) -> IO (ForeignPtr a)
created fin mk = alloca $ \out -> do
  check (mk out)
  peek out >>= newForeignPtr fin

newContext :: Int -> IO Context
newContext dev = created p_ctxRelease (c_ctxCreate (fromIntegral dev))

newModel :: Context -> GhConfig -> IO Model
newModel ctx cfg = withForeignPtr ctx $ \c -> alloca $ \pc -> do
  poke pc cfg
  created p_modelRelease (c_modelCreate c pc)

loadGGUF :: Context -> FilePath -> Int -> IO Model
loadGGUF ctx path maxSeq = withForeignPtr ctx $ \c -> withCString path $ \p ->
  created p_modelRelease (c_modelLoadGGUF c p (fromIntegral maxSeq))

newCache :: Model -> Int -> IO Cache
newCache m maxSeq = withForeignPtr m $ \mp -> created p_kvRelease (c_kvCreate mp (fromIntegral maxSeq))

uploadQ4 :: Context -> Ptr Word8 -> Int -> Int -> IO Q4Tensor
uploadQ4 ctx raw rows cols = withForeignPtr ctx $ \c ->
  created p_q4Release (c_q4Upload c (castPtr raw) (fromIntegral rows) (fromIntegral cols) 0)
