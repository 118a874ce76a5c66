{-|
Module: Gemma.Layers.LinearQ4
Description: Q4_0 matrix-vector product on MI355X through libgemma_hip

The exports and signatures of the reference's Gemma.Layers.LinearQ4
(src/Gemma/Layers/LinearQ4.hs:17-74).  The body is gh_linear_q4: the raw
GGUF Q4_0 bytes (as little-endian Word32s, 18-byte blocks along each row)
are repacked and multiplied on the device, with the optional soft cap
sigma * tanh(y / sigma) on the result.  As in the reference, each call makes
its own GPU context.
-}
module Gemma.Layers.LinearQ4
  ( runLinearQ4
  , runLinearQ4WithContext
  , runLinearQ4GPU
  ) where

import Control.Monad.IO.Class (liftIO)
import Control.Monad.Trans.Cont (ContT)
import qualified Data.Vector.Storable as V
import qualified Data.Vector.Storable.Mutable as VM
import Data.Vector.Storable (Vector)
import Data.Word (Word32)
import Foreign.ForeignPtr (withForeignPtr)
import Foreign.Ptr (castPtr)

import qualified Graphics.HIP as HIP
import Graphics.HIP (check)

runLinearQ4 :: Vector Word32  -- Q4_0 weights (raw GGUF bytes)
            -> Vector Float   -- input [nCols]
            -> Int            -- nRows
            -> Int            -- nCols (multiple of 32)
            -> Bool           -- applySoftCap
            -> Float          -- softCapSigma
            -> ContT r IO (Vector Float)
runLinearQ4 w x nRows nCols softCap sigma = liftIO $ do
  ctx <- HIP.newContext 0
  y <- VM.new nRows
  withForeignPtr ctx $ \c -> V.unsafeWith w $ \wp -> V.unsafeWith x $ \xp -> VM.unsafeWith y $ \yp ->
    check (HIP.c_linearQ4 c wp (fromIntegral (V.length w)) (castPtr xp) (fromIntegral nRows)
                          (fromIntegral nCols) (if softCap then 1 else 0) (realToFrac sigma) (castPtr yp))
  V.unsafeFreeze y

runLinearQ4WithContext :: ctx -> Vector Word32 -> Vector Float -> Int -> Int -> Bool -> Float
                       -> ContT r IO (Vector Float)
runLinearQ4WithContext _ = runLinearQ4

runLinearQ4GPU :: Vector Word32 -> Vector Float -> Int -> Int -> Bool -> Float -> ContT r IO (Vector Float)
runLinearQ4GPU = runLinearQ4
